"""Where the repository's parts are, and the package loaded under an importable name."""
import importlib.util
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE_DIR = os.path.join(REPO, "pyodide-llm_amd")
ORACLE_DIR = os.path.join(REPO, "oracle")
GOLDEN_DIR = os.path.join(REPO, "tests", "golden")


def package():
    """pyodide-llm_amd/ as the module pyodide_llm_amd"""
    if "pyodide_llm_amd" in sys.modules:
        return sys.modules["pyodide_llm_amd"]
    spec = importlib.util.spec_from_file_location("pyodide_llm_amd", os.path.join(PACKAGE_DIR, "__init__.py"),
                                                  submodule_search_locations=[PACKAGE_DIR])
    module = importlib.util.module_from_spec(spec)
    sys.modules["pyodide_llm_amd"] = module
    spec.loader.exec_module(module)
    return module
