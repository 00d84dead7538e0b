"""pyodide-llm's quantized forward path on MI355X: HIP kernels for gfx950 behind the interface public/forward.js gives
its Python caller. The directory's name is not a Python identifier: load it through importlib under the name
pyodide_llm_amd (importlib.util.spec_from_file_location with submodule_search_locations=[this directory])."""
from .hip_engine import (KINDS, HeConfig, HeTensor, HipError, TensorArray, TENSORS, T, Engine, External, config,
                         external, group_size, library, open_config, open_synthetic, places, plan_to_config,
                         rope_tables, start)

__all__ = ["KINDS", "group_size", "places", "rope_tables", "HeConfig", "HeTensor", "HipError", "TensorArray", "TENSORS", "T", "Engine", "External", "config",
           "external", "library", "open_config", "open_synthetic", "plan_to_config", "start"]
