"""hk_sample_static, the sampler for callers that cannot allocate device memory (its scratch is a static device array
of the library), against hk_sample, which allocates its own: the same token for the same logits and random number,
on two calls in a row on one GPU, the second over fewer logits (the array keeps the first call's contents); and its
limit (HK_SAMPLE_STATIC_MOST logits) refused with HE_E_ARG."""
import ctypes

import numpy as np
import pytest

from gpu_lib import check, sample, upload
from paths import package

pytestmark = pytest.mark.gpu

MOST = 262144  # HK_SAMPLE_STATIC_MOST


def sample_static(logits, temperature, topp, random):
    x = upload(np.ascontiguousarray(logits, dtype=np.float32))
    token = ctypes.c_int32(0)
    check(package().library().hk_sample_static(x.ptr, x.shape[0], float(temperature), float(topp), float(random),
                                               ctypes.byref(token), None))
    del x
    return int(token.value)


@pytest.mark.parametrize("temperature, topp", [(0.8, 0.9), (1.0, 1.0), (0.5, 0.6), (1.3, 0.95)])
def test_two_calls_in_a_row_equal_hk_sample(temperature, topp):
    rng = np.random.default_rng(int(100 * temperature + 10 * topp))
    big = (rng.standard_normal(152064) * 3).astype(np.float32)
    small = (rng.standard_normal(32000) * 2).astype(np.float32)
    for logits in (big, small):
        for u in (0.0, 0.37, 0.999):
            assert sample_static(logits, temperature, topp, u) == sample(logits, temperature, topp, u)


def test_largest_size_and_special_logits():
    rng = np.random.default_rng(7)
    full = (rng.standard_normal(MOST) * 4).astype(np.float32)
    assert sample_static(full, 0.9, 0.9, 0.5) == sample(full, 0.9, 0.9, 0.5)
    peaked = np.full(1000, -5.0, dtype=np.float32)
    peaked[123] = 30.0
    assert sample_static(peaked, 1.0, 0.9, 0.7) == 123
    bad = np.zeros(64, dtype=np.float32)
    bad[5] = np.nan
    assert sample_static(bad, 1.0, 0.9, 0.5) == sample(bad, 1.0, 0.9, 0.5) == -1


def test_refuses_more_logits_than_its_array_holds():
    # a device buffer of as many logits as the call names: were the size check ever to come after the launch, the
    # sampler would read valid memory and the test fail on its return code, never fault
    pk = package()
    x = upload(np.zeros(MOST + 1, dtype=np.float32))
    token = ctypes.c_int32(0)
    rc = pk.library().hk_sample_static(x.ptr, MOST + 1, 1.0, 0.9, 0.5, ctypes.byref(token), None)
    assert rc == pk.hip_engine.HE_E_ARG
    assert b"262144" in pk.library().he_last_error()


def test_refuses_a_stream_under_graph_capture():
    # the token is copied to the host and the stream waited for, which a capture cannot record: refused before any
    # launch, and the capture ends cleanly
    from gpu_lib import hip, hip_check
    pk = package()
    h = hip()
    stream, graph = ctypes.c_void_p(), ctypes.c_void_p()
    hip_check(h.hipStreamCreate(ctypes.byref(stream)))
    x = upload(np.zeros(64, dtype=np.float32))
    token = ctypes.c_int32(7)
    hip_check(h.hipStreamBeginCapture(stream, 2))  # hipStreamCaptureModeRelaxed
    rc = pk.library().hk_sample_static(x.ptr, 64, 1.0, 0.9, 0.5, ctypes.byref(token), stream)
    hip_check(h.hipStreamEndCapture(stream, ctypes.byref(graph)))
    if graph:
        hip_check(h.hipGraphDestroy(graph))
    hip_check(h.hipStreamDestroy(stream))
    assert rc == pk.hip_engine.HE_E_ARG
    assert b"capture" in pk.library().he_last_error()
    assert token.value == 7
