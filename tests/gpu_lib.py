"""The kernel-level C ABI (hk_*) driven from NumPy through device buffers from the HIP runtime (hipMalloc/hipMemcpy
over ctypes: plumbing for the tests, on the default stream)."""
import ctypes

import numpy as np

from paths import package

_hip = None


def hip():
    global _hip
    if _hip is None:
        lib = ctypes.CDLL("libamdhip64.so")
        lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        lib.hipFree.argtypes = [ctypes.c_void_p]
        lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        lib.hipDeviceSynchronize.argtypes = []
        lib.hipGetErrorString.restype = ctypes.c_char_p
        _hip = lib
    return _hip


def hip_check(code):
    if code != 0:
        raise RuntimeError("HIP: " + hip().hipGetErrorString(code).decode())


class Dev:
    """a device buffer with a NumPy dtype and shape"""

    def __init__(self, shape, dtype, init=None):
        self.shape, self.dtype = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape, np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = ctypes.c_void_p()
        hip_check(hip().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)))
        if init is not None:
            a = np.ascontiguousarray(init, dtype=self.dtype)
            assert a.nbytes == self.nbytes
            hip_check(hip().hipMemcpy(self.ptr, ctypes.c_void_p(a.ctypes.data), self.nbytes, 1))  # host to device
        else:
            zeros = np.zeros(self.shape, dtype=self.dtype)
            hip_check(hip().hipMemcpy(self.ptr, ctypes.c_void_p(zeros.ctypes.data), self.nbytes, 1))

    def numpy(self):
        hip_check(hip().hipDeviceSynchronize())
        out = np.zeros(self.shape, dtype=self.dtype)
        hip_check(hip().hipMemcpy(ctypes.c_void_p(out.ctypes.data), self.ptr, self.nbytes, 2))  # device to host
        return out

    def __del__(self):
        if self.ptr:
            hip().hipDeviceSynchronize()  # never free what a queued kernel may still read
            hip().hipFree(self.ptr)
            self.ptr = None


def upload(a):
    a = np.ascontiguousarray(a)
    return Dev(a.shape, a.dtype, a)


def check(code):
    return package().hip_engine.check(code)


def quantize_x(x, bias):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, np.shape(x)[-1])
    m, n = x.shape
    xd = upload(x)
    q, s = Dev((m, n), np.int8), Dev((m, n // 32), np.float32)
    check(package().library().hk_quantize_x(q.ptr, s.ptr, xd.ptr, m, n, bias, None))
    out = q.numpy(), s.numpy()
    del xd
    return out


def matmul(xq, xs, w, ws, rows, k, bias, six):
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    m = xq.shape[0]
    y = Dev((m, rows), np.float32)
    args = [upload(xq), upload(np.ascontiguousarray(xs, dtype=np.float32).reshape(m, k // 32)), upload(w),
            upload(np.ascontiguousarray(ws, dtype=np.float32))]
    check(package().library().hk_matmul(y.ptr, *(a.ptr for a in args), m, rows, k, bias, six, None))
    out = y.numpy()  # synchronizes before the inputs are freed
    del args
    return out


def group_sums(xq, w, rows, k, bias, six, gemm=0):
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    m = xq.shape[0]
    per = (k // 32) * (1 if bias else 4)
    s = Dev((m, rows, per), np.int32)
    xd, wd = upload(xq), upload(w)  # kept alive until the kernel has run
    check(package().library().hk_group_sums(s.ptr, xd.ptr, wd.ptr, m, rows, k, bias, six, gemm, None))
    out = s.numpy()
    del xd, wd
    return out


def penalize(logits, tokens, penalty):
    """hk_penalize on a device copy of the float32 logits"""
    x = upload(np.ascontiguousarray(logits, dtype=np.float32))
    t = np.ascontiguousarray(np.asarray(list(tokens), dtype=np.int32))
    check(package().library().hk_penalize(x.ptr, x.shape[0], ctypes.c_void_p(t.ctypes.data), t.size, float(penalty),
                                          None))
    return x.numpy()


def ordered_sum(p, nucleus):
    """hk_ordered_sum: the float64 total of p in index order and the running sum before every 256 values (nucleus: as
    the draw with a nucleus takes them, in one block; else as the draw without one)"""
    x = upload(np.ascontiguousarray(p, dtype=np.float32))
    total = ctypes.c_double(0.0)
    cps = np.zeros((x.shape[0] + 255) // 256, dtype=np.float64)
    check(package().library().hk_ordered_sum(x.ptr, x.shape[0], int(nucleus), ctypes.byref(total),
                                             ctypes.c_void_p(cps.ctypes.data), None))
    del x
    return total.value, cps


def sample(logits, temperature, topp, random):
    """hk_sample: the token drawn for one random number (-1 not finite, -2 a nucleus larger than the device sorts)"""
    x = upload(np.ascontiguousarray(logits, dtype=np.float32))
    token = ctypes.c_int32(0)
    check(package().library().hk_sample(x.ptr, x.shape[0], float(temperature), float(topp), float(random),
                                        ctypes.byref(token), None))
    del x
    return int(token.value)
