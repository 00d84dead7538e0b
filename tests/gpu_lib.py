"""The kernel-level C ABI (hk_*) driven from NumPy through device buffers that torch allocates (torch is plumbing
here: memory and the default stream)."""
import ctypes

import numpy as np

from paths import package


def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU")
    return torch


def dev(a):
    torch = torch_cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    torch = torch_cuda()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def check(code):
    return package().hip_engine.check(code)


def quantize_x(x, bias):
    torch = torch_cuda()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, np.shape(x)[-1])
    m, n = x.shape
    xd = dev(x)
    q = torch.zeros((m, n), dtype=torch.int8, device="cuda")
    s = torch.zeros((m, n // 32), dtype=torch.float32, device="cuda")
    check(package().library().hk_quantize_x(vp(q), vp(s), vp(xd), m, n, bias, None))
    return host(q), host(s)


def matmul(xq, xs, w, ws, rows, k, bias, six):
    torch = torch_cuda()
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    m = xq.shape[0]
    y = torch.zeros((m, rows), dtype=torch.float32, device="cuda")
    args = [dev(xq), dev(np.ascontiguousarray(xs, dtype=np.float32).reshape(m, k // 32)), dev(np.ascontiguousarray(w)),
            dev(np.ascontiguousarray(ws, dtype=np.float32))]
    check(package().library().hk_matmul(vp(y), *(vp(a) for a in args), m, rows, k, bias, six, None))
    return host(y)


def group_sums(xq, w, rows, k, bias, six, gemm=0):
    torch = torch_cuda()
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, k)
    m = xq.shape[0]
    per = (k // 32) * (1 if bias else 4)
    s = torch.zeros((m, rows, per), dtype=torch.int32, device="cuda")
    check(package().library().hk_group_sums(vp(s), vp(dev(xq)), vp(dev(np.ascontiguousarray(w))), m, rows, k, bias,
                                            six, gemm, None))
    return host(s)
