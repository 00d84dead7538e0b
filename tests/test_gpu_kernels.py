"""The HIP kernels through the C ABI against the oracle, to the bit: quantize_x, the exact int32 group sums and the
float32 outputs of the decode GEMV and the prefill GEMM (matmul_q8r / q8 / q6r / q6), at the reference's
known-answer sizes and at the standalone matmul's full sizes (K=4096, N in {4096, 14336}, M in {1, 4, 16, 512})."""
import ctypes

import numpy as np
import pytest

import gpu_lib as gl
from paths import package
import oracle_lib as ol

pytestmark = pytest.mark.gpu


def weights(rows, k, six, seed=3):
    x = ol.synth(rows * k, seed=seed, stream=2, sigma=0.02).reshape(rows, k)
    if six:
        q, s = ol.quantize6(x)
        return ol.pack6(q).reshape(rows, k // 32 * 24), s.reshape(rows, k // 32)
    q, s = ol.quantize(x)
    return q, s.reshape(rows, k // 32)


def activations(m, k, bias, seed=1):
    x = ol.synth(m * k, seed=seed, stream=9, sigma=1.0).reshape(m, k)
    return ol.quantize_x(x, bias)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("bias", [64, 0])
@pytest.mark.parametrize("n", [32, 288, 4096, 14336])
def test_quantize_x(bias, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((5, n)) * rng.uniform(0.01, 30, (5, 1))).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 32:64] = 1e-40 if n > 32 else 0.0
    q, s = gl.quantize_x(x, bias)
    q0, s0 = ol.quantize_x(x, bias)
    assert np.array_equal(q, q0) and same_bits(s, s0)


CASES = [(k, rows, m) for k in (32, 96, 288, 1056, 4096) for rows, m in ((37, 1), (64, 3), (130, 8))]


@pytest.mark.parametrize("six", [0, 1])
@pytest.mark.parametrize("bias", [64, 0])
@pytest.mark.parametrize("k,rows,m", CASES)
def test_gemv_bits(k, rows, m, bias, six):
    w, ws = weights(rows, k, six)
    xq, xs = activations(m, k, bias)
    want = ol.matmul(xq, xs, w, ws, rows, k, bias, six)
    got = gl.matmul(xq, xs, w, ws, rows, k, bias, six)
    assert same_bits(got, want)
    sums = gl.group_sums(xq, w, rows, k, bias, six)
    assert np.array_equal(sums, ol.group_sums(xq, w, rows, k, bias, six))


@pytest.mark.parametrize("k", [64, 192, 640, 3584, 18944])
@pytest.mark.parametrize("rows", [37, 130])
def test_int6_decode_bits(k, rows):
    """one token against int6 rows of an even number of groups: the int6 decode path (two groups a lane), tails of
    0 and 2 groups, the Qwen2.5-7B widths"""
    w, ws = weights(rows, k, 1)
    xq, xs = activations(1, k, 64)
    assert same_bits(gl.matmul(xq, xs, w, ws, rows, k, 64, 1), ol.matmul(xq, xs, w, ws, rows, k, 64, 1))


@pytest.mark.parametrize("k", [5120, 11008, 14336, 16384, 20480])
@pytest.mark.parametrize("rows", [37, 130])
def test_int8_decode_bits(k, rows):
    """one token against int8 rows longer than 4 KiB: the decode path's 8, 14, 16 and 20-step waves, with and
    without tail groups"""
    w, ws = weights(rows, k, 0)
    xq, xs = activations(1, k, 64)
    assert same_bits(gl.matmul(xq, xs, w, ws, rows, k, 64, 0), ol.matmul(xq, xs, w, ws, rows, k, 64, 0))


GEMM_CASES = [(k, rows, m) for k in (32, 96, 288, 1056, 4096)
              for rows, m in ((37, 9), (64, 96), (37, 128), (64, 130), (130, 200))]


@pytest.mark.parametrize("six", [0, 1])
@pytest.mark.parametrize("k,rows,m", GEMM_CASES)
def test_gemm_bits(k, rows, m, six):
    """more than 8 tokens: the MFMA GEMM, every output to the bit and every int32 group sum exact, ragged rows and
    tokens, K with and without tail groups (G % 4 != 0)"""
    w, ws = weights(rows, k, six)
    xq, xs = activations(m, k, 64)
    want = ol.matmul(xq, xs, w, ws, rows, k, 64, six)
    got = gl.matmul(xq, xs, w, ws, rows, k, 64, six)
    assert same_bits(got, want)
    sums = gl.group_sums(xq, w, rows, k, 64, six, gemm=1)
    assert np.array_equal(sums, ol.group_sums(xq, w, rows, k, 64, six))


@pytest.mark.parametrize("six", [0, 1])
def test_plain_order_with_many_tokens(six):
    """bias 0 (matmul_q8's lanes) with more than 8 tokens stays on the GEMV, in passes of 8"""
    k, rows, m = 288, 40, 20
    w, ws = weights(rows, k, six)
    xq, xs = activations(m, k, 0)
    assert same_bits(gl.matmul(xq, xs, w, ws, rows, k, 0, six), ol.matmul(xq, xs, w, ws, rows, k, 0, six))


@pytest.mark.parametrize("n", [4096, 14336])
@pytest.mark.parametrize("m", [1, 4, 16, 512])
def test_standalone_matmul_full_size(n, m):
    """K=4096, N in {4096, 14336}, M in {1, 4, 16, 512}: weights N(0, 0.02) by the reference's quantize(), activations
    N(0, 1) by quantize_x(bias 64); every output to the bit and every group sum exact"""
    k = 4096
    w, ws = weights(n, k, 0, seed=11)
    xq, xs = activations(m, k, 64, seed=12)
    want = ol.matmul(xq, xs, w, ws, n, k, 64, 0)
    got = gl.matmul(xq, xs, w, ws, n, k, 64, 0)
    assert same_bits(got, want)
    if m <= 16:
        assert np.array_equal(gl.group_sums(xq, w, n, k, 64, 0), ol.group_sums(xq, w, n, k, 64, 0))
    if m > 8 and n == 4096:
        assert np.array_equal(gl.group_sums(xq, w, n, k, 64, 0, gemm=1), ol.group_sums(xq, w, n, k, 64, 0))


@pytest.mark.parametrize("reps", [1, 3])
def test_extremes_of_int8_equal_float64(reps):
    """tests/forward-check.mjs:244-276 on the device: rows of -128 and 127 against activations 127 and 1, scales
    powers of two: the float32 result is the exact float64 sum (4 tokens on the GEMV, 12 on the GEMM)"""
    rows, groups = 8, 5
    n = groups * 32
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, size=(rows, n)).astype(np.int8)
    w[0], w[1] = -128, 127
    w[2, ::2], w[2, 1::2] = -128, 127
    xq = np.stack([np.full(n, 127), np.ones(n), np.where(np.arange(n) & 1, 1, 127), rng.integers(1, 128, n)]).astype(np.int8)
    xs = np.stack([np.full(groups, 2.0 ** -(2 + t)) for t in range(4)]).astype(np.float32)
    xq, xs = np.tile(xq, (reps, 1)), np.tile(xs, (reps, 1))
    ws = np.full((rows, groups), 2.0 ** -7, dtype=np.float32)
    got = gl.matmul(xq, xs, w, ws, rows, n, 64, 0)
    want = (w.astype(np.float64)[None] * (xq.astype(np.float64)[:, None] - 64)).sum(-1) * 2.0 ** -7 * xs[:, :1].astype(np.float64)
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("nbytes, passes", [(64, 1), (4096, 3), (1 << 20, 2), ((1 << 20) + 192, 5)])
def test_read_ceiling_checksum(nbytes, passes):
    """hk_read_ceiling returns kernels/ceilings.ts:9-25 read()'s checksum: the xor of the four lanes j of passes times
    the sum (mod 2^32) of the 32-bit words at p + 16k + 4j"""
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = gl.upload(words)
    lanes = [int(words[j::4].astype(np.uint64).sum() * passes) & 0xFFFFFFFF for j in range(4)]
    want = lanes[0] ^ lanes[1] ^ lanes[2] ^ lanes[3]
    got, ms = ctypes.c_int32(0), ctypes.c_double(0.0)
    gl.check(package().library().hk_read_ceiling(buf.ptr, nbytes, passes, ctypes.byref(got), ctypes.byref(ms), None))
    assert (got.value & 0xFFFFFFFF) == want
    assert ms.value > 0


def test_read_floor_times_cold_windows():
    """hk_read_floor times one launch of the read kernel over each next window of the span: a positive time a launch
    that grows with the bytes read, and arguments it cannot use refused"""
    span = 64 << 20
    buf = gl.upload(np.ones(span // 4, dtype=np.uint32))
    lib = package().library()
    small, large = ctypes.c_double(0.0), ctypes.c_double(0.0)
    gl.check(lib.hk_read_floor(buf.ptr, span, 1 << 20, 8, ctypes.byref(small), None))
    gl.check(lib.hk_read_floor(buf.ptr, span, 32 << 20, 4, ctypes.byref(large), None))
    assert 0 < small.value < large.value
    for nbytes, spanned in ((100, span), (1 << 20, 1 << 19)):
        assert lib.hk_read_floor(buf.ptr, spanned, nbytes, 1, ctypes.byref(small), None) != 0


def fma_lane(passes, w, x0, step):
    """kernels/ceilings.ts fma() for one lane in float32, each step rounded (the benchmark page's fmaSum before its
    four-lane sum)"""
    f = np.float32
    ws = [f(w), f(w) + f(0.0009765625), f(w) + f(0.001953125), f(w) + f(0.0029296875)]
    x, d = f(x0), f(step)
    y = x + f(0.25)
    a = [f(i) for i in range(8)]
    for _ in range(passes):
        for k in range(4):
            a[k] = a[k] + ws[k] * x
            a[4 + k] = a[4 + k] + ws[k] * y
        x, y = x - d, y - d
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))


@pytest.mark.parametrize("passes, w, x0, step", [(1, 1.0, 0.9999, 1e-7), (1000, 1.0, 0.9999, 1e-7),
                                                 (333, 0.37, -1.5, 0.003)])
def test_valu_ceiling_sum(passes, w, x0, step):
    """hk_valu_ceiling computes ceilings.ts fma()'s float32 sums (no FMA, no reordering) in every lane"""
    result, ms, pairs = ctypes.c_float(0), ctypes.c_double(0), ctypes.c_double(0)
    gl.check(package().library().hk_valu_ceiling(passes, w, x0, step, ctypes.byref(result), ctypes.byref(ms),
                                                 ctypes.byref(pairs), None))
    want = fma_lane(passes, w, x0, step)
    assert np.float32(result.value).view(np.uint32) == want.view(np.uint32)
    assert ms.value > 0 and pairs.value == 8192 * 64 * passes * 8


def int8(v):
    return ((v + 128) % 256) - 128


@pytest.mark.parametrize("passes, first, times, flip", [(1, 3, 5, 0x81), (2, 3, 5, 0x81), (255, -128, 127, 0xFF),
                                                        (1000, 3, 5, 0x81)])
def test_mfma_ceiling_checksum(passes, first, times, flip):
    """hk_mfma_ceiling's v_mfma_i32_32x32x32_i8 sums: every element of a 32 x 32 product gains 32 * a * b a pass (A's
    bytes first, then first ^ flip, alternately; B's times), on accumulators that start at 1000 n + e"""
    checksum, ms, ops = ctypes.c_int32(0), ctypes.c_double(0), ctypes.c_double(0)
    gl.check(package().library().hk_mfma_ceiling(passes, first, times, flip, ctypes.byref(checksum), ctypes.byref(ms),
                                                 ctypes.byref(ops), None))
    a0, a1 = int8(first & 255), int8((first ^ flip) & 255)
    sum_a = ((passes + 1) // 2) * a0 + (passes // 2) * a1
    start = 64 * (16 * (0 + 1000 + 2000 + 3000) + 4 * sum(range(16)))
    want = (start + 4 * 1024 * 32 * int8(times & 255) * sum_a) & 0xFFFFFFFF
    assert (checksum.value & 0xFFFFFFFF) == want
    assert ms.value > 0 and ops.value == 4096 * passes * 4 * 32768 * 2
