"""The oracle's kernels against the reference's known-answer tests: the seeded LCG cases and closed forms of
tests/forward-check.mjs:119-276, the invariant quantize_x(bias 0) == quantize() (tests/smoke.mjs:285-289), the
far-leading softmax cases of tests/attention-check.mjs, and float64 mathematics where a formula fixes the answer."""
import math

import numpy as np
import pytest

import oracle_lib as ol
from lcg import Lcg

f32 = np.float32


def r32(x):
    return f32(x)


# ------------------------------------------------------------------------------------------------ quantize_x

def test_quantize_x_bias0_is_quantize():
    """tests/smoke.mjs:285-289: quantize_x with bias 0 writes the bytes llama2_convert.quantize() writes"""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((7, 256)) * rng.uniform(0.01, 10, size=(7, 1))).astype(np.float32)
    x[0, :32] = 0.0
    q, s = ol.quantize_x(x, 0)
    q2, s2 = ol.quantize(x)
    assert np.array_equal(q.reshape(-1), q2.reshape(-1))
    assert np.array_equal(s.reshape(-1).view(np.uint32), s2.view(np.uint32))


def test_quantize_x_bias64_range_and_step():
    """bias 64 (kernels/kernel.ts:129-156): q in 1..127 (qmax 63), and (q - 64) * scale within half a step of x"""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    q, s = ol.quantize_x(x, 64)
    assert q.min() >= 1 and q.max() <= 127
    back = (q.astype(np.float64) - 64) * np.repeat(s.astype(np.float64), 32, axis=-1)
    assert np.all(np.abs(back - x) <= 0.5 * np.repeat(s, 32, axis=-1) * (1 + 1e-5))


def test_quantize_x_tiny_scale_edge():
    """kernels/kernel.ts:214-220: a group whose scale is below 2.9e-39 has 1/scale overflow to infinity; the
    saturating conversions then give -128/127 (bias 0) and -128 (bias 64, the wrapped add)"""
    x = np.zeros(32, dtype=np.float32)
    x[0], x[1] = 1e-40, -1e-40
    q0, s0 = ol.quantize_x(x, 0)
    assert s0[0] > 0 and np.isinf(f32(1) / s0[0])
    assert q0[0] == 127 and q0[1] == -128 and q0[2] == 0
    q1, _ = ol.quantize_x(x, 64)
    assert q1[0] == -128 and q1[1] == -128 and q1[2] == 64


# ------------------------------------------------------------------------------------------------ matmuls (T165-T167)

def six_value(raw, i, j, groups):
    """tests/forward-check.mjs:139-143: the int8 of int6 weight j of row i"""
    at = (i * groups + (j >> 5)) * 24
    m = j & 31
    low = raw[at + m] & 15 if m < 16 else raw[at + m - 16] >> 4
    top = (raw[at + 16 + (m % 8)] >> (2 * (m // 8))) & 3
    v = ((int(low) | (int(top) << 4)) << 2) & 255
    return v - 256 if v >= 128 else v


class Kat:
    """the inputs of tests/forward-check.mjs:119-136 (seed 7): rows 24, 41 groups"""

    def __init__(self):
        rng = Lcg(7)
        self.rows, self.n = 24, 32 * 41
        ng = self.n // 32
        self.pool = np.array([(rng.next() & 255) - 128 for _ in range(self.rows * self.n)], dtype=np.int64)
        x = [(rng.next() % 255) - 127 for _ in range(self.n)]
        for j in range(32):
            x[j], x[32 + j] = 127, -127
        self.x = np.array(x, dtype=np.int64)
        self.ws = np.array([r32(1e-3 * (1 + rng.next() % 1000)) for _ in range(self.rows * ng)], dtype=np.float32)
        self.xs = np.array([r32(1e-2 * (1 + rng.next() % 1000)) for _ in range(ng)], dtype=np.float32)
        self.raw6 = np.array([rng.next() & 255 for _ in range(self.rows * ng * 24)], dtype=np.uint8)
        self.rng = rng


KAT = Kat()
GROUPS = [1, 2, 3, 4, 5, 6, 7, 8, 11, 41]


def kat_weights(groups):
    m = groups * 32
    w = np.zeros((KAT.rows, m), dtype=np.int8)
    for i in range(KAT.rows):
        w[i] = KAT.pool[i * KAT.n:i * KAT.n + m]
    w[0, :32] = 127
    w[1, (32 if groups > 1 else 0):(32 if groups > 1 else 0) + 32] = -128
    return w


@pytest.mark.parametrize("groups", GROUPS)
def test_matmul_q8_lane_closed_form(groups):
    """tests/forward-check.mjs:144-159: lane k of a group sums products 2k, 2k+1, 2k+8, 2k+9 of each half; every lane
    scaled by f32(ws * xs) into its own float32 accumulator, the four added in order"""
    m = groups * 32
    w = kat_weights(groups)
    xq = KAT.x[:m].astype(np.int8)
    ws = KAT.ws[:KAT.rows * groups].reshape(KAT.rows, groups)
    xs = KAT.xs[:groups]
    got = ol.matmul(xq, xs, w, ws, KAT.rows, m, 0, 0)[0]
    for i in range(KAT.rows):
        lanes = [f32(0)] * 4
        for g in range(groups):
            s = f32(ws[i, g] * xs[g])
            for lane in range(4):
                total = 0
                for j in (2 * lane, 2 * lane + 1, 2 * lane + 8, 2 * lane + 9, 2 * lane + 16, 2 * lane + 17,
                          2 * lane + 24, 2 * lane + 25):
                    total += int(w[i, g * 32 + j]) * int(xq[g * 32 + j])
                lanes[lane] = f32(lanes[lane] + f32(f32(total) * s))
        want = f32(f32(f32(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])
        assert got[i].view(np.uint32) == want.view(np.uint32), (i, groups)


@pytest.mark.parametrize("groups", GROUPS)
def test_matmul_q6_is_q8_on_the_widened_values(groups):
    """tests/forward-check.mjs:160-172 (matmul_q6 against the lane closed form on six()'s values) and :183-190
    (matmul_q6r == matmul_q8r on the widened int8)"""
    m = groups * 32
    raw = KAT.raw6[:KAT.rows * groups * 24]
    wide = np.array([[six_value(raw, i, j, groups) for j in range(m)] for i in range(KAT.rows)], dtype=np.int8)
    ws = KAT.ws[:KAT.rows * groups].reshape(KAT.rows, groups)
    xs = KAT.xs[:groups]
    xq0 = KAT.x[:m].astype(np.int8)
    assert np.array_equal(ol.matmul(xq0, xs, raw, ws, KAT.rows, m, 0, 1), ol.matmul(xq0, xs, wide, ws, KAT.rows, m, 0, 0))
    xq64 = (np.arange(m) * 37 % 128).astype(np.int8)
    a = ol.matmul(xq64, xs, raw, ws, KAT.rows, m, 64, 1)
    b = ol.matmul(xq64, xs, wide, ws, KAT.rows, m, 64, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("groups", GROUPS)
def test_matmul_q8r_closed_form(groups):
    """tests/forward-check.mjs:191-210: each group's exact dot(w, q - 64) times f32(ws * xs) rounded once, into lane
    g % 4 for the groups in fours, the lanes added in order, then the groups past the fours one at a time"""
    m = groups * 32
    rng = Lcg(1000 + groups)
    w = np.array([[(rng.next() & 255) - 128 for _ in range(m)] for _ in range(KAT.rows)], dtype=np.int8)
    xq = np.array([rng.next() % 128 for _ in range(m)], dtype=np.int8)
    ws = KAT.ws[:KAT.rows * groups].reshape(KAT.rows, groups)
    xs = KAT.xs[:groups]
    got = ol.matmul(xq, xs, w, ws, KAT.rows, m, 64, 0)[0]
    fours = groups & ~3
    for i in range(KAT.rows):
        def part(g):
            dot = int(np.dot(w[i, g * 32:(g + 1) * 32].astype(np.int64), xq[g * 32:(g + 1) * 32].astype(np.int64) - 64))
            return f32(f32(dot) * f32(ws[i, g] * xs[g]))
        lanes = [f32(0)] * 4
        for g in range(fours):
            lanes[g & 3] = f32(lanes[g & 3] + part(g))
        total = f32(f32(f32(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])
        for g in range(fours, groups):
            total = f32(total + part(g))
        assert got[i].view(np.uint32) == total.view(np.uint32), (i, groups)


def test_matmul_q8r_at_the_ends_of_int8_equals_float64():
    """tests/forward-check.mjs:244-276: rows of -128 and 127 against activations of 127 and 1 with power-of-two scales:
    every group sum times the scales and their total are exact, so the float32 result is the float64 sum"""
    rows, groups = 8, 5
    n = groups * 32
    rng = Lcg(11)
    patterns = [lambda j: -128, lambda j: 127, lambda j: 127 if j & 1 else -128, lambda j: -128 if (j & 31) < 16 else 127]
    w = np.array([[patterns[i](j) if i < 4 else (rng.next() & 255) - 128 for j in range(n)] for i in range(rows)],
                 dtype=np.int8)
    acts = [lambda j: 127, lambda j: 1, lambda j: 1 if j & 1 else 127, None]
    ws = np.full((rows, groups), 2.0 ** -7, dtype=np.float32)
    for t in range(4):
        xq = np.array([acts[t](j) if acts[t] else 1 + rng.next() % 127 for j in range(n)], dtype=np.int8)
        xs = np.full(groups, 2.0 ** -(2 + t), dtype=np.float32)
        got = ol.matmul(xq, xs, w, ws, rows, n, 64, 0)[0]
        for i in range(rows):
            want = sum(int(w[i, j]) * (int(xq[j]) - 64) for j in range(n)) * 2.0 ** -7 * 2.0 ** -(2 + t)
            assert float(got[i]) == want


def test_group_sums_are_the_exact_integers():
    """the int32 sums the matmuls scale: dot(w, q - 64) a group (bias 64) and the four lanes (bias 0)"""
    rng = np.random.default_rng(5)
    w = rng.integers(-128, 128, size=(6, 128), dtype=np.int8)
    q = rng.integers(1, 128, size=128, dtype=np.int8)
    s = ol.group_sums(q, w, 6, 128, 64, 0)[0]
    want = (w.astype(np.int64).reshape(6, 4, 32) * (q.astype(np.int64).reshape(4, 32) - 64)).sum(-1)
    assert np.array_equal(s, want)
    q0 = rng.integers(-127, 128, size=128, dtype=np.int8)
    s0 = ol.group_sums(q0, w, 6, 128, 0, 0)[0].reshape(6, 4, 4)
    assert np.array_equal(s0.sum(-1), (w.astype(np.int64).reshape(6, 4, 32) * q0.astype(np.int64).reshape(4, 32)).sum(-1))


# ------------------------------------------------------------------------------------------------ elementwise

def test_fexp_vexp_within_two_ulp_of_exp():
    """the Cephes expf (kernels/kernel.ts:15-45) over [-87, 88]: within 2 ulp of the correctly rounded exp, exact at
    0; vexp equals fexp except below -87, where fexp is 0 and vexp exp(-87)'s neighbourhood"""
    xs = np.linspace(-87, 88, 20001).astype(np.float32)
    v = ol.vexp(xs)
    for x, got in zip(xs[::7], v[::7]):
        want = f32(math.exp(float(x)))
        assert abs(int(got.view(np.int32)) - int(want.view(np.int32))) <= 2, x
        assert ol.fexp(float(x)) == float(got)
    assert ol.fexp(0.0) == 1.0
    assert ol.fexp(-90.0) == 0.0 and ol.vexp([-90.0])[0] > 0
    assert ol.vexp([100.0])[0] == ol.vexp([88.0])[0]


def test_f16_conversions_match_numpy():
    """to_f16 (kernels/kernel.ts:570-599) is NumPy's astype(float16) (round to nearest even, subnormals, overflow to
    inf); from_f16 (:383-392) widens every finite half exactly"""
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
                        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 70000.0, 6e-8, 3e-8, 2.9e-8, 1e-12, -5.96e-8],
                                 dtype=np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ol.to_f16(x), want)
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(halves.view(np.float16))
    assert np.array_equal(ol.from_f16(halves)[finite].view(np.uint32),
                          halves.view(np.float16)[finite].astype(np.float32).view(np.uint32))


def test_rmsnorm_against_float64():
    rng = np.random.default_rng(2)
    for n in (288, 4096, 61):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        got = ol.rmsnorm(x, w, 1e-5).astype(np.float64)
        want = w.astype(np.float64) * x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("nh, hs, rot", [(4, 16, 0), (3, 32, 32), (2, 32, 12), (5, 64, 16)])
def test_rope_is_the_float64_rotation_of_interleaved_pairs(nh, hs, rot):
    """kernels/kernel.ts:344-357: each head's pairs (v[2i], v[2i+1]), i < rot / 2 (rot 0 or hs: all of them), turned by
    the angle whose cosine and sine the tables give at i; the values past rot untouched. Against the float64 rotation
    of the same float32 inputs: a rotation the other way, swapped pair members, a table read at i instead of i / 2 or
    a head offset by a pair all miss it by far more than float32's rounding"""
    rng = np.random.default_rng(hs + rot)
    v = (rng.standard_normal(nh * hs) * 2).astype(np.float32)
    angles = rng.uniform(-math.pi, math.pi, hs // 2)
    fcr, fci = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    out = v.copy()
    ol.load().or_rope(ol.ptr(out), ol.ptr(fcr), ol.ptr(fci), nh, hs, rot)
    turned = rot if 0 < rot < hs else hs
    heads, got = v.reshape(nh, hs).astype(np.float64), out.reshape(nh, hs)
    v0, v1 = heads[:, 0:turned:2], heads[:, 1:turned:2]
    c, s_ = fcr[:turned // 2].astype(np.float64), fci[:turned // 2].astype(np.float64)
    want0, want1 = v0 * c - v1 * s_, v0 * s_ + v1 * c
    # each output is a difference or sum of two rounded products: within 2 ulps of the larger product, at most
    bound = 2.0 ** -22 * (np.abs(v0 * c) + np.abs(v1 * s_)) + 1e-30
    assert (np.abs(got[:, 0:turned:2] - want0) <= bound).all()
    assert (np.abs(got[:, 1:turned:2] - want1) <= bound).all()
    assert np.array_equal(got[:, turned:], v.reshape(nh, hs)[:, turned:])
    # a rotation keeps each pair's length
    assert np.allclose(np.hypot(got[:, 0:turned:2], got[:, 1:turned:2]), np.hypot(v0, v1), rtol=1e-6)


def test_rope_by_the_tables_turns_position_p_by_p_times_the_pair_frequency():
    """or_rope_tables (public/llama2_numpy.py:484-542 for theta, no scaling): turning a pair by position a's angle then
    by position b's is turning it by position a + b's (float64, to float32's rounding), and position 0 is the
    identity"""
    hs, theta, seq = 64, 10000.0, 64
    cos, sin = ol.rope_tables(seq, hs, theta)
    assert np.array_equal(cos[0], np.ones(hs // 2, np.float32)) and np.array_equal(sin[0], np.zeros(hs // 2, np.float32))
    rng = np.random.default_rng(9)
    v = rng.standard_normal(hs).astype(np.float32)
    for a, b in ((3, 5), (10, 31), (1, 1)):
        once = v.copy()
        ol.load().or_rope(ol.ptr(once), ol.ptr(cos[a]), ol.ptr(sin[a]), 1, hs, 0)
        ol.load().or_rope(ol.ptr(once), ol.ptr(cos[b]), ol.ptr(sin[b]), 1, hs, 0)
        both = v.copy()
        ol.load().or_rope(ol.ptr(both), ol.ptr(cos[a + b]), ol.ptr(sin[a + b]), 1, hs, 0)
        assert np.allclose(once, both, rtol=0, atol=2e-6 * np.abs(v).max())
        freq = 1.0 / theta ** (np.arange(0, hs, 2) / hs)
        assert np.allclose(cos[a], np.cos(a * freq), atol=1e-7) and np.allclose(sin[a], np.sin(a * freq), atol=1e-7)


def attention64(q, kc, vc, pos, nh, nkv, hs):
    out = np.zeros(nh * hs)
    for h in range(nh):
        kh = h // (nh // nkv)
        qh = q[h * hs:(h + 1) * hs].astype(np.float64)
        k = kc.reshape(-1, nkv * hs)[:pos + 1, kh * hs:(kh + 1) * hs].astype(np.float64)
        v = vc.reshape(-1, nkv * hs)[:pos + 1, kh * hs:(kh + 1) * hs].astype(np.float64)
        s = k @ qh / math.sqrt(hs)
        p = np.exp(s - s.max())
        out[h * hs:(h + 1) * hs] = (p / p.sum()) @ v
    return out


@pytest.mark.parametrize("half", [0, 1])
def test_attention_against_float64(half):
    """kernels/kernel.ts:448-566: GQA softmax(q k / sqrt(hs)) v over positions 0..pos, float32 or float16 cache"""
    rng = np.random.default_rng(4)
    nh, nkv, hs = 8, 2, 16
    for pos in (0, 1, 2, 3, 4, 5, 17, 63):
        q = rng.standard_normal(nh * hs).astype(np.float32)
        kc = rng.standard_normal((pos + 1) * nkv * hs).astype(np.float32)
        vc = rng.standard_normal((pos + 1) * nkv * hs).astype(np.float32)
        if half:
            k16, v16 = ol.to_f16(kc), ol.to_f16(vc)
            got = ol.attention(q, k16, v16, pos, nh, nkv, hs, half=True)
            kc, vc = ol.from_f16(k16), ol.from_f16(v16)
        else:
            got = ol.attention(q, kc, vc, pos, nh, nkv, hs)
        assert np.allclose(got, attention64(q, kc, vc, pos, nh, nkv, hs), rtol=1e-5, atol=1e-5)


def test_attention_far_leading_scores():
    """tests/attention-check.mjs: two positions far above the rest (3 apart), at pairs 1, 4 and 32 apart, for 2..72
    positions, one head far above zero and one far below it: the output is the two values' mix within 1e-3"""
    nh, hs, lead = 2, 8, 3.0
    kv_dim = nh * hs
    rng = Lcg(12345)
    rand = lambda: rng.next() / 2 ** 24  # noqa: E731
    u = np.array([rand() * 2 - 1 for _ in range(hs)])
    uu = float((u * u).sum())
    q = np.tile(u, nh).astype(np.float32)
    levels = [((-2.0, 2.0), 110.0), ((-260.0, -250.0), -100.0)]
    worst = 0.0
    for count in range(2, 73, 3):
        for apart in (1, 4, 32):
            for a in range(0, count - apart, max(1, (count - apart) // 4)):
                b = a + apart
                kc = np.zeros((count, kv_dim), dtype=np.float32)
                vc = np.zeros((count, kv_dim), dtype=np.float32)
                for h in range(nh):
                    (low, high), top = levels[h]
                    for t in range(count):
                        score = top if t == a else top - lead if t == b else low + (high - low) * rand()
                        kc[t, h * hs:(h + 1) * hs] = (score * math.sqrt(hs) / uu) * u
                        vc[t, h * hs:(h + 1) * hs] = 1.0 if t == a else -1.0 if t == b else [rand() * 2 - 1 for _ in range(hs)]
                for half in (0, 1):
                    if half:
                        k16, v16 = ol.to_f16(kc), ol.to_f16(vc)
                        got = ol.attention(q, k16, v16, count - 1, nh, nh, hs, half=True)
                        kr, vr = ol.from_f16(k16), ol.from_f16(v16)
                    else:
                        got = ol.attention(q, kc, vc, count - 1, nh, nh, hs)
                        kr, vr = kc.reshape(-1), vc.reshape(-1)
                    want = attention64(q, kr, vr, count - 1, nh, nh, hs)
                    off = float(np.abs(got - want).max())
                    worst = max(worst, off)
                    assert off <= 1e-3, (count, a, b, half)
    assert worst <= 1e-3


def test_swiglu_and_argmax():
    rng = np.random.default_rng(8)
    h1 = (rng.standard_normal(1000) * 30).astype(np.float32)
    h3 = rng.standard_normal(1000).astype(np.float32)
    got = np.zeros_like(h1)
    ol.load().or_swiglu(ol.ptr(got), ol.ptr(h1), ol.ptr(h3), 1000)
    want = h1.astype(np.float64) / (1 + np.exp(-h1.astype(np.float64))) * h3
    assert np.allclose(got, want, rtol=1e-5, atol=1e-30)
    x = np.array([1.0, 3.0, 2.0, 3.0], dtype=np.float32)
    assert ol.load().or_argmax(ol.ptr(x), 4) == 1  # the first of the largest (kernels/kernel.ts:695-699)
