"""The sampler kernels (hk_penalize, hk_sample) against the oracle's or_penalize / or_sample (kernels/kernel.ts:705-868)
to the token and the bit, over vocabularies up to the 8B's, temperatures, top-p values with and without a nucleus,
ties, -inf and non-finite logits; and generateMany's sampled steps against the oracle's steps."""
import numpy as np
import pytest

import gpu_lib as gl
import oracle_lib as ol

pytestmark = pytest.mark.gpu

SORT_MOST = 8192


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def nucleus_size(logits, temperature, topp):
    """how many tokens the nucleus sort takes (float64 NumPy: away from SORT_MOST that decides)"""
    best = float(logits.max())
    floor = best - temperature * 16.118095 if 0 < topp < 1 else -np.inf
    p = np.exp((logits[logits >= floor].astype(np.float64) - best) / temperature)
    cutoff = min((1 - topp) / max(p.size - 1, 1) * p.sum(), p.max())
    return int((p >= cutoff).sum())


def test_penalize_matches_the_oracle():
    rng = np.random.default_rng(0)
    logits = (rng.standard_normal(1000) * 3).astype(np.float32)
    logits[:4] = [0.0, -0.0, 5.0, -5.0]
    tokens = list(rng.integers(0, 1000, size=60)) + [0, 1, 2, 3]
    for penalty in (1.3, 0.7, 2.0):
        assert np.array_equal(bits(gl.penalize(logits, tokens, penalty)), bits(ol.penalize(logits, tokens, penalty)))


@pytest.mark.parametrize("n, scale", [(200, 3.0), (320, 1.0), (32000, 6.0), (128256, 8.0), (262144, 4.0)])
@pytest.mark.parametrize("temperature, topp", [(0.7, 0.9), (1.0, 1.0), (0.3, 0.5), (1.3, 0.95), (0.8, 0.0)])
def test_sample_matches_the_oracle(n, scale, temperature, topp):
    rng = np.random.default_rng(n + int(10 * temperature) + int(100 * topp))
    for trial in range(3):
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        if trial == 1:
            logits[rng.integers(0, n, size=n // 7)] = -np.inf
        if trial == 2:
            logits[rng.integers(0, n, size=5)] = logits.max()  # ties at the top
        large = 0 < topp < 1 and nucleus_size(logits, temperature, topp) > SORT_MOST
        for u in [0.0, 0.5, 0.999999] + list(rng.random(5)):
            got = gl.sample(logits, temperature, topp, u)
            if large:
                assert got == -2
            else:
                assert got == ol.sample(logits, temperature, topp, u), (trial, u)


def in_order(p):
    """the float64 running sums of p in index order, each add rounded (NumPy's cumsum adds one after another)"""
    return np.cumsum(np.asarray(p, np.float32).astype(np.float64))


def probabilities(kind, n, rng):
    """float32 values of the draw's kind (in [0, 1]) with many rounding cases of the float64 sum: exact ties (powers of
    two, short mantissas), values far below the running sum's last bit, a tiny first value, leading zeros"""
    u = rng.random(n)
    if kind == "spread":
        x = np.exp(-u * 10)
    elif kind == "tails":
        x = np.exp(-u * 80)
    elif kind == "powers":
        x = np.where(rng.random(n) < 0.25, 0.0, np.ldexp(1.0, -rng.integers(0, 40, n)))
    elif kind == "short":
        x = np.ldexp(rng.integers(0, 16, n).astype(np.float64), -rng.integers(0, 30, n))
    elif kind == "tiny_first":
        x = np.exp(-u * 5)
        x[0] = 1e-40
    elif kind == "leading_zeros":
        x = np.where(np.arange(n) < min(5000, n // 2), 0.0, np.exp(-u * 3))
    else:
        x = np.ldexp(1.0 + rng.integers(0, 1 << 23, n) / float(1 << 23), -rng.integers(0, 60, n))
    return x.astype(np.float32)


@pytest.mark.parametrize("nucleus", [1, 0])
@pytest.mark.parametrize("kind", ["spread", "tails", "powers", "short", "tiny_first", "leading_zeros", "mantissas"])
@pytest.mark.parametrize("n", [1, 31, 2049, 40961, 128256, 262144])
def test_ordered_sum_bits(kind, n, nucleus):
    """the draw's float64 total (taken in parallel a binade at a time, kernels/kernel.ts:845-850 adds in order) and its
    checkpoints equal the running sums of the adds in index order, to the bit, both as the draw with a nucleus takes
    them (one block) and as the draw without one does (the chunks guessed over the CUs, the first chunk and the
    chunks whose sum crosses a binade walked from their lanes at two binades)"""
    rng = np.random.default_rng(n * 7 + len(kind))
    p = probabilities(kind, n, rng)
    total, cps = gl.ordered_sum(p, nucleus)
    want = in_order(p)
    assert np.float64(total).view(np.uint64) == want[-1].view(np.uint64)
    before = np.concatenate([[0.0], want])[np.arange(0, n, 256)]
    assert np.array_equal(cps.view(np.uint64), before.view(np.uint64))


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_logits_that_are_not_finite_give_minus_one(bad):
    logits = np.random.default_rng(1).standard_normal(5000).astype(np.float32)
    logits[1234] = bad
    assert gl.sample(logits, 0.8, 0.9, 0.5) == -1
    assert gl.sample(np.full(300, -np.inf, dtype=np.float32), 0.8, 0.9, 0.5) == -1


def test_ties_go_in_index_order():
    logits = np.zeros(50, dtype=np.float32)
    logits[[5, 17, 33]] = 3.0
    assert gl.sample(logits, 1.0, 0.5, 0.0) == 5
    assert gl.sample(logits, 1.0, 0.5, 0.999) == 33


def test_a_nucleus_larger_than_the_sort_is_declined():
    logits = np.zeros(20000, dtype=np.float32)  # flat: every token in the nucleus
    assert gl.sample(logits, 1.0, 0.9, 0.5) == -2
    assert gl.sample(logits, 1.0, 1.0, 0.5) == ol.sample(logits, 1.0, 1.0, 0.5)  # no nucleus: no sort
