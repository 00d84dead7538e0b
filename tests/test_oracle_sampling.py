"""The oracle's sampler (or_penalize, or_sample: kernels/kernel.ts:705-868) pinned by the reference's own sampler
tests restated (tests/test_sample.py) and by the draws of NumPy's Llama.sample (public/llama2_numpy.py:1529-1563),
restated below in float64 NumPy, away from its boundaries (tests/smoke.mjs:176-272 holds the kernel to it)."""
import math

import numpy as np
import pytest

import oracle_lib as ol

GRID = np.linspace(0.0, 1.0, 1001)[:-1]


def softmax(logits, temperature=1.0):
    p = np.exp((logits.astype(np.float64) - logits.max()) / temperature)
    return p / p.sum()


def reference_nucleus(logits, temperature, topp):
    """tests/test_sample.py:30-35: the smallest set of most probable tokens whose probabilities reach topp"""
    p = softmax(logits, temperature)
    order = np.argsort(-p)
    cumulative = np.cumsum(p[order])
    return set(order[:int(np.searchsorted(cumulative, topp)) + 1].tolist())


def numpy_sample(logits, temperature, topp, u):
    """public/llama2_numpy.py:1529-1563 Llama.sample in NumPy, with the boundaries its draw lies between: (token,
    distance from u * mass to the nearest running sum, mass)"""
    best = logits.max()
    nucleus = 0.0 < topp < 1.0
    if nucleus:
        candidates = np.flatnonzero(logits >= best + temperature * math.log(1e-7))
        p = np.exp((logits[candidates] - best) / np.float32(temperature)).astype(np.float64)
    else:
        candidates = np.arange(logits.size)
        p = np.exp((logits - best) / np.float32(temperature)).astype(np.float64)
    p /= p.sum()
    if nucleus:
        cutoff = min((1.0 - topp) / max(p.size - 1, 1), p.max())
        likely = np.flatnonzero(p >= cutoff)
        likely = likely[np.argsort(-p[likely], kind="stable")]
        candidates, p = candidates[likely], p[likely]
        cumulative = np.cumsum(p)
        cumulative = cumulative[:np.searchsorted(cumulative, topp) + 1]
    else:
        cumulative = np.cumsum(p)
    target = u * cumulative[-1]
    chosen = np.searchsorted(cumulative, target, side="right")
    gap = np.min(np.abs(cumulative - target))
    return int(candidates[min(chosen, cumulative.size - 1)]), gap, cumulative[-1]


def test_nucleus_is_exactly_the_top_p_set():
    """tests/test_sample.py:44-49"""
    logits = (np.random.default_rng(1).standard_normal(200) * 3.0).astype(np.float32)
    drawn = {ol.sample(logits, 1.0, 0.9, u) for u in GRID}
    assert drawn == reference_nucleus(logits, 1.0, 0.9)


def test_a_peaked_distribution_leaves_one_candidate():
    """tests/test_sample.py:52-56"""
    logits = np.full(200, -20.0, dtype=np.float32)
    logits[42] = 20.0
    assert {ol.sample(logits, 1.0, 0.9, u) for u in (0.0, 0.5, 0.999)} == {42}


def test_frequencies_follow_the_distribution():
    """tests/test_sample.py:59-65"""
    logits = np.array([2.0, 1.0, 0.0, -1.0, -2.0], dtype=np.float32)
    expected = softmax(logits)
    draws = 4000
    rng = np.random.default_rng(3)
    counts = np.bincount([ol.sample(logits, 1.0, 1.0, rng.random()) for _ in range(draws)], minlength=logits.size)
    sigma = np.sqrt(draws * expected * (1 - expected))
    assert (np.abs(counts - draws * expected) < 5 * sigma).all(), counts


def test_a_low_temperature_sharpens():
    """tests/test_sample.py:68-71"""
    logits = np.array([2.0, 1.9, 0.0], dtype=np.float32)
    assert [ol.sample(logits, 0.01, 1.0, u) for u in (0.1, 0.5, 0.9)] == [0, 0, 0]


def test_penalize_divides_positive_and_multiplies_negative_logits():
    """tests/test_sample.py:74-77: each distinct token once"""
    out = ol.penalize(np.array([2.0, -2.0, 5.0, -5.0], dtype=np.float32), [0, 1, 1], 2.0)
    assert out.tolist() == [1.0, -4.0, 5.0, -5.0]


def test_penalize_rounds_as_float32():
    logits = np.array([3.0, -3.0, 0.0, -0.0], dtype=np.float32)
    out = ol.penalize(logits, [0, 1, 2, 3], 1.3)
    assert out.tolist() == [np.float32(3.0) / np.float32(1.3), np.float32(-3.0) * np.float32(1.3), 0.0, -0.0]


@pytest.mark.parametrize("topp", [0.05, 0.1, 0.2, 0.45])
@pytest.mark.parametrize("above", [1, 2, 3, 5])
def test_a_low_top_p_over_few_likely_tokens(topp, above):
    """tests/test_sample.py:86-100 (T178)"""
    rng = np.random.default_rng(above)
    for spread in (0.0, 0.05, 0.5):
        logits = np.full(200, -100.0, dtype=np.float32)
        logits[rng.choice(200, above, replace=False)] = (5.0 + rng.standard_normal(above) * spread).astype(np.float32)
        for temperature in (0.1, 0.2, 1.0):
            drawn = {ol.sample(logits, temperature, topp, u) for u in np.linspace(0.0, 1.0, 101)[:-1]}
            if spread == 0.0:
                assert drawn <= set(np.flatnonzero(logits == logits.max()).tolist())
            else:
                assert drawn == reference_nucleus(logits, temperature, topp)


@pytest.mark.parametrize("where", [0, 7, 199])
@pytest.mark.parametrize("bad", [np.nan, np.inf])
@pytest.mark.parametrize("temperature, topp", [(1.0, 0.9), (0.7, 1.0)])
def test_logits_that_are_not_finite_give_minus_one(where, bad, temperature, topp):
    """tests/test_sample.py:103-114 (T195): kernel.ts's sample() returns -1"""
    logits = np.random.default_rng(where).standard_normal(200).astype(np.float32)
    logits[where] = bad
    assert ol.sample(logits, temperature, topp, 0.5) == -1
    assert ol.sample(np.full(200, -np.inf, dtype=np.float32), temperature, topp, 0.5) == -1


def test_some_minus_infinity_is_never_drawn():
    """tests/test_sample.py:117-125"""
    logits = np.random.default_rng(3).standard_normal(200).astype(np.float32)
    logits[::3] = -np.inf
    for topp in (0.9, 1.0):
        drawn = {ol.sample(logits, 1.0, topp, u) for u in np.linspace(0.0, 1.0, 51)[:-1]}
        assert all(np.isfinite(logits[t]) for t in drawn)


def test_equal_probabilities_in_the_nucleus_go_in_index_order():
    """ties: the lowest index first (public/shaders.js's sampleLikeCpu), so u = 0 draws the first of the largest"""
    logits = np.zeros(50, dtype=np.float32)
    logits[[5, 17, 33]] = 3.0
    assert ol.sample(logits, 1.0, 0.5, 0.0) == 5
    assert ol.sample(logits, 1.0, 0.5, 0.999) == 33


@pytest.mark.parametrize("n, scale", [(200, 3.0), (1000, 1.0), (32000, 4.0)])
@pytest.mark.parametrize("temperature, topp", [(0.7, 0.9), (1.0, 1.0), (0.3, 0.5), (1.3, 0.95)])
def test_draws_equal_numpy_sample_away_from_boundaries(n, scale, temperature, topp):
    rng = np.random.default_rng(n + int(100 * temperature))
    agreed = 0
    for _ in range(4):
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        for u in rng.random(25):
            want, gap, mass = numpy_sample(logits, temperature, topp, u)
            if gap < 1e-5 * mass:
                continue  # within float32 exp's difference of a boundary
            assert ol.sample(logits, temperature, topp, u) == want
            agreed += 1
    assert agreed >= 80
