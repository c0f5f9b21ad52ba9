"""The oracle's restatement of src/sampling.rs (oc_sample), pinned before it checks the device
sampler: the reference's own unit tests (src/sampling.rs:139-207) as known answers, the textbook
xorshift64 (Marsaglia's 13, 7, 17 triple) for the draw stream, the softmax distribution of the
draws (chi-square), the top-k / top-p truncation against float64 arithmetic, and an inverse-CDF
brute force over the same uniform draws."""
import ctypes

import numpy as np
import pytest
from scipy import stats

import cpu_oracle as O
from cpu_oracle import OracleSampler, bitset

M64 = (1 << 64) - 1


def xorshift_ref(seed, n):
    """Marsaglia's xorshift64 (13, 7, 17) from Sampler::new's seeding, as 24-bit fractions."""
    x = ((seed * 0x9E3779B97F4A7C15) & M64) | 1
    out = []
    for _ in range(n):
        x ^= (x << 13) & M64
        x ^= x >> 7
        x ^= (x << 17) & M64
        out.append((x >> 40) / float(1 << 24))
    return out


# ---- the reference's unit tests (src/sampling.rs:139-207) ----

def test_reference_impossible_and_corrupt_distributions_are_errors():
    s = OracleSampler()
    with pytest.raises(ValueError):
        s.sample([1.0, 2.0], mask=bitset([], 2), mask_len=2)
    for bad in ([np.nan], [-np.inf], []):
        with pytest.raises(ValueError):
            s.sample(bad)


def test_reference_greedy_picks_max_and_respects_mask():
    logits = [0.0, 3.0, 1.0, 2.0]
    s = OracleSampler(temperature=0.0)
    assert s.sample(logits) == 1
    assert s.sample(logits, mask=bitset([2, 3], 4), mask_len=4) == 3


def test_reference_stochastic_respects_mask_and_top_k():
    logits = [5.0, 4.9, 4.8, -9.0]
    s = OracleSampler(temperature=1.0, top_k=1, top_p=1.0, seed=7)
    for _ in range(50):
        assert s.sample(logits, mask=bitset([1, 3], 4), mask_len=4) == 1


def test_reference_same_seed_is_deterministic():
    logits = np.sin(np.arange(100, dtype=np.float32) * np.float32(0.7))

    def draw(seed):
        s = OracleSampler(temperature=1.0, top_k=50, top_p=0.95, seed=seed)
        return [s.sample(logits) for _ in range(30)]

    assert draw(1) == draw(1)
    assert draw(1) != draw(2)


def test_reference_tool_call_bias_flips_greedy_when_added_to_logits():
    logits = np.array([1.0, 3.0, 0.0], np.float32)
    assert OracleSampler(temperature=0.0).sample(logits) == 1
    logits[0] += 4.0
    assert OracleSampler(temperature=0.0).sample(logits) == 0
    logits[0] -= 12.0
    assert OracleSampler(temperature=0.0).sample(logits) == 1


def test_reference_presence_penalty_avoids_repeats_but_not_under_a_mask():
    logits = [0.0, 3.0, 2.5, 0.0]
    s = OracleSampler(temperature=0.0, presence_penalty=1.0)
    assert s.sample(logits) == 1
    assert s.sample(logits) == 2  # token 1 is penalised once generated
    assert s.sample(logits, mask=bitset([1, 2], 4), mask_len=4) == 1  # no penalty inside the grammar


# ---- the draw stream and the distribution ----

def test_draw_stream_is_xorshift64():
    L = O.lib("f32")
    for seed in (0, 1, 42, 7, 2**63 + 5):
        st = ctypes.c_uint64(L.oc_sampler_seed(seed))
        got = [L.oc_sampler_next_f32(ctypes.byref(st)) for _ in range(2000)]
        assert got == xorshift_ref(seed, 2000)


def test_draws_follow_the_softmax():
    logits = np.array([1.0, 0.3, -0.5, 2.0, 0.0, 1.2], np.float32)
    t = 0.7
    s = OracleSampler(temperature=t, top_k=6, top_p=1.0, seed=3)
    n = 40000
    counts = np.bincount([s.sample(logits) for _ in range(n)], minlength=6)
    p = np.exp((logits.astype(np.float64) - logits.max()) / t)
    p /= p.sum()
    assert stats.chisquare(counts, p * counts.sum()).pvalue > 1e-3


@pytest.mark.parametrize("top_k,top_p", [(3, 1.0), (8, 0.5), (8, 0.9), (2, 0.3)])
def test_draws_stay_in_the_top_k_top_p_prefix(top_k, top_p):
    rng = np.random.default_rng(top_k * 10 + int(top_p * 10))
    logits = rng.normal(0, 1.5, size=8).astype(np.float32)
    t = 0.9
    s = OracleSampler(temperature=t, top_k=top_k, top_p=top_p, seed=11)
    n = 20000
    draws = np.array([s.sample(logits) for _ in range(n)])
    order = np.argsort(-logits.astype(np.float64), kind="stable")[:top_k]
    w = np.exp((logits[order].astype(np.float64) - logits[order[0]]) / t)
    cum = np.cumsum(w)
    m = int(np.searchsorted(cum, top_p * w.sum() * (1 - 1e-6)) + 1)  # smallest prefix reaching top_p
    keep = order[:min(m, top_k)]
    assert set(np.unique(draws)) <= set(keep.tolist())
    counts = np.array([(draws == i).sum() for i in keep])
    q = w[:len(keep)] / w[:len(keep)].sum()
    if len(keep) > 1:
        assert stats.chisquare(counts, q * counts.sum()).pvalue > 1e-3


def test_inverse_cdf_brute_force():
    """Each draw is the token whose cumulative weight first reaches u * kept, u the stream's next
    value: recomputed in float64 from the same u (ties within 1e-5 of a boundary are skipped)."""
    rng = np.random.default_rng(5)
    for trial in range(20):
        V = int(rng.integers(2, 40))
        logits = rng.normal(0, 2, size=V).astype(np.float32)
        t, k, p = float(rng.uniform(0.3, 2.0)), int(rng.integers(1, V + 1)), float(rng.uniform(0.2, 1.0))
        seed = int(rng.integers(0, 2**32))
        s = OracleSampler(temperature=t, top_k=k, top_p=p, seed=seed)
        us = xorshift_ref(seed, 30)
        order = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
        w = np.exp((logits[order].astype(np.float64) - logits[order[0]]) / t)
        cum = np.cumsum(w)
        m = int(np.argmax(cum >= p * w.sum() * (1 - 1e-9))) + 1
        kept = cum[m - 1]
        for u in us:
            got = s.sample(logits)
            target = u * kept
            j = int(np.argmax(cum[:m] >= target)) if target <= kept else m - 1
            if np.min(np.abs(cum[:m] - target)) < 1e-5 * kept:
                continue
            assert got == order[j], (trial, u)


def test_penalty_marks_tokens_under_a_mask_too():
    """sample() remembers every pick for the penalty, including picks made under a mask."""
    logits = [0.0, 3.0, 2.5, 0.0]
    s = OracleSampler(temperature=0.0, presence_penalty=1.0)
    assert s.sample(logits, mask=bitset([1, 2], 4), mask_len=4) == 1
    assert s.sample(logits) == 2


def test_nan_outside_the_mask_is_ignored_and_equal_maxima_take_the_lowest_token():
    logits = [np.nan, 1.0, 1.0, 0.5]
    assert OracleSampler(temperature=0.0).sample(logits, mask=bitset([1, 2, 3], 4), mask_len=4) == 1
    s = OracleSampler(temperature=1.0, top_k=1, top_p=1.0)
    assert s.sample([0.0, 2.0, 2.0]) == 1
