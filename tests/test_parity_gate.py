"""The whole-model logit checks (tests/parity.py) against what they must accept and reject (CPU),
and the committed fixtures' full-vocabulary logits against the rest of each fixture.

The gate is the reference's (kernels/src/bin/model_bench.rs:125-153). Planted mistakes: a swapped
top-1 / top-2 pair, a scaled vector (cosine 1, values off), a single far-off logit, a shuffled
tail. The fixtures' logits_full rows must hold exactly the sampled values at the sampled indices,
and their argmax must be the next greedy id."""
import json
from pathlib import Path

import numpy as np
import pytest

import parity as P

GOLDEN = Path(__file__).resolve().parent / "golden"


def logits(seed=0, n=151936):
    return np.random.default_rng(seed).normal(0.0, 2.0, size=n).astype(np.float32)


def test_identical_vectors_pass():
    v = logits()
    g = P.check_logits(v, v.copy(), "same")
    assert g["cosine"] > 0.999999 and g["overlap"] == 5 and g["max_diff"] == 0.0


def test_small_noise_passes_and_top_k_follows_the_values():
    v = logits(1)
    w = v + np.random.default_rng(2).normal(0.0, 1e-4, size=v.size).astype(np.float32)
    P.check_logits(w, v, "noise")
    assert P.top(np.array([1.0, 5.0, 3.0, 5.0, -1.0]), 3) == [1, 3, 2]  # equal values: lower id first


def test_swapped_top1_fails_the_gate():
    v = logits(3)
    a, b = P.top(v, 2)
    w = v.copy()
    w[a], w[b] = v[b], v[a]
    g = P.reference_gate(w, v)
    assert not g["top1"] and not g["ok"]


def test_scaled_vector_passes_cosine_but_fails_the_tolerance():
    v = logits(4)
    w = v * 1.01
    g = P.reference_gate(w, v)
    assert g["ok"] and g["cosine"] > 0.99999  # the reference's gate alone accepts it
    with pytest.raises(AssertionError):
        P.check_logits(w, v, "scaled")


def test_one_far_off_logit_fails_the_tolerance():
    v = logits(5)
    w = v.copy()
    w[12345] += 0.05
    with pytest.raises(AssertionError):
        P.check_logits(w, v, "one off")


def test_shuffled_tail_fails_cosine():
    v = logits(6)
    w = v.copy()
    keep = P.top(v, 5)
    rest = np.setdiff1d(np.arange(v.size), keep)
    w[rest] = np.random.default_rng(7).permutation(v[rest])
    g = P.reference_gate(w, v)
    assert g["overlap"] == 5 and g["cosine"] < P.COSINE_MIN and not g["ok"]


@pytest.mark.parametrize("name", ["c1", "c2", "c2_long"])
def test_fixture_full_logits_agree_with_the_rest_of_the_fixture(name):
    f = np.load(GOLDEN / f"{name}_greedy.npz")
    if "logits_full" not in f.files:
        pytest.skip(f"{name}: fixture without full logits")
    full, idx, val, steps, ids = f["logits_full"], f["logit_idx"], f["logit_val"], f["steps"], f["ids"]
    case = json.loads(str(f["case"]))
    assert full.shape == (len(steps), 151936) and full.dtype == np.float32
    for j, s in enumerate(steps):
        assert np.array_equal(full[j][idx[j]], val[j]), f"{name} step {s}: sampled values differ"
        # logits after the prompt and s fed ids: their argmax is greedy id s
        assert int(np.argmax(full[j])) == int(ids[s]), f"{name} step {s}"
        assert np.all(np.isfinite(full[j]))
    assert len(ids) == case["steps"]
