"""Whole-model logit checks shared by the parity tests.

reference_gate() is the reference's own model-level gate (kernels/src/bin/model_bench.rs:125-153,
helpers top / cosine at :34-47): cosine similarity of the two logit vectors (accumulated in f64)
above 0.9999, the same top-1 id, and at least 4 of the 5 largest ids shared. check_logits() adds
the tolerance this engine is held to over the whole vocabulary: max |logit - oracle logit| <= 1e-2.
"""
from __future__ import annotations

import numpy as np

LOGIT_TOL = 1e-2  # max |logit - oracle logit| over the whole vocabulary
COSINE_MIN = 0.9999  # model_bench.rs:132
TOP5_MIN = 4  # model_bench.rs:132


def top(v: np.ndarray, k: int) -> list[int]:
    """Ids of the k largest values, largest first (model_bench.rs:34-40; equal values by id)."""
    return [int(i) for i in np.argsort(-np.asarray(v, dtype=np.float64), kind="stable")[:k]]


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    """model_bench.rs:42-47: products and norms accumulated in f64."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.dot(a, b) / (np.sqrt(np.dot(a, a)) * np.sqrt(np.dot(b, b))))


def reference_gate(got: np.ndarray, want: np.ndarray) -> dict:
    ours5, ref5 = top(got, 5), top(want, 5)
    overlap = sum(1 for i in ours5 if i in ref5)
    cos = cosine(got, want)
    return {"cosine": cos, "top1": ours5[0] == ref5[0], "overlap": overlap,
            "max_diff": float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)))),
            "ok": cos > COSINE_MIN and ours5[0] == ref5[0] and overlap >= TOP5_MIN}


def check_logits(got: np.ndarray, want: np.ndarray, what: str) -> dict:
    """Asserts the reference's gate and the full-vocabulary tolerance; returns the figures."""
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite logits"
    g = reference_gate(got, want)
    assert g["ok"], f"{what}: reference gate failed: {g}"
    assert g["max_diff"] <= LOGIT_TOL, f"{what}: max |dlogit| {g['max_diff']:.3e} > {LOGIT_TOL}"
    return g
