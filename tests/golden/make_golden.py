"""Writes the golden fixtures of the whole-model parity tests (tests/test_gpu_golden.py,
tests/test_gpu_batch.py).

Each fixture is the oracle's answer (oracle/oracle.c, f32: the precision the reference computes in)
for one seeded synthetic model and seeded prompts:

  prompt      u32[P]     prompt ids, uniform over the vocabulary (rows cases: u32[R][P_max],
                         with plen i32[R] the length of each row's prompt)
  ids         u32[S]     greedy ids: ids[0] is the pick after the prompt, ids[i] the pick after
                         feeding ids[i-1] (Model::decode, kernels/src/model.rs:426-449)
                         (rows cases: u32[R][S])
  margin      f32[S+1]   top-1 minus top-2 logit of every logits vector (how close a pick was)
  steps       i32[4]     steps whose logits are sampled: logits after the prompt and s fed ids
  logit_idx   i32[4, N]  sampled vocabulary indices: the 16 largest logits, then a fixed random set
  logit_val   f32[4, N]  oracle logits at those indices (rows cases: an extra leading row axis)
  logits_full f32[4, V]  every oracle logit at the logged steps (single-sequence cases), for the
                         full-vocabulary check and the reference's model-level gate (cosine, top-1,
                         top-5 overlap; kernels/src/bin/model_bench.rs:125-153)
  weights_sha256         hash of weights.bin, so a change of the synthetic generator is caught

The models: "c1" is the 0.8B-shaped decoder with f16 weights, "c2" the 2B-shaped decoder with the
int4 g64 body and f16 embedding / LM head (the model the decode benchmark runs) at a short context.
"c2_long" is the same 2B model after a 4000-id prompt, decoded over positions 4000..4095 (the
decode benchmark's own positions). "small_long" is the 8-layer "small" model with an 8192-token
cache after a 5500-id prompt: its attention splits hold more positions than the decode kernel
prefetches, so the kernel's direct-load path runs. "c5_rows" holds three sequences of the 2B model (prompts of 256,
640 and 1024 ids, 16 greedy steps each) that the batched-decode test admits into a 64-row batch.
Run from the repository root: python3 tests/golden/make_golden.py [c1] [c2] [c2_long] [c5_rows]
[small_long]
(c2_long runs the oracle over ~4100 tokens of the 2B model: about half an hour on 8 cores).
"""
from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "qwen-native-engine_amd"), str(ROOT / "oracle")]

import cpu_oracle as O  # noqa: E402
import weights as W  # noqa: E402

CASES = {
    "c1": dict(config="0.8b", body="f16", head="f16", group=64, seed=1, prompt_seed=2, prompt=128, steps=128),
    "c2": dict(config="2b", body="q4", head="f16", group=64, seed=0, prompt_seed=3, prompt=128, steps=128),
    "c2_long": dict(config="2b", body="q4", head="f16", group=64, seed=0, prompt_seed=5, prompt=4000, steps=96,
                    logged=[0, 1, 47, 95]),
    "c5_rows": dict(config="2b", body="q4", head="f16", group=64, seed=0, prompt_seed=7, prompt=[256, 640, 1024],
                    steps=16, logged=[0, 1, 8, 15]),
    "small_long": dict(config="small", body="q4", head="f16", group=64, seed=12, prompt_seed=13, prompt=5500, steps=16,
                       logged=[0, 1, 8, 15], max_context=8192),
}
LOGGED = [0, 1, 63, 127]
RANDOM_IDX = 1024


def synth(case: dict):
    return W.synth_model(case["config"], seed=case["seed"], body=case["body"], head=case["head"], group=case["group"])


def prompt_ids(case: dict, vocab: int) -> np.ndarray:
    """The case's prompt; for a rows case, row r is the first plen[r] ids of row r of the result."""
    rng = np.random.default_rng(case["prompt_seed"])
    if isinstance(case["prompt"], list):
        lens = case["prompt"]
        out = np.zeros((len(lens), max(lens)), dtype=np.uint32)
        for r, n in enumerate(lens):
            out[r, :n] = rng.integers(0, vocab, size=n)
        return out
    return rng.integers(0, vocab, size=case["prompt"]).astype(np.uint32)


def weights_hash(buf) -> str:
    return hashlib.sha256(memoryview(np.ascontiguousarray(buf).view(np.uint8))).hexdigest()


def top2_margin(v: np.ndarray) -> float:
    a = np.partition(v, -2)[-2:]
    return float(a[1] - a[0])


def run_sequence(om, prompt, steps: int, name: str):
    """Prefill (in 500-token calls, so progress shows; the oracle runs tokens one by one either way)
    then greedy decode; returns (ids, logits per step)."""
    om.reset()
    t0 = time.time()
    n = len(prompt)
    for s in range(0, n, 500):
        part = prompt[s:s + 500]
        logits = om.prefill_chunk(part, s, s + len(part) == n)
        print(f"  {name}: prefilled {s + len(part)}/{n} ids in {time.time() - t0:.0f} s", flush=True)
    ids, all_logits = [], [logits]
    pos = n
    for i in range(steps):
        t = int(np.argmax(logits))  # lowest index among equal maxima, like oc_argmax
        ids.append(t)
        logits = om.token(t, pos)
        all_logits.append(logits)
        pos += 1
    print(f"  {name}: {steps} greedy steps done at {time.time() - t0:.0f} s", flush=True)
    return ids, all_logits


def sampled(logits, logged, rand):
    idx, val = [], []
    for s in logged:
        v = logits[s]
        top = np.argsort(-v, kind="stable")[:16]
        sel = np.concatenate([top, rand]).astype(np.int32)
        idx.append(sel)
        val.append(v[sel].astype(np.float32))
    return np.stack(idx), np.stack(val)


def make(name: str) -> Path:
    case = CASES[name]
    t0 = time.time()
    index, buf = synth(case)
    vocab = json.loads(index)["config"]["vocab"]
    om = O.OracleModel(index, buf, "f32", max_context=case.get("max_context", 4096))
    prompt = prompt_ids(case, vocab)
    logged = case.get("logged", LOGGED)
    rand = np.random.default_rng(99).choice(vocab, size=RANDOM_IDX, replace=False)
    out = ROOT / "tests" / "golden" / f"{name}_greedy.npz"
    common = dict(steps=np.asarray(logged, dtype=np.int32), weights_sha256=np.asarray(weights_hash(buf)),
                  case=np.asarray(json.dumps(case)))
    if prompt.ndim == 2:
        rows = [run_sequence(om, prompt[r, :n], case["steps"], f"{name} row {r}") for r, n in enumerate(case["prompt"])]
        si = [sampled(lg, logged, rand) for _, lg in rows]
        np.savez_compressed(out, prompt=prompt, plen=np.asarray(case["prompt"], dtype=np.int32),
                            ids=np.asarray([ids for ids, _ in rows], dtype=np.uint32),
                            margin=np.asarray([[top2_margin(v) for v in lg] for _, lg in rows], dtype=np.float32),
                            logit_idx=np.stack([a for a, _ in si]), logit_val=np.stack([b for _, b in si]), **common)
        margins = [top2_margin(v) for _, lg in rows for v in lg]
    else:
        ids, logits = run_sequence(om, prompt, case["steps"], name)
        idx, val = sampled(logits, logged, rand)
        full = np.stack([np.asarray(logits[s], dtype=np.float32) for s in logged])
        np.savez_compressed(out, prompt=prompt, ids=np.asarray(ids, dtype=np.uint32),
                            margin=np.asarray([top2_margin(v) for v in logits], dtype=np.float32),
                            logit_idx=idx, logit_val=val, logits_full=full, **common)
        margins = [top2_margin(v) for v in logits]
    print(f"{name}: {out.name} written in {time.time() - t0:.0f} s; min margin {min(margins):.4f}", flush=True)
    return out


if __name__ == "__main__":
    for n in sys.argv[1:] or list(CASES):
        make(n)
