"""Writes the golden fixtures of the whole-model parity tests (tests/test_gpu_golden.py).

Each fixture is the oracle's answer (oracle/oracle.c, f32: the precision the reference computes in)
for one seeded synthetic model and one seeded prompt:

  prompt      u32[P]     prompt ids, uniform over the vocabulary
  ids         u32[S]     greedy ids: ids[0] is the pick after the prompt, ids[i] the pick after
                         feeding ids[i-1] (Model::decode, kernels/src/model.rs:426-449)
  margin      f32[S+1]   top-1 minus top-2 logit of every logits vector (how close a pick was)
  steps       i32[4]     steps whose logits are sampled: logits after the prompt and s fed ids
  logit_idx   i32[4, N]  sampled vocabulary indices: the 16 largest logits, then a fixed random set
  logit_val   f32[4, N]  oracle logits at those indices
  weights_sha256         hash of weights.bin, so a change of the synthetic generator is caught

The models: "c1" is the 0.8B-shaped decoder with f16 weights, "c2" the 2B-shaped decoder with the
int4 g64 body and f16 embedding / LM head (the model the decode benchmark runs, at a short
context). Run from the repository root: python3 tests/golden/make_golden.py [c1] [c2]
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
}
LOGGED = [0, 1, 63, 127]
RANDOM_IDX = 1024


def synth(case: dict):
    return W.synth_model(case["config"], seed=case["seed"], body=case["body"], head=case["head"], group=case["group"])


def prompt_ids(case: dict, vocab: int) -> np.ndarray:
    return np.random.default_rng(case["prompt_seed"]).integers(0, vocab, size=case["prompt"]).astype(np.uint32)


def weights_hash(buf) -> str:
    return hashlib.sha256(memoryview(np.ascontiguousarray(buf).view(np.uint8))).hexdigest()


def top2_margin(v: np.ndarray) -> float:
    a = np.partition(v, -2)[-2:]
    return float(a[1] - a[0])


def make(name: str) -> Path:
    case = CASES[name]
    t0 = time.time()
    index, buf = synth(case)
    vocab = json.loads(index)["config"]["vocab"]
    om = O.OracleModel(index, buf, "f32")
    prompt = prompt_ids(case, vocab)
    ids, logits = om.greedy(prompt, case["steps"])
    rng = np.random.default_rng(99)
    rand = rng.choice(vocab, size=RANDOM_IDX, replace=False)
    idx, val = [], []
    for s in LOGGED:
        v = logits[s]
        top = np.argsort(-v, kind="stable")[:16]
        sel = np.concatenate([top, rand]).astype(np.int32)
        idx.append(sel)
        val.append(v[sel].astype(np.float32))
    out = ROOT / "tests" / "golden" / f"{name}_greedy.npz"
    np.savez_compressed(out, prompt=prompt, ids=np.asarray(ids, dtype=np.uint32),
                        margin=np.asarray([top2_margin(v) for v in logits], dtype=np.float32),
                        steps=np.asarray(LOGGED, dtype=np.int32), logit_idx=np.stack(idx), logit_val=np.stack(val),
                        weights_sha256=np.asarray(weights_hash(buf)), case=np.asarray(json.dumps(case)))
    print(f"{name}: {out.name} written in {time.time() - t0:.0f} s; min margin {min(top2_margin(v) for v in logits):.4f}",
          flush=True)
    return out


if __name__ == "__main__":
    for n in sys.argv[1:] or list(CASES):
        make(n)
