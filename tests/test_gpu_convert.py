"""A converted transformers checkpoint on the GPU: the engine's logits at every prompt position
against transformers' own forward pass (f16 body), and the int4-converted file against the oracle
with identical greedy ids. Bar: max |logit error| <= 2e-3 against transformers (the f16 K/V cache
moves these logits by up to ~4e-4; the oracle/engine gap is far smaller) and <= 1e-3 against
the oracle."""
import numpy as np
import pytest

import hf_tiny
import cpu_oracle as O
import convert_safetensors as C
import qne as Q

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not hf_tiny.available(), reason="transformers qwen3_5 / safetensors not importable")]


IDS = np.random.default_rng(5).integers(0, hf_tiny.TINY["vocab_size"], size=24)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    """The seeded tiny transformers model, saved, and its logits at every position of IDS; made in a
    child process so that this GPU test process never loads torch."""
    src, want = hf_tiny.build_in_subprocess(3, tmp_path_factory.mktemp("hf"), IDS)
    return want, src


def load(d):
    return (d / "index.json").read_text(encoding="utf-8"), np.fromfile(d / "weights.bin", dtype=np.uint8)


@pytest.mark.parametrize("engine", ["persistent", "graph"])
def test_engine_on_converted_checkpoint_matches_transformers(checkpoint, tmp_path, engine):
    want, src = checkpoint
    C.convert(src, tmp_path / "f16", body="f16", head="f16")
    index, buf = load(tmp_path / "f16")
    ids = IDS
    m = Q.Model.load(index, buf, options={"engine": engine})
    try:
        got = np.stack([m.step(int(t), p) for p, t in enumerate(ids)])
    finally:
        m.close()
    err = float(np.abs(got - want).max())
    assert err <= 2e-3, err
    assert (got.argmax(1) == want.argmax(1)).all()


def test_int4_converted_checkpoint_greedy_matches_oracle(checkpoint, tmp_path):
    _, src = checkpoint
    C.convert(src, tmp_path / "q4", body="q4", head="f16", group=64)
    index, buf = load(tmp_path / "q4")
    ids = np.random.default_rng(6).integers(0, hf_tiny.TINY["vocab_size"], size=30).astype(np.uint32)
    om = O.OracleModel(index, buf, "f64")
    want_ids, want_logits = om.greedy(ids, 32)
    m = Q.Model.load(index, buf)
    try:
        m.prefill_batched(ids)
        first = m.logits()
        out = m.decode_ids(32, 8, [])
    finally:
        m.close()
    assert float(np.abs(first - want_logits[0]).max()) <= 1e-3
    assert out == want_ids
