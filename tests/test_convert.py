"""The safetensors converter (qwen-native-engine_amd/convert_safetensors.py) against transformers'
own Qwen3.5 implementation: a tiny seeded model is saved as a checkpoint, converted, and the
oracle run on the converted files must give transformers' logits at every prompt position.

This pins the converter's tensor mapping (names, the (1 + w) norm gains, -exp(A_log), the
q/gate de-interleave, the q, k, v, z, a, b row order, the conv tap layout) and, independently of
the reference, the oracle's model math. Tolerance: transformers runs in float32 (chunked delta
rule, SDPA), the oracle in float64, on identical weights (bf16 values are exact in f16); the
oracle keeps K and V as f16, as the engine's cache does, which alone moves these logits (of
magnitude ~2.5) by up to ~4e-4. Bar: max |logit error| <= 1e-3, identical argmax at every
position. Planted mistakes in the converted data (one per kind of mapping error) must each move
the logits by more than 20x that."""
import json

import numpy as np
import pytest

import hf_tiny
import cpu_oracle as O
import convert_safetensors as C
import weights as W

pytestmark = pytest.mark.skipif(not hf_tiny.available(), reason="transformers qwen3_5 / safetensors not importable")

TOL = 1e-3


@pytest.fixture(scope="module")
def hf_model():
    return hf_tiny.build(seed=3)


@pytest.fixture(scope="module")
def converted(hf_model, tmp_path_factory):
    src = hf_tiny.save(hf_model, tmp_path_factory.mktemp("hf"))
    out = tmp_path_factory.mktemp("native")
    C.convert(src, out, body="f16", head="f16")
    return out


def prompt(n=24, seed=5):
    return np.random.default_rng(seed).integers(0, hf_tiny.TINY["vocab_size"], size=n)


def oracle_logits(index, buf, ids):
    om = O.OracleModel(index, buf, "f64")
    return np.stack([om.token(int(t), p) for p, t in enumerate(ids)])


def load(d):
    return (d / "index.json").read_text(encoding="utf-8"), np.fromfile(d / "weights.bin", dtype=np.uint8)


def test_config_maps_to_format_2(converted):
    ix = json.loads((converted / "index.json").read_text(encoding="utf-8"))
    assert ix["format_version"] == 2
    want = W.full_config("tiny")
    for k in ("layers", "full_attention_every", "hidden", "intermediate", "vocab", "rope_dim", "n_q_heads",
              "n_kv_heads", "head_dim", "gdn_heads", "gdn_dk", "gdn_dv", "conv_kernel"):
        assert ix["config"][k] == want[k], k
    assert ix["config"]["rope_theta"] == 1e7
    assert all(m["dtype"] == "f16" for m in ix["matrices"].values())


def test_oracle_on_converted_checkpoint_matches_transformers(hf_model, converted):
    ids = prompt()
    want = hf_tiny.logits(hf_model, ids)
    index, buf = load(converted)
    got = oracle_logits(index, buf, ids)
    assert float(np.abs(want).max()) > 0.3  # logits carry signal
    err = float(np.abs(got - want).max())
    assert err <= TOL, err
    assert (got.argmax(1) == want.argmax(1)).all()


def _vector(ix, buf, name):
    t = ix["tensors"][name]
    return np.frombuffer(buf, dtype=np.float32, count=t["bytes"] // 4, offset=t["offset"])


def _matrix_f16(ix, buf, name):
    t = ix["tensors"][name + ".w"]
    return np.frombuffer(buf, dtype=np.uint16, count=t["bytes"] // 2, offset=t["offset"]).reshape(t["shape"])


@pytest.mark.parametrize("mistake", ["norm_without_one", "a_b_swapped", "decay_sign", "q_gate_interleaved",
                                     "conv_taps_reversed"])
def test_planted_mapping_mistakes_are_caught(hf_model, converted, mistake):
    ids = prompt(12, 7)
    want = hf_tiny.logits(hf_model, ids)
    index, buf = load(converted)
    ix = json.loads(index)
    buf = buf.copy()
    cfg = ix["config"]
    H, dk, dv = cfg["gdn_heads"], cfg["gdn_dk"], cfg["gdn_dv"]
    if mistake == "norm_without_one":
        _vector(ix, buf, "layer0.input_norm")[:] -= 1.0
    elif mistake == "a_b_swapped":
        w = _matrix_f16(ix, buf, "layer0.mixer_in")
        a0 = 2 * H * dk + 2 * H * dv
        a, b = w[a0:a0 + H].copy(), w[a0 + H:a0 + 2 * H].copy()
        w[a0:a0 + H], w[a0 + H:a0 + 2 * H] = b, a
    elif mistake == "decay_sign":
        v = _vector(ix, buf, "layer0.gdn_params")
        v[H:2 * H] = -v[H:2 * H]
    elif mistake == "q_gate_interleaved":
        w = _matrix_f16(ix, buf, "layer3.mixer_in")
        hd, nq = cfg["head_dim"], cfg["n_q_heads"]
        qg = w[:2 * nq * hd].copy().reshape(2, nq, hd, -1)
        w[:2 * nq * hd] = qg.transpose(1, 0, 2, 3).reshape(2 * nq * hd, -1)
    elif mistake == "conv_taps_reversed":
        v = _vector(ix, buf, "layer0.conv_w").reshape(-1, cfg["conv_kernel"])
        v[:] = v[:, ::-1].copy()
    got = oracle_logits(index, buf, ids)
    err = float(np.abs(got - want).max())
    assert not err <= 20 * TOL, err  # a NaN (a decay above 1 blows up) counts as caught


def test_multimodal_names_and_tied_head(tmp_path):
    m = hf_tiny.build(seed=4, tied=True)
    src = hf_tiny.save(m, tmp_path / "hf", multimodal=True)
    C.convert(src, tmp_path / "native", body="f16", head="f16")
    index, buf = load(tmp_path / "native")
    ix = json.loads(index)
    assert ix["tensors"]["lm_head.w"]["offset"] == ix["tensors"]["embed.w"]["offset"]  # stored once
    ids = prompt(10, 9)
    err = float(np.abs(oracle_logits(index, buf, ids) - hf_tiny.logits(m, ids)).max())
    assert err <= TOL, err


def test_int4_body_is_the_groupwise_quantisation(hf_model, tmp_path):
    """--body q4: every layer matrix is the group-64 int4 quantisation of the checkpoint's values
    (each weight within half a step, (q - z) * s, of its bf16 value), the f16 embedding and head
    are untouched, and the oracle runs the file."""
    src = hf_tiny.save(hf_model, tmp_path / "hf")
    ix = C.convert(src, tmp_path / "q4", body="q4", head="f16", group=64)
    assert ix["matrices"]["layer0.down"] == {"rows": 512, "k": 1024, "dtype": "q4", "group": 64, "zero": "f16"}
    assert ix["matrices"]["embed"]["dtype"] == "f16" and ix["matrices"]["lm_head"]["dtype"] == "f16"
    index, buf = load(tmp_path / "q4")
    sd = hf_model.state_dict()
    for name, ref in (("layer0.down", sd["model.layers.0.mlp.down_proj.weight"]),
                      ("layer3.mixer_out", sd["model.layers.3.self_attn.o_proj.weight"])):
        m = ix["matrices"][name]
        rows, k, g = m["rows"], m["k"], m["group"]
        t = lambda suffix, dt: np.frombuffer(buf, dtype=dt, count=ix["tensors"][name + suffix]["bytes"] // np.dtype(dt).itemsize,
                                             offset=ix["tensors"][name + suffix]["offset"])
        words = t(".w", np.uint32).reshape(rows, k // 8)
        q = ((words[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(rows, k).astype(np.float64)
        sc = t(".s", np.float16).astype(np.float64).reshape(rows, k // g)
        zp = t(".z", np.float16).astype(np.float64).reshape(rows, k // g)
        deq = (q - np.repeat(zp, g, 1)) * np.repeat(sc, g, 1)
        w = ref.double().numpy()
        assert np.all(np.abs(deq - w) <= 0.5 * np.repeat(sc, g, 1) * 1.01 + 1e-7), name
    out = oracle_logits(index, buf, prompt(6, 11))
    assert np.isfinite(out).all()


@pytest.mark.parametrize("change,msg", [({"linear_num_value_heads": 8}, "linear_num_key_heads"),
                                        ({"layer_types": ["full_attention"] + ["linear_attention"] * 3},
                                         "layer_types"),
                                        ({"hidden_act": "gelu"}, "silu")])
def test_unsupported_architectures_are_rejected(change, msg):
    hf = dict(hf_tiny.TINY, num_hidden_layers=4)
    hf.update(change)
    with pytest.raises(ValueError, match=msg):
        C.engine_config(hf)
