"""Pins the CPU oracle before it is trusted as the checker.

The reference stores no golden vectors for this path (its kernel checks regenerate inputs from an
xorshift seed and record only errors, kernels/src/lib.rs:513-712). Each oracle function is pinned
here by something other than its own formula: known-answer packings, library routines (numpy,
torch), closed forms and special cases chosen so that a dropped term, a swapped index or a
transposed operand fails.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import cpu_oracle as O
from torch_ref import TorchModel

L64 = lambda: O.lib("f64")
L32 = lambda: O.lib("f32")


def f16(a):
    return np.asarray(a, dtype=np.float16)


# ---------------------------------------------------------------- f16 conversion

@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_f16_decode_matches_numpy_for_every_bit_pattern(prec):
    L = O.lib(prec)
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.oc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_f16_encode_rounds_like_numpy():
    L = L32()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000), rng.normal(0, 3e4, 2000),
                           [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                            np.inf, -np.inf]]).astype(np.float32)
    # exact ties between two halves
    base = rng.normal(0, 1, 2000).astype(np.float16).astype(np.float32)
    vals = np.concatenate([vals, base + np.spacing(base.astype(np.float16)).astype(np.float32) / 2])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.oc_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- dequantisation (known answers)

def pack_nibbles(q):
    """Independent packing: value c goes to bits 4*(c%8) of word c/8 (little-endian bytes, low
    nibble first, the ONNX MatMulNBits order)."""
    rows, k = q.shape
    b = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(b).view(np.uint32).reshape(rows, k // 8)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_dequant_q4_group_f16_zero_known_answer(group):
    rng = np.random.default_rng(group)
    rows, k = 5, 512
    q = rng.integers(0, 16, size=(rows, k), dtype=np.uint32)
    s = f16(rng.choice([0.25, 0.5, 0.015625, 1.5, 0.0234375], size=(rows, k // group)))
    z = f16(rng.choice([0.0, 7.5, 8.0, 3.25, 15.0], size=(rows, k // group)))
    want = (q.astype(np.float32) - np.repeat(z.astype(np.float32), group, 1)) * np.repeat(s.astype(np.float32), group, 1)
    w = pack_nibbles(q)
    m = O.mat_struct(None, O.OC_Q4G, rows, k, group, w, s.view(np.uint16), z.view(np.uint16))
    out = np.empty(k, dtype=np.float32)
    for r in range(rows):
        L64().oc_dequant_row(ctypes.byref(m), r, O.ptr(out))
        assert np.array_equal(out, want[r])


def test_dequant_reference_matmulnbits_layout_known_answer():
    """Reference layout (kernels/src/lib.rs:484-497): block 32, scales as two f16 per u32,
    zero points as eight u4 per u32 word."""
    rng = np.random.default_rng(7)
    rows, k = 3, 1024
    q = rng.integers(0, 16, size=(rows, k), dtype=np.uint32)
    zp = rng.integers(0, 16, size=(rows, k // 32), dtype=np.uint32)
    s = f16(rng.choice([0.02, 0.5, 0.125], size=(rows, k // 32)))
    zwords = np.zeros((rows, k // 256), dtype=np.uint32)
    for r in range(rows):
        for b in range(k // 32):
            zwords[r, b // 8] |= np.uint32(zp[r, b] << (4 * (b % 8)))
    want = (q.astype(np.float32) - np.repeat(zp.astype(np.float32), 32, 1)) * np.repeat(s.astype(np.float32), 32, 1)
    w = pack_nibbles(q)
    sw = np.ascontiguousarray(s).view(np.uint32)  # two halves per word, block b in half b&1
    m = O.mat_struct(None, O.OC_Q4V1, rows, k, 32, w, sw, zwords)
    out = np.empty(k, dtype=np.float32)
    for r in range(rows):
        L64().oc_dequant_row(ctypes.byref(m), r, O.ptr(out))
        assert np.array_equal(out, want[r])


# ---------------------------------------------------------------- GEMV epilogues vs numpy

def dequant_all(m):
    rows, k = m.rows, m.k
    out = np.empty((rows, k), dtype=np.float32)
    for r in range(rows):
        L64().oc_dequant_row(ctypes.byref(m), r, O.ptr(out[r]))
    return out.astype(np.float64)


@pytest.mark.parametrize("prec,tol", [("f64", 2e-7), ("f32", 2e-6)])  # outputs are stored as f32
@pytest.mark.parametrize("epi", [O.STORE, O.ACCUMULATE, O.SWIGLU])
def test_gemv_epilogues_match_numpy(prec, tol, epi):
    rng = np.random.default_rng(3 + epi)
    rows, k = 74, 1024
    q = rng.integers(0, 16, size=(rows, k), dtype=np.uint32)
    s = f16(rng.uniform(0.001, 0.03, size=(rows, k // 64)))
    z = f16(rng.uniform(0, 15, size=(rows, k // 64)))
    m = O.mat_struct(None, O.OC_Q4G, rows, k, 64, pack_nibbles(q), s.view(np.uint16), z.view(np.uint16))
    W = dequant_all(m)
    x = rng.normal(size=k).astype(np.float32)
    out_rows = rows // 2 if epi == O.SWIGLU else rows
    y0 = rng.normal(size=out_rows).astype(np.float32)
    y = y0.copy()
    O.lib(prec).oc_gemv(ctypes.byref(m), O.ptr(x), O.ptr(y), epi)
    wx = W @ x.astype(np.float64)
    if epi == O.STORE:
        want = wx
    elif epi == O.ACCUMULATE:
        want = y0 + wx
    else:
        want = F.silu(torch.from_numpy(wx[:out_rows])).numpy() * wx[out_rows:]
    assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < tol


def test_gemv_f16_matches_numpy():
    rng = np.random.default_rng(11)
    w = f16(rng.normal(0, 0.02, size=(33, 512)))
    m = O.mat_struct(None, O.OC_F16, 33, 512, 0, w.view(np.uint16))
    x = rng.normal(size=512).astype(np.float32)
    y = np.zeros(33, dtype=np.float32)
    L64().oc_gemv(ctypes.byref(m), O.ptr(x), O.ptr(y), O.STORE)
    want = w.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y, want, rtol=1e-6, atol=1e-7)


def test_rmsnorm_matches_torch():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, size=2048).astype(np.float32)
    g = rng.normal(1, 0.1, size=2048).astype(np.float32)
    y = np.empty_like(x)
    L64().oc_rmsnorm(O.ptr(x), O.ptr(g), O.ptr(y), 2048, 1e-6)
    want = F.rms_norm(torch.from_numpy(x).double(), (2048,), weight=torch.from_numpy(g).double(), eps=1e-6).numpy()
    assert np.allclose(y, want, rtol=1e-6, atol=1e-7)


def test_argmax_planted_maximum_and_ties():
    """The reference's known answer: a planted maximum at 123457 (kernels/src/lib.rs:684-710)."""
    rng = np.random.default_rng(0)
    v = rng.uniform(-1, 1, size=248320).astype(np.float32)
    v[123457] = 9.0
    idx, val = ctypes.c_uint32(), ctypes.c_float()
    L32().oc_argmax(O.ptr(v), v.size, ctypes.byref(idx), ctypes.byref(val))
    assert idx.value == 123457 and val.value == 9.0
    v[200000] = 9.0  # tie: the lower index wins
    v[5] = np.nan
    L32().oc_argmax(O.ptr(v), v.size, ctypes.byref(idx), ctypes.byref(val))
    assert idx.value == 123457


# ---------------------------------------------------------------- Gated DeltaNet

def test_delta_rule_matches_matrix_form():
    rng = np.random.default_rng(9)
    dk = dv = 128
    S0 = rng.normal(0, 0.1, size=(dk, dv)).astype(np.float32)
    q = rng.normal(size=dk).astype(np.float32)
    k = rng.normal(size=dk).astype(np.float32)
    k /= np.linalg.norm(k)
    v = rng.normal(size=dv).astype(np.float32)
    beta, g = 0.7, 0.9
    S = S0.copy()
    out = np.empty(dv, dtype=np.float32)
    L64().oc_delta_rule(dk, dv, O.ptr(q), O.ptr(k), O.ptr(v), beta, g, O.ptr(S), O.ptr(out))
    kk = k.astype(np.float64)[:, None]
    Sw = g * (np.eye(dk) - beta * kk @ kk.T) @ S0.astype(np.float64) + beta * kk @ v.astype(np.float64)[None, :]
    np.testing.assert_allclose(S, Sw, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(out, Sw.T @ q.astype(np.float64), rtol=1e-6, atol=1e-6)


def test_delta_rule_beta_zero_is_pure_decay():
    rng = np.random.default_rng(10)
    S0 = rng.normal(size=(128, 128)).astype(np.float32)
    q, k, v = (rng.normal(size=128).astype(np.float32) for _ in range(3))
    S = S0.copy()
    out = np.empty(128, dtype=np.float32)
    L64().oc_delta_rule(128, 128, O.ptr(q), O.ptr(k), O.ptr(v), 0.0, 0.5, O.ptr(S), O.ptr(out))
    np.testing.assert_array_equal(S, (0.5 * S0.astype(np.float64)).astype(np.float32))
    np.testing.assert_allclose(out, 0.5 * S0.astype(np.float64).T @ q.astype(np.float64), rtol=1e-6, atol=1e-6)


def test_delta_rule_associative_recall_with_orthonormal_keys():
    """g = 1, beta = 1: writing value v_i under orthonormal key k_i and reading with q = k_j
    returns v_j."""
    rng = np.random.default_rng(12)
    Kq, _ = np.linalg.qr(rng.normal(size=(128, 128)))
    vals = rng.normal(size=(16, 128)).astype(np.float32)
    S = np.zeros((128, 128), dtype=np.float32)
    out = np.empty(128, dtype=np.float32)
    for i in range(16):
        k = Kq[:, i].astype(np.float32)
        L64().oc_delta_rule(128, 128, O.ptr(k), O.ptr(k), O.ptr(vals[i]), 1.0, 1.0, O.ptr(S), O.ptr(out))
        np.testing.assert_allclose(out, vals[i], atol=1e-5)
    for j in range(16):
        k = Kq[:, j].astype(np.float32)
        zero = np.zeros(128, dtype=np.float32)
        L64().oc_delta_rule(128, 128, O.ptr(k), O.ptr(k), O.ptr(zero), 0.0, 1.0, O.ptr(S), O.ptr(out))
        np.testing.assert_allclose(out, vals[j], atol=1e-5)


def small_cfg(**kw):
    c = dict(hidden=512, layers=4, full_attention_every=4, intermediate=1024, vocab=256, n_q_heads=4, n_kv_heads=2,
             head_dim=256, rope_dim=64, gdn_heads=2, gdn_dk=128, gdn_dv=128, conv_kernel=4, rope_theta=1e7,
             rms_eps=1e-6)
    c.update(kw)
    return c


def test_gdn_step_matches_torch_formulation():
    cfg = small_cfg()
    C = O.config_struct(cfg)
    rng = np.random.default_rng(21)
    H, dk, dv = 2, 128, 128
    ch = 2 * H * dk + H * dv
    proj = rng.normal(size=2 * H * dk + 2 * H * dv + 2 * H).astype(np.float32)
    conv = rng.normal(size=(ch, 3)).astype(np.float32)
    cw = rng.normal(0, 0.5, size=(ch, 4)).astype(np.float32)
    S0 = rng.normal(0, 0.1, size=(H, dk, dv)).astype(np.float32)
    prm = np.concatenate([rng.normal(0, 1, H), -rng.uniform(0.1, 1, H), rng.normal(1, 0.2, dv)]).astype(np.float32)
    conv_g, S = conv.copy(), S0.copy()
    o = np.empty(H * dv, dtype=np.float32)
    L64().oc_gdn_step(ctypes.byref(C), O.ptr(proj), O.ptr(conv_g), O.ptr(cw), O.ptr(S), O.ptr(o), O.ptr(prm))
    # independent formulation (torch_ref.TorchModel.gdn) on the same inputs
    tm = TorchModel.__new__(TorchModel)
    tm.c = cfg
    tm.V = {"layer0.conv_w": torch.from_numpy(cw.reshape(-1)).double(), "layer0.gdn_params": torch.from_numpy(prm).double()}
    tm.conv = {0: torch.from_numpy(conv).double()}
    tm.S = {0: torch.from_numpy(S0).double()}
    want = tm.gdn(0, torch.from_numpy(proj).double()).numpy()
    np.testing.assert_allclose(o, want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(S, tm.S[0].numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(conv_g, tm.conv[0].numpy(), rtol=0, atol=0)


# ---------------------------------------------------------------- attention

def attn_inputs(cfg, pos, seed):
    rng = np.random.default_rng(seed)
    nq, nkv, hd = cfg["n_q_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    proj = rng.normal(size=2 * nq * hd + 2 * nkv * hd).astype(np.float32)
    kc = np.zeros((nkv, 4096, hd), dtype=np.float16)
    vc = np.zeros((nkv, 4096, hd), dtype=np.float16)
    kc[:, :pos] = rng.normal(size=(nkv, pos, hd))
    vc[:, :pos] = rng.normal(size=(nkv, pos, hd))
    prm = rng.normal(1, 0.3, size=2 * hd).astype(np.float32)
    return proj, kc, vc, prm


@pytest.mark.parametrize("pos", [0, 5, 300, 4095])
def test_attention_step_matches_sdpa(pos):
    cfg = small_cfg()
    C = O.config_struct(cfg)
    nq, nkv, hd = 4, 2, 256
    proj, kc, vc, prm = attn_inputs(cfg, pos, 30 + pos)
    o = np.empty(nq * hd, dtype=np.float32)
    kc_g, vc_g = kc.copy(), vc.copy()
    L64().oc_attention_step(ctypes.byref(C), O.ptr(proj), O.ptr(kc_g.view(np.uint16)), O.ptr(vc_g.view(np.uint16)),
                            pos, O.ptr(o), O.ptr(prm))
    tm = TorchModel.__new__(TorchModel)
    tm.c = cfg
    tm.V = {"layer3.attn_norms": torch.from_numpy(prm).double()}
    tm.K = {3: [torch.from_numpy(kc[:, l].astype(np.float64)) for l in range(pos)]}
    tm.Vc = {3: [torch.from_numpy(vc[:, l].astype(np.float64)) for l in range(pos)]}
    want = tm.attention(3, torch.from_numpy(proj).double(), pos).numpy()
    np.testing.assert_allclose(o, want, rtol=1e-5, atol=1e-6)
    # the appended slot holds the f16 rounding of the normed, rotated key and of the value
    np.testing.assert_array_equal(kc_g[:, pos].astype(np.float64), tm.K[3][-1].numpy())
    np.testing.assert_array_equal(vc_g[:, pos].astype(np.float64), tm.Vc[3][-1].numpy())
    assert np.array_equal(kc_g[:, :pos], kc[:, :pos]) and np.array_equal(kc_g[:, pos + 1:], kc[:, pos + 1:])


def test_attention_first_position_returns_gated_value():
    """pos = 0: softmax over one key, so o = f16(v) * sigmoid(gate) for every head of the group."""
    cfg = small_cfg()
    C = O.config_struct(cfg)
    proj, kc, vc, prm = attn_inputs(cfg, 0, 77)
    o = np.empty(4 * 256, dtype=np.float32)
    L64().oc_attention_step(ctypes.byref(C), O.ptr(proj), O.ptr(kc.view(np.uint16)), O.ptr(vc.view(np.uint16)), 0,
                            O.ptr(o), O.ptr(prm))
    v = proj[2 * 4 * 256 + 2 * 256:].reshape(2, 256).astype(np.float16).astype(np.float64)
    gate = proj[4 * 256: 8 * 256].reshape(4, 256).astype(np.float64)
    want = np.repeat(v, 2, axis=0) / (1 + np.exp(-gate))
    np.testing.assert_allclose(o.reshape(4, 256), want, rtol=2e-7, atol=1e-9)  # f32 output rounding


def test_attention_rope_preserves_norms_and_uniform_keys_average_values():
    rng = np.random.default_rng(4)
    nq, nkv, hd, n = 4, 2, 256, 37
    k = np.repeat(rng.normal(size=(nkv, 1, hd)), n, axis=1).astype(np.float16)
    v = rng.normal(size=(nkv, n, hd)).astype(np.float16)
    q = rng.normal(size=(nq, hd)).astype(np.float32)
    out = np.empty(nq * hd, dtype=np.float32)
    L64().oc_attn_dense(nq, nkv, hd, O.ptr(q), O.ptr(k.view(np.uint16)), O.ptr(v.view(np.uint16)), n, 0.0625, O.ptr(out))
    want = np.repeat(v.astype(np.float64).mean(axis=1), 2, axis=0)
    np.testing.assert_allclose(out.reshape(nq, hd), want, rtol=2e-7, atol=1e-9)  # f32 output rounding
    # RoPE is a rotation: the norm of a rotated key is the norm of the normed key
    tm = TorchModel.__new__(TorchModel)
    tm.c = small_cfg()
    x = torch.from_numpy(rng.normal(size=hd))
    for pos in (1, 1000, 4095):
        assert abs(float(tm.rope(x, pos).norm() - x.norm())) < 1e-12


def test_attn_dense_matches_sdpa():
    rng = np.random.default_rng(8)
    nq, nkv, hd, n = 8, 2, 256, 129
    k = rng.normal(size=(nkv, n, hd)).astype(np.float16)
    v = rng.normal(size=(nkv, n, hd)).astype(np.float16)
    q = rng.normal(size=(nq, hd)).astype(np.float32)
    out = np.empty(nq * hd, dtype=np.float32)
    L64().oc_attn_dense(nq, nkv, hd, O.ptr(q), O.ptr(k.view(np.uint16)), O.ptr(v.view(np.uint16)), n, 0.0625, O.ptr(out))
    K = torch.from_numpy(k.astype(np.float64)).repeat_interleave(4, 0)
    V = torch.from_numpy(v.astype(np.float64)).repeat_interleave(4, 0)
    want = F.scaled_dot_product_attention(torch.from_numpy(q).double()[:, None], K, V, scale=0.0625)[:, 0]
    np.testing.assert_allclose(out.reshape(nq, hd), want.numpy(), rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------- whole model

@pytest.fixture(scope="module")
def tiny_model():
    import weights as W
    return W.synth_model("tiny", seed=5, body="q4", head="f16", norm_jitter=0.1)


def test_model_graph_matches_torch_formulation(tiny_model):
    index, buf = tiny_model
    om = O.OracleModel(index, buf, "f64")
    tm = TorchModel(index, buf)
    for pos, tok in enumerate([17, 4000, 3, 999, 2048, 1]):
        a = om.token(tok, pos)
        b = tm.token(tok, pos)
        assert np.max(np.abs(a - b)) < 1e-5 * max(1.0, np.max(np.abs(b))), pos


def test_model_f32_oracle_tracks_f64(tiny_model):
    index, buf = tiny_model
    a, b = O.OracleModel(index, buf, "f64"), O.OracleModel(index, buf, "f32")
    for pos, tok in enumerate([1, 2, 3, 4, 5]):
        la, lb = a.token(tok, pos), b.token(tok, pos)
        assert np.max(np.abs(la - lb)) < 1e-4


@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("body", ["q4", "f16"])
def test_layered_prefill_is_bitwise_token_by_token(prec, body):
    """oc_prefill_chunk runs a prompt layer by layer (each projection over all tokens at once); every
    token must see exactly oc_token's arithmetic, so the state and the logits after the prompt are
    bitwise those of feeding the tokens one at a time (model.rs:337-338 asks for the same state).
    70 tokens span two full 32-token blocks of the projections and a ragged one, and the prompt is
    split into two calls so a non-zero start is covered."""
    import weights as W
    index, buf = W.synth_model("tiny", seed=9, body=body, head="f16", norm_jitter=0.1)
    ids = np.random.default_rng(3).integers(0, 4096, size=70).astype(np.uint32)
    a, b = O.OracleModel(index, buf, prec, max_context=128), O.OracleModel(index, buf, prec, max_context=128)
    for pos, t in enumerate(ids[:-1]):
        a.token(int(t), pos, want_logits=False)
    want = a.token(int(ids[-1]), len(ids) - 1)
    b.prefill_chunk(ids[:45], 0, False)
    got = b.prefill_chunk(ids[45:], 45, True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert a.state_bytes() == b.state_bytes()
