"""weights.bin / index.json writer and the seeded synthetic model tooling (CPU).

The first two tests are the reference's own converter checks (tests/test_conversion.py:13-30 in the
reference: 256-byte alignment with content dedup, and the query/gate head order)."""
import ctypes
import json
import math

import numpy as np
import pytest

import weights as W


def test_shared_weights_and_alignment(tmp_path):
    writer = W.Writer(tmp_path / "weights.bin")
    original = np.arange(16, dtype=np.uint8)
    writer.add("embed", original, "q4")
    writer.add("head", original.copy(), "q4")
    writer.add("other", original + 1, "q4")
    writer.close()
    assert writer.index["embed"] == writer.index["head"]
    assert writer.index["other"]["offset"] == 256
    data = (tmp_path / "weights.bin").read_bytes()
    assert data[:16] == original.tobytes()
    assert data[256:] == (original + 1).tobytes()


def test_query_and_gate_head_order():
    data = np.arange(8).reshape(8, 1)
    result = W.split_query_gate_rows((data, data, data), 2, 2)
    assert result[0].ravel().tolist() == [0, 1, 4, 5, 2, 3, 6, 7]


def splitmix_normals(seed, stream, n):
    """Pure-Python statement of the generator documented in csrc/synth.cpp."""
    M = 0xFFFFFFFFFFFFFFFF

    def mix(x):
        x = (x + 0x9E3779B97F4A7C15) & M
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M
        return x ^ (x >> 31)

    key = mix(seed ^ mix(stream))
    out = []
    for p in range((n + 1) // 2):
        a, b = mix((key + 2 * p) & M), mix((key + 2 * p + 1) & M)
        u1 = ((a >> 11) + 1) * 2.0 ** -53
        u2 = (b >> 11) * 2.0 ** -53
        r = math.sqrt(-2.0 * math.log(u1))
        out += [r * math.cos(2 * math.pi * u2), r * math.sin(2 * math.pi * u2)]
    return np.array(out[:n])


def test_generator_known_answer_and_statistics(qne):
    lib = qne.load_library()
    got = np.empty(9, dtype=np.float32)
    lib.qne_synth_normal_f32(123, 456, 9, ctypes.c_float(1.0), got.ctypes.data_as(ctypes.c_void_p))
    np.testing.assert_allclose(got, splitmix_normals(123, 456, 9).astype(np.float32), rtol=1e-6, atol=1e-7)
    big = np.empty(1 << 20, dtype=np.float32)
    lib.qne_synth_normal_f32(7, 1, big.size, ctypes.c_float(0.02), big.ctypes.data_as(ctypes.c_void_p))
    assert abs(big.mean()) < 1e-4 and abs(big.std() - 0.02) < 1e-4
    other = np.empty(1 << 20, dtype=np.float32)
    lib.qne_synth_normal_f32(7, 2, other.size, ctypes.c_float(0.02), other.ctypes.data_as(ctypes.c_void_p))
    assert abs(np.corrcoef(big, other)[0, 1]) < 5e-3
    h = np.empty(1000, dtype=np.uint16)
    lib.qne_synth_normal_f16(7, 1, h.size, ctypes.c_float(0.02), h.ctypes.data_as(ctypes.c_void_p))
    np.testing.assert_array_equal(h.view(np.float16), big[:1000].astype(np.float16))


def test_quantiser_bounds(qne):
    lib = qne.load_library()
    rng = np.random.default_rng(0)
    rows, k, g = 16, 512, 64
    w = rng.normal(0, 0.02, size=(rows, k)).astype(np.float32)
    w[3, :64] = 0.5  # constant group
    q = np.zeros(rows * k // 8, dtype=np.uint32)
    s = np.zeros(rows * k // g, dtype=np.uint16)
    z = np.zeros(rows * k // g, dtype=np.uint16)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.qne_quantize_q4g(P(w), rows, k, g, P(q), P(s), P(z)) == 0
    nib = ((q.reshape(rows, k // 8)[:, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15).reshape(rows, k)
    sf = np.repeat(s.view(np.float16).astype(np.float32).reshape(rows, -1), g, 1)
    zf = np.repeat(z.view(np.float16).astype(np.float32).reshape(rows, -1), g, 1)
    deq = (nib - zf) * sf
    err = np.abs(deq - w)
    # within half a step, plus the f16 rounding of the scale and zero
    assert np.all(err <= 0.5 * sf + 2e-3 * np.abs(w) + 1e-3 * sf)
    # each non-constant group spans the 4-bit range: its minimum maps near 0, its maximum near 15
    grp = nib.reshape(rows, k // g, g)
    assert np.all(grp.min(axis=2)[np.arange(rows) != 3] <= 1) and np.all(grp.max(axis=2)[np.arange(rows) != 3] >= 14)
    assert abs(deq[3, 0] - 0.5) < 1e-3


def test_plan_is_aligned_and_matches_shapes():
    cfg = W.full_config("2b")
    lay, mats = W.plan(cfg, body="q4", head="f16")
    for name, t in lay.tensors.items():
        assert t["offset"] % 256 == 0
    assert mats["lm_head"]["dtype"] == "f16" and mats["layer0.mixer_in"]["dtype"] == "q4"
    assert mats["layer3.mixer_in"]["rows"] == 2 * 16 * 256 + 2 * 4 * 256  # q, gate, k, v
    assert mats["layer0.mixer_in"]["rows"] == 8224
    assert mats["layer3.mixer_out"]["k"] == 4096 and mats["layer0.mixer_out"]["k"] == 2048
    # int4 body bytes = elements * (1/2 + 2 * 2/64)
    body = sum(r * k for n, (r, k) in W.matrix_shapes(cfg).items() if n not in ("embed", "lm_head"))
    assert body == 1_704_263_680
    ix = json.loads(W.index_json(cfg, lay, mats, "t"))
    assert ix["format_version"] == 2 and ix["config"]["n_kv_heads"] == 4


def test_synth_model_is_deterministic(qne):
    a_ix, a = W.synth_model("tiny", seed=3)
    b_ix, b = W.synth_model("tiny", seed=3)
    c_ix, c = W.synth_model("tiny", seed=4)
    assert a_ix == b_ix and np.array_equal(a, b)
    assert not np.array_equal(a, c)
