"""The Model API (include/qne.h, mirroring kernels/src/model.rs) on the GPU against the oracle.

Bar (BASELINE parity target): max |logit error| <= 1e-2 and identical greedy ids; the kernels are
f32-accumulating, so the logits are expected far closer than that (checked at 1e-3 here)."""
import json

import numpy as np
import pytest

import cpu_oracle as O
import qne as Q
import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=[("tiny", "q4", "f16", "persistent"), ("tiny", "f16", "q4", "persistent"),
                                        ("small", "q4", "f16", "persistent"), ("tiny", "q4", "f16", "graph"),
                                        ("small", "q4", "f16", "graph")],
                ids=["tiny-q4body", "tiny-f16body-q4head", "small-q4body", "tiny-q4body-graph", "small-q4body-graph"])
def pair(request):
    name, body, head, engine = request.param
    index, buf = W.synth_model(name, seed=11, body=body, head=head, norm_jitter=0.1)
    m = Q.Model.load(index, buf, options={"engine": engine})
    om = O.OracleModel(index, buf, "f64")
    yield name, m, om, index, buf
    m.close()


def prompt(vocab, n, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.uint32)


def test_prefill_logits_and_greedy_decode(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 40, 1)
    m.reset()
    om.reset()
    m.prefill_batched(ids)
    want = om.prefill_chunk(ids, 0, True)
    got = m.logits()
    assert np.max(np.abs(got - want)) < 1e-3
    first, pos = m.last_token()
    assert first == int(np.argmax(want)) and pos == len(ids)
    steps = 64
    out = m.decode(steps, 1, [])
    om.reset()
    want_ids, want_logits = om.greedy(ids, steps)
    assert out == want_ids


MAX = 0xFFFFFFFF


def test_decode_window_returns_every_id(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 9, 2)
    m.reset()
    m.prefill_batched(ids)
    w1 = m.decode(20, 1, [])
    m.reset()
    m.prefill_batched(ids)
    w8 = m.decode_ids(20, 8, [])
    assert w1 == w8 and len(w8) == 20
    ms, steps = m.last_decode_timing()  # windows of 8, 8 and 3 steps after the pending id
    assert steps == 19 and ms > 0.0


def test_decode_windows_push_placeholders_like_the_reference(pair):
    """Model::decode (model.rs:426-449): a window of s > 1 steps pushes s u32::MAX values, a one-step
    window pushes its pick, and `stop` is only checked against the last value pushed."""
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 9, 2)
    m.reset()
    m.prefill_batched(ids)
    w1 = m.decode(20, 1, [])
    m.reset()
    m.prefill_batched(ids)
    # n = 20, window 8: [first], 8 placeholders, 8 placeholders, then a 3-step window
    assert m.decode(20, 8, []) == [w1[0]] + [MAX] * 19
    assert m.last_token() == (w1[19], len(ids) + 19)
    m.reset()
    m.prefill_batched(ids)
    # n = 10, window 8: [first], 8 placeholders, then a one-step window that returns its pick
    assert m.decode(10, 8, []) == [w1[0]] + [MAX] * 8 + [w1[9]]
    m.reset()
    m.prefill_batched(ids)
    # a stop id inside a window is not seen (the window returns placeholders)
    assert m.decode(20, 8, [w1[3]]) == [w1[0]] + [MAX] * 19
    m.reset()
    m.prefill_batched(ids)
    # the first id is checked before any window runs
    assert m.decode(20, 8, [w1[0]]) == [w1[0]]
    assert m.last_token() == (w1[0], len(ids))


def test_decode_is_bitwise_repeatable(pair):
    """Every reduction runs in a fixed order, so two runs from the same state agree bit for bit: a
    race on shared staging buffers or on the hand-over between phases shows up here."""
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 33, 5)
    runs = []
    for _ in range(2):
        m.reset()
        m.prefill_batched(ids)
        first = m.logits()
        out = m.decode_ids(24, 8, [])
        tok, pos = m.last_token()
        runs.append((first, out, m.step(tok, pos)))
    assert np.array_equal(runs[0][0], runs[1][0])
    assert runs[0][1] == runs[1][1]
    assert np.array_equal(runs[0][2], runs[1][2])


def test_decode_stops_at_stop_token(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 7, 3)
    m.reset()
    m.prefill_batched(ids)
    full = m.decode(12, 1, [])
    stop = full[5]
    m.reset()
    m.prefill_batched(ids)
    cut = m.decode(12, 1, [stop])
    assert cut == full[: full.index(stop) + 1]


def test_step_returns_logits_and_leaves_the_greedy_pick(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 12, 4)
    m.reset()
    om.reset()
    m.prefill_batched(ids)
    om.prefill_chunk(ids, 0, True)
    got = m.step(5, len(ids))
    want = om.token(5, len(ids))
    assert np.max(np.abs(got - want)) < 1e-3
    assert m.last_token() == (5, len(ids))  # step does not run the device argmax (model.rs:386-387)


def test_token_prefill_equals_chunked_prefill(pair):
    """prefill (token by token) and prefill_chunk (the batched GEMM path) leave the same state
    (model.rs:337-338): the same math in a different summation order, so to f32 rounding."""
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 33, 5)
    m.reset()
    m.prefill(ids)
    a = m.logits()
    ta = m.last_token()
    m.reset()
    m.prefill_chunk(ids[:20], 0, False)
    m.prefill_chunk(ids[20:], 20, True)
    b = m.logits()
    assert np.max(np.abs(a - b)) < 1e-4 and ta == m.last_token()
    # and the state continues alike: one decode step from each
    m.reset()
    m.prefill(ids)
    s1 = m.step(*m.last_token())
    m.reset()
    m.prefill_chunk(ids, 0, True)
    s2 = m.step(*m.last_token())
    assert np.max(np.abs(s1 - s2)) < 1e-4


def test_chunked_prefill_does_not_depend_on_the_chunking(pair):
    """A token's result in the batched prefill depends only on its own row (the GEMMs' split counts
    and the attention splits are fixed for the model) and on the recurrent state, and the GDN
    recurrence runs every 64-position block in one form (WY when the call holds the whole block,
    else sequential): calls cut at multiples of 64 positions give the same bits, across the 512-token
    passes too; any other cut runs some blocks in the other form, the same math to f32 rounding."""
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 600, 9)
    m.reset()
    m.prefill_chunk(ids, 0, True)
    a, ta = m.logits(), m.last_token()
    m.reset()
    m.prefill_chunk(ids[:64], 0, False)
    m.prefill_chunk(ids[64:576], 64, False)
    m.prefill_chunk(ids[576:], 576, True)
    assert np.array_equal(a, m.logits()) and ta == m.last_token()
    m.reset()
    m.prefill_chunk(ids[:7], 0, False)
    m.prefill_chunk(ids[7:71], 7, False)
    m.prefill_chunk(ids[71:], 71, True)
    assert np.max(np.abs(a - m.logits())) < 1e-4 and ta == m.last_token()


def test_chunked_prefill_matches_oracle_over_many_chunks(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 1100, 12)  # one pass (passes hold up to 2048 tokens)
    m.reset()
    om.reset()
    m.prefill_batched(ids)
    want = om.prefill_chunk(ids, 0, True)
    assert np.max(np.abs(m.logits() - want)) < 1e-3
    assert m.last_token() == (int(np.argmax(want)), len(ids))


def test_chunked_prefill_in_several_passes_matches_oracle():
    """A pass holds min(2048, max_context rounded up to 64) tokens: a 2200-id prompt in one call runs
    as passes of 2048 and 152 tokens, and split into calls at 1024 (a multiple of 64: the GDN blocks
    line up) as 1024 + 1024 + 152."""
    index, buf = W.synth_model("tiny", seed=11, body="q4", head="f16", norm_jitter=0.1)
    om = O.OracleModel(index, buf, "f64")
    ids = prompt(json.loads(index)["config"]["vocab"], 2200, 13)
    want = om.prefill_chunk(ids, 0, True)
    with Q.Model.load(index, buf) as m:
        m.prefill_chunk(ids, 0, True)
        a = m.logits()
        assert np.max(np.abs(a - want)) < 1e-3 and m.last_token() == (int(np.argmax(want)), len(ids))
        m.reset()
        m.prefill_chunk(ids[:1024], 0, False)
        m.prefill_chunk(ids[1024:], 1024, True)
        # the same rows in other passes: the same bits (split counts are fixed per model)
        assert np.array_equal(m.logits(), a)


def test_prefill_gemm_epilogues_equal_the_reduce_pass():
    """With hidden 2048 and a 2048-token pass every prefill GEMM has one split, so gate_up applies
    the SwiGLU and the out- and down-projections the residual add, each staging the next GEMM's
    operand, inside the GEMM; {"gemm_fusion": false} runs the reduce pass after each of them
    instead. Both compute the same arithmetic in the same order: the logits after a 2100-id prompt
    (passes of 2048 and 52 tokens) and after a further 1-id call are identical bit for bit."""
    cfg = dict(layers=4, full_attention_every=4, hidden=2048, intermediate=2048, vocab=4096, n_q_heads=8,
               n_kv_heads=2, head_dim=256, gdn_heads=16)
    index, buf = W.synth_model(cfg, seed=23, body="q4", head="f16", norm_jitter=0.1)
    ids = prompt(cfg["vocab"], 2101, 17)
    runs = []
    for fusion in (True, False):
        with Q.Model.load(index, buf, options={"gemm_fusion": fusion}) as m:
            m.prefill_chunk(ids[:2100], 0, True)
            a = m.logits()
            m.prefill_chunk(ids[2100:], 2100, True)
            runs.append(np.stack([a, m.logits()]))
    assert np.all(np.isfinite(runs[0]))
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32)), float(np.max(np.abs(runs[0] - runs[1])))


def test_snapshot_restore_and_reset(pair):
    name, m, om, _, _ = pair
    ids = prompt(m.vocab, 16, 6)
    with pytest.raises(Q.QneError) as e:
        Q.Model.load(*W.synth_model("tiny", seed=1)).restore()
    assert e.value.code == Q.ENOSNAPSHOT and str(e.value) == "no snapshot taken"
    m.reset()
    m.prefill_batched(ids[:8])
    m.snapshot()
    m.prefill_from(ids[8:], 8)
    a = m.logits()
    m.restore()
    m.prefill_from(ids[8:], 8)
    assert np.array_equal(a, m.logits())
    m.reset()
    m.prefill_batched(ids)
    assert np.array_equal(a, m.logits())


def test_context_limits(pair):
    name, m, om, _, _ = pair
    with pytest.raises(Q.QneError) as e:
        m.step(1, m.max_context)
    assert e.value.code == Q.ECONTEXT
    with pytest.raises(Q.QneError) as e:
        m.prefill_chunk([1, 2], m.max_context - 2, True)
    assert e.value.code == Q.ECONTEXT
    with pytest.raises(Q.QneError) as e:
        m.prefill([])
    assert e.value.code == Q.EINVAL
    assert m.max_context == 4096 and m.dispatches_per_token() > 0 and "gfx" in m.adapter


def test_small_context_capacity_and_decode_guard():
    index, buf = W.synth_model("tiny", seed=2)
    m = Q.Model.load(index, buf, options={"max_context": 32})
    assert m.max_context == 32
    m.prefill_batched(list(range(30)))
    with pytest.raises(Q.QneError) as e:
        m.decode(5, 1, [])
    assert e.value.code == Q.ECONTEXT and "context limit" in str(e.value)
    m.close()


def test_reference_format1_model_loads_and_matches():
    """A format-1 file (the reference's q4 block-32 u4-zero layout at Qwen3.5-0.8B shapes)."""
    import json
    cfg = W.full_config(dict(W.CONFIGS["0.8b"], vocab=248320))
    # build format-1 tensors: q4 g32 with u4 zero points for every matrix
    lay, mats = W.plan(cfg, body="q4", head="q4", group=32)
    rng = np.random.default_rng(0)
    buf = np.zeros(lay.size, dtype=np.uint8)
    tensors = {}
    for n, t in lay.tensors.items():
        tensors[n] = {"offset": t["offset"], "bytes": t["bytes"]}
    v1_tensors = {}
    for name, mm in mats.items():
        rows, k = mm["rows"], mm["k"]
        wv = lay.view(buf.data, name + ".w", np.uint32)
        wv[:] = rng.integers(0, 2 ** 32, size=wv.size, dtype=np.uint64).astype(np.uint32)
        sv = lay.view(buf.data, name + ".s", np.uint16)
        sv[:] = np.float16(0.02).view(np.uint16) + rng.integers(0, 64, size=sv.size).astype(np.uint16)
        # u4 zero points occupy the first rows * k / 64 bytes of the .z slot
        zt = dict(tensors[name + ".z"])
        zt["bytes"] = rows * k // 64
        zv = np.frombuffer(buf.data, dtype=np.uint8, count=zt["bytes"], offset=zt["offset"])
        zv[:] = rng.integers(0, 256, size=zv.size).astype(np.uint8)
        v1_tensors[name + ".z"] = zt
    for n, t in lay.tensors.items():
        if t["kind"] == "f32":
            v = lay.view(buf.data, n, np.float32)
            v[:] = 1.0 if "norm" in n else rng.normal(0, 0.02, size=v.size)
            if n.endswith("gdn_params"):
                v[:16], v[16:32], v[32:] = 0.0, -0.5, 1.0
    tensors.update(v1_tensors)
    index = json.dumps({"format_version": 1, "config": {"layers": 24, "full_attention_every": 4, "hidden": 1024,
                        "intermediate": 3584, "vocab": 248320, "rope_theta": 10000000.0, "rope_dim": 64},
                        "matrices": {n: {"rows": mm["rows"], "k": mm["k"]} for n, mm in mats.items()},
                        "tensors": tensors})
    m = Q.Model.load(index, buf)
    om = O.OracleModel(index, buf, "f32")
    ids = [1, 2, 3]
    m.prefill_batched(ids)
    want = om.prefill_chunk(ids, 0, True)
    assert np.max(np.abs(m.logits() - want)) < 1e-3 * max(1.0, np.max(np.abs(want)))
    m.close()


def test_profile_token_consumes_one_greedy_token_and_reports_every_phase(pair):
    """Model::profile_token (model.rs:305): one greedy token, timed. The profiled token is the one a
    plain greedy decode step takes from the same state, and the persistent engine's timeline names
    every phase of the token and where each workgroup ran."""
    name, m, om, index, _ = pair
    ids = prompt(m.vocab, 24, 5)
    m.reset()
    m.prefill_batched(ids)
    want = m.decode_ids(2, 1)  # the pending pick, then one greedy step from it
    m.reset()
    m.prefill_batched(ids)
    assert m.profile_token() > 0.0
    assert m.last_token() == (want[1], len(ids) + 1)
    m.reset()
    m.prefill_batched(ids)
    try:
        d = m.profile_token_detail()
    except Q.QneError as e:  # the graph engine has no device timeline
        assert e.code == Q.EINVAL
        return
    assert m.last_token() == (want[1], len(ids) + 1)
    cfg = json.loads(index)["config"]
    layers = cfg["layers"]
    attn = sum(1 for i in range(layers) if (i + 1) % cfg["full_attention_every"] == 0)
    # a GDN layer is 4 phases when its in-projection and step run fused ("gdn.mixer_in+gdn"), else 5;
    # an attention layer 5 when the combine of the partials runs in the attention phase, else 6
    fused = "gdn.mixer_in+gdn" in d["labels"]
    folded = "attn.attention+combine" in d["labels"]
    assert fused == (name == "small")  # 16 GDN heads and q4 rows: fused on a 256-workgroup grid
    assert folded  # every test model has splits >= 4 q heads per kv head
    assert len(d["phases"]) == (4 if fused else 5) * (layers - attn) + (5 if folded else 6) * attn + 1
    assert all(v >= 0.0 for v in d["labels"].values())
    phases = ("mixer_in", "gdn", "mixer_in+gdn", "attention", "attention+combine", "combine", "mixer_out", "gate_up",
              "down")
    assert set(d["labels"]) <= {f"{k}.{p}" for k in ("gdn", "attn") for p in phases} | {"lm_head"}
    places = d["places"]
    assert len(places) == len(d["input_ticks"][0]) and all(p is not None and p[0] >= 0 for p in places)
    assert d["total_ms"] > 0.0


@pytest.mark.parametrize("name", ["small", "2b"])
def test_fused_gdn_phase_equals_the_separate_phases(name):
    """The decode program's fused GDN phase (in-projection rows, head-group q/k exchange and the
    delta rule step in one phase) against the same model with the in-projection and the step as two
    phases ({"gdn_fusion": false}): every row and the state update run the same arithmetic, so the
    logits after the prompt and after each of 24 greedy steps, and the ids, are identical bit for
    bit. "small" has q4 rows of 1024 columns, "2b" the benchmark model's rows of 2048."""
    index, buf = W.synth_model(name, seed=21, body="q4", head="f16")
    ids = prompt(json.loads(index)["config"]["vocab"], 33, 9)
    runs = []
    for fusion in (True, False):
        with Q.Model.load(index, buf, options={"gdn_fusion": fusion}) as m:
            m.prefill_batched(ids)
            lg = [m.logits()]
            out = m.decode_ids(24, 8, [])
            m.reset()
            m.prefill_batched(ids)
            for i in range(23):
                lg.append(m.step(out[i], len(ids) + i))
            runs.append((out, np.stack(lg)))
    (a_ids, a_lg), (b_ids, b_lg) = runs
    assert a_ids == b_ids
    assert np.array_equal(a_lg.view(np.uint32), b_lg.view(np.uint32)), float(np.max(np.abs(a_lg - b_lg)))


@pytest.mark.parametrize("name", ["small", "2b"])
def test_mfma_gemv_matches_the_vector_path(name):
    """The decode program's q4 GEMVs on the int8 matrix cores (x as three signed base-256 digits of a
    22-bit fixed-point value per 64 columns, exact integer products) against the same GEMVs on the
    vector ALUs in f32 ({"mfma_gemv": false}): the same greedy ids over 24 steps, and logits after
    the prompt and every step within 2e-4 of each other (the two paths round x differently: the
    digits keep 2^-22 of each 64-column group's largest value, f32 products 2^-24 of each product)."""
    index, buf = W.synth_model(name, seed=23, body="q4", head="f16")
    ids = prompt(json.loads(index)["config"]["vocab"], 33, 10)
    runs = []
    for mfma in (True, False):
        with Q.Model.load(index, buf, options={"mfma_gemv": mfma}) as m:
            m.prefill_batched(ids)
            lg = [m.logits()]
            out = m.decode_ids(24, 8, [])
            m.reset()
            m.prefill_batched(ids)
            for i in range(23):
                lg.append(m.step(out[i], len(ids) + i))
            runs.append((out, np.stack(lg)))
    (a_ids, a_lg), (b_ids, b_lg) = runs
    err = float(np.max(np.abs(a_lg - b_lg)))
    print(f"{name}: matrix-core vs vector GEMVs: ids identical {a_ids == b_ids}, max |dlogit| {err:.2e}")
    assert a_ids == b_ids
    assert err <= 2e-4
