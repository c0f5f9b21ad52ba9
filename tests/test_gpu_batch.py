"""Batched decode through the C ABI on the GPU: the M <= 64 MFMA GEMM against the oracle's GEMV row
by row, and whole batches of sequences against the oracle's single-sequence decode.

The GEMM splits x into two f16 halves (hi + lo) so its products keep about 22 bits; it accumulates
in f32, so it is held to the GEMV's bar (rel_err < 2e-5 against the f64 oracle). Batched decode is
held to the model tests' bar: logits within 1e-3 of the oracle, identical greedy ids."""
import ctypes

import numpy as np
import pytest
import cpu_oracle as O
import devmem as D
import qne as Q
import weights as W
from test_gpu_kernels import f16_matrix, q4_matrix, rel_err, to_dev

pytestmark = pytest.mark.gpu


def oracle_rows(m, X, G, epi, y0, norm):
    """Row by row with the oracle GEMV (and RMSNorm prologue): the reference's gemm semantics."""
    out = y0.copy()
    for r in range(X.shape[0]):
        x = np.ascontiguousarray(X[r])
        if norm:
            xn = np.empty_like(x)
            O.lib("f64").oc_rmsnorm(O.ptr(x), O.ptr(G), O.ptr(xn), x.size, 1e-6)
            x = xn
        O.lib("f64").oc_gemv(ctypes.byref(m), O.ptr(x), O.ptr(out[r]), {0: O.STORE, 1: O.ACCUMULATE, 2: O.SWIGLU}[epi])
    return out


def run_gemm(kind, group, rows, k, M, epi, norm, seed, x_pad=0, y_pad=0):
    rng = np.random.default_rng(seed)
    m, w, sz = q4_matrix(rows, k, group, rng) if kind == Q.MAT_Q4 else f16_matrix(rows, k, rng)
    X = rng.normal(0, 1, size=(M, k + x_pad)).astype(np.float32)
    G = rng.normal(1, 0.2, size=k).astype(np.float32)
    n_out = rows // 2 if epi == Q.EPI_SWIGLU else rows
    Y0 = rng.normal(size=(M, n_out + y_pad)).astype(np.float32)
    want = Y0.copy()
    want[:, :n_out] = oracle_rows(m, np.ascontiguousarray(X[:, :k]), G, epi, np.ascontiguousarray(Y0[:, :n_out]), norm)
    dw, dx, dy, dg = to_dev(w), to_dev(X), to_dev(Y0), to_dev(G)
    dsz = to_dev(sz) if sz is not None else None
    Q.gemm(kind, dw.data_ptr(), dsz.data_ptr() if dsz is not None else 0, rows, k, group, dx.data_ptr(), k + x_pad, M,
           dy.data_ptr(), n_out + y_pad, epi, norm=dg.data_ptr() if norm else 0)
    D.sync()
    return dy.numpy(), want


@pytest.mark.parametrize("k", [512, 2048, 6144])
@pytest.mark.parametrize("kind,group", [(Q.MAT_Q4, 64), (Q.MAT_Q4, 128), (Q.MAT_F16, 0)])
@pytest.mark.parametrize("epi", [Q.EPI_STORE, Q.EPI_ACCUMULATE, Q.EPI_SWIGLU])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("M", [1, 7, 64])
def test_gemm_matches_oracle(k, kind, group, epi, norm, M):
    rows = 2 * 150 if epi == Q.EPI_SWIGLU else 300  # ragged last tile of 128 rows
    got, want = run_gemm(kind, group, rows, k, M, epi, norm, seed=k + 7 * epi + 3 * group + norm + 101 * M)
    err = rel_err(got, want)
    assert err < 2e-5, err


@pytest.mark.parametrize("kind,group", [(Q.MAT_Q4, 64), (Q.MAT_F16, 0)])
@pytest.mark.parametrize("epi", [Q.EPI_STORE, Q.EPI_SWIGLU])
@pytest.mark.parametrize("M", [65, 200])
def test_gemm_row_tiles_match_oracle(kind, group, epi, M):
    """More than 64 rows run as tiles of 64 rows (the prefill's passes), each over the same weights;
    a ragged last tile."""
    rows = 2 * 150 if epi == Q.EPI_SWIGLU else 300
    got, want = run_gemm(kind, group, rows, 1024, M, epi, True, seed=41 + M + 5 * epi + group)
    assert rel_err(got, want) < 2e-5


@pytest.mark.parametrize("norm", [False, True])
def test_gemm_swiglu_applied_by_the_gemm(norm):
    """A SwiGLU GEMM with one split over several row tiles (K = 128: two chunks) applies
    silu(gate) * up in the GEMM itself, with no reduce pass; gate and up rows 256 apart, two
    workgroups of 128 output columns, a ragged last row tile."""
    got, want = run_gemm(Q.MAT_Q4, 64, 2 * 256, 128, 200, Q.EPI_SWIGLU, norm, seed=61 + norm)
    assert rel_err(got, want) < 2e-5


@pytest.mark.parametrize("M", [512, 2048])
def test_gemm_full_pass_of_rows(M):
    got, want = run_gemm(Q.MAT_Q4, 64, 256, 512, M, Q.EPI_ACCUMULATE, True, seed=77 + M)
    assert rel_err(got, want) < 2e-5


@pytest.mark.parametrize("kind,group", [(Q.MAT_Q4, 64), (Q.MAT_F16, 0)])
def test_gemm_one_split_direct_epilogue(kind, group):
    """More than 512 tiles of 128 rows: one split, the GEMM applies 1 / rms and the epilogue itself
    (the LM head's path)."""
    got, want = run_gemm(kind, group, 66000, 512, 3, Q.EPI_ACCUMULATE, True, seed=5)
    assert rel_err(got, want) < 2e-5


def test_gemm_strided_rows_untouched_padding():
    got, want = run_gemm(Q.MAT_Q4, 64, 260, 1024, 5, Q.EPI_STORE, True, seed=9, x_pad=12, y_pad=7)
    assert rel_err(got, want) < 2e-5
    assert np.array_equal(got[:, 260:], want[:, 260:])  # columns past the outputs keep their values


def test_gemm_row_result_does_not_depend_on_other_rows():
    """Each row's sum runs in the same order whatever the other rows hold: bitwise equal."""
    rng = np.random.default_rng(3)
    rows, k = 640, 2048
    _, w, sz = q4_matrix(rows, k, 64, rng)
    X = rng.normal(size=(64, k)).astype(np.float32)
    dw, dsz = to_dev(w), to_dev(sz)
    full = D.zeros((64, rows), np.float32)
    one = D.zeros((1, rows), np.float32)
    dx = to_dev(X)
    Q.gemm(Q.MAT_Q4, dw.data_ptr(), dsz.data_ptr(), rows, k, 64, dx.data_ptr(), k, 64, full.data_ptr(), rows)
    dx1 = to_dev(X[37:38])
    Q.gemm(Q.MAT_Q4, dw.data_ptr(), dsz.data_ptr(), rows, k, 64, dx1.data_ptr(), k, 1, one.data_ptr(), rows)
    # and in the fourth row tile of a 250-row call
    X4 = rng.normal(size=(250, k)).astype(np.float32)
    X4[237] = X[37]
    big = D.zeros((250, rows), np.float32)
    dx4 = to_dev(X4)
    Q.gemm(Q.MAT_Q4, dw.data_ptr(), dsz.data_ptr(), rows, k, 64, dx4.data_ptr(), k, 250, big.data_ptr(), rows)
    D.sync()
    assert np.array_equal(full.numpy()[37], one.numpy()[0])
    assert np.array_equal(big.numpy()[237], one.numpy()[0])


def test_gemm_rejects_bad_shapes():
    for args in [(Q.MAT_F16, 0, 256, 1000, 4), (Q.MAT_Q4, 32, 256, 1024, 4), (Q.MAT_F16, 0, 256, 1024, 2049),
                 (Q.MAT_F16, 0, 256, 1024, 0)]:
        kind, group, rows, k, M = args
        with pytest.raises(Q.QneError) as e:
            Q.gemm(kind, 1, 1, rows, k, group, 1, k, M, 1, rows)
        assert e.value.code == Q.EINVAL


# ---- whole batches ----

@pytest.fixture(scope="module", params=[("tiny", "q4", "f16"), ("small", "q4", "f16"), ("tiny", "f16", "q4")],
                ids=["tiny-q4body", "small-q4body", "tiny-f16body-q4head"])
def pair(request):
    name, body, head = request.param
    index, buf = W.synth_model(name, seed=11, body=body, head=head, norm_jitter=0.1)
    m = Q.Model.load(index, buf)
    om = O.OracleModel(index, buf, "f64")
    yield m, om
    m.close()


def prompts(vocab, lengths, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, size=n).astype(np.uint32) for n in lengths]


def test_batch_continues_each_sequence_like_the_oracle(pair):
    m, om = pair
    lengths = [5, 17, 40, 1, 33]
    ps = prompts(m.vocab, lengths, 21)
    steps = 20
    with Q.Batch(m, max_rows=8, max_context=512) as b:
        for r, p in enumerate(ps):
            m.reset()
            m.prefill_batched(p)
            b.admit(r)
        tok, pos = b.row_state(len(ps))
        assert list(pos) == lengths
        picks, logits = b.step(len(ps), logits=True)
        ids = b.decode(len(ps), steps - 1)
        ms, n = b.last_decode_timing()  # the device time of the chained steps
        assert n == steps - 1 and ms > 0.0
    for r, p in enumerate(ps):
        om.reset()
        want_ids, want_logits = om.greedy(p, steps + 1)
        assert tok[r] == want_ids[0]
        assert np.max(np.abs(logits[r] - want_logits[1])) < 1e-3, r
        got = [int(picks[r])] + [int(x) for x in ids[:, r]]
        assert got == want_ids[1:], r


def test_batch_teacher_forced_logits_and_empty_rows(pair):
    """Rows started empty (reset_row) and fed given tokens: every step's logits against the
    oracle's token-by-token run from position 0."""
    m, om = pair
    R, T = 3, 6
    seqs = prompts(m.vocab, [T] * R, 8)
    with Q.Batch(m, max_rows=R, max_context=64) as b:
        for r in range(R):
            b.reset_row(r, int(seqs[r][0]))
        got = []
        for t in range(T):
            _, lg = b.step(R, tokens=[int(s[t]) for s in seqs], logits=True)
            got.append(lg)
    for r in range(R):
        om.reset()
        for t in range(T):
            want = om.token(int(seqs[r][t]), t)
            assert np.max(np.abs(got[t][r] - want)) < 1e-3, (r, t)


def test_batch_is_bitwise_repeatable(pair):
    m, _ = pair
    ps = prompts(m.vocab, [9, 3, 27], 4)
    runs = []
    for _ in range(2):
        with Q.Batch(m, max_rows=4, max_context=256) as b:
            for r, p in enumerate(ps):
                m.reset()
                m.prefill_batched(p)
                b.admit(r)
            _, lg = b.step(3, logits=True)
            runs.append((lg, b.decode(3, 12)))
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])


def test_batch_errors(pair):
    m, _ = pair
    with Q.Batch(m, max_rows=2, max_context=32) as b:
        with pytest.raises(Q.QneError) as e:
            b.admit(2)
        assert e.value.code == Q.EINVAL
        with pytest.raises(Q.QneError) as e:
            b.step(3)
        assert e.value.code == Q.EINVAL
        b.reset_row(0, 1)
        b.reset_row(1, 2)
        with pytest.raises(Q.QneError) as e:
            b.decode(2, 33)  # past the batch context
        assert e.value.code == Q.ECONTEXT
        with pytest.raises(Q.QneError) as e:
            b.step(2, tokens=[1, m.vocab])
        assert e.value.code == Q.EINVAL
        m.reset()
        m.prefill_batched(np.arange(40, dtype=np.uint32))
        with pytest.raises(Q.QneError) as e:
            b.admit(0)  # the model's sequence is longer than the batch context
        assert e.value.code == Q.ECONTEXT
    with pytest.raises(Q.QneError):
        Q.Batch(m, max_rows=65, max_context=32)


def test_batch_row_equals_the_same_row_in_a_one_row_batch(pair):
    """A row's step does not depend on the other rows: every row of a 5-row step is bitwise the step
    of a 1-row batch holding the same sequence (qne_batch_copy_row)."""
    m, _ = pair
    ps = prompts(m.vocab, [12, 1, 30, 7, 19], 31)
    with Q.Batch(m, max_rows=5, max_context=128) as b, Q.Batch(m, max_rows=1, max_context=128) as one:
        for r, p in enumerate(ps):
            m.reset()
            m.prefill_batched(p)
            b.admit(r)
        single = []
        for r in range(5):
            one.copy_row(0, b, r)
            single.append(one.step(1, logits=True))
        picks, lg = b.step(5, logits=True)
    for r in range(5):
        assert int(single[r][0][0]) == int(picks[r]), r
        assert np.array_equal(single[r][1][0].view(np.uint32), lg[r].view(np.uint32)), r


# ---- config 5 at its own workload: 64 rows of the 2B int4 model, contexts U[256, 4096) ----

C5_ROWS = [0, 31, 63]  # where the fixture sequences sit among the synthetic rows


@pytest.fixture(scope="module")
def c5():
    """The c5_rows fixture (three sequences of the 2B int4 model decoded by the oracle) and the model."""
    from test_gpu_golden import fixture, synth
    g = fixture("c5_rows")
    case = __import__("json").loads(str(g["case"]))
    index, buf = synth(case)
    m = Q.Model.load(index, buf)
    yield g, m
    m.close()


def c5_batch(m, g, seed):
    """64 rows: synthetic KV caches and recurrent states at contexts U[256, 4096), with the fixture's
    three sequences (prefilled through the model) admitted at C5_ROWS."""
    b = Q.Batch(m, max_rows=64, max_context=4096)
    ctx = np.random.default_rng(seed).integers(256, 4096 - 32, size=64).astype(np.uint32)
    b.fill_synthetic(ctx, seed=seed)
    b.prompt_logits = {}  # fixture row -> the model's logits after its prompt (logged step 0)
    for i, r in enumerate(C5_ROWS):
        n = int(g["plen"][i])
        p = g["prompt"][i, :n]
        m.reset()
        for s in range(0, n, 512):
            m.prefill_chunk(p[s:s + 512], s, s + 512 >= n)
        b.prompt_logits[i] = m.logits()
        b.admit(r)
    return b, ctx


def test_config5_fixture_rows_decode_like_the_oracle(c5):
    """The three fixture sequences inside a 64-row batch of the 2B model: 16 greedy ids identical to
    the oracle's, and at each of the fixture's logged steps (0, 1, 8, 15) the row's logits within
    1e-2 (the stated bar) of the oracle's sampled logits (kernels/src/model.rs:380-392 per row).
    Step 0 is the prompt's logits from prefill_chunk; steps 1, 8 and 15 come from batched steps
    that return logits, with greedy decode windows between them."""
    g, m = c5
    b, ctx = c5_batch(m, g, seed=17)
    steps = [int(x) for x in g["steps"]]
    assert steps == [0, 1, 8, 15], steps
    lg_at = {}
    with b:
        tok, pos = b.row_state(64)
        for i, r in enumerate(C5_ROWS):
            assert int(pos[r]) == int(g["plen"][i]) and int(tok[r]) == int(g["ids"][i][0]), r
            assert all(int(pos[x]) == int(ctx[x]) for x in range(64) if x not in C5_ROWS)
        p1, lg_at[1] = b.step(64, logits=True)   # feeds ids[0]: logits of step 1, pick ids[1]
        r1 = b.decode(64, 6)                      # picks ids[2..7]
        p8, lg_at[8] = b.step(64, logits=True)   # feeds ids[7]: step 8, pick ids[8]
        r2 = b.decode(64, 6)                      # picks ids[9..14]
        p15, lg_at[15] = b.step(64, logits=True)  # feeds ids[14]: step 15, pick ids[15]
    worst = 0.0
    for i, r in enumerate(C5_ROWS):
        got = ([int(tok[r]), int(p1[r])] + [int(x) for x in r1[:, r]] + [int(p8[r])] + [int(x) for x in r2[:, r]]
               + [int(p15[r])])
        want = [int(x) for x in g["ids"][i]]
        assert got == want, f"row {r}: first divergence at step {next(j for j, (a, c) in enumerate(zip(got, want)) if a != c)}"
        for j, s in enumerate(steps):
            v = b.prompt_logits[i] if s == 0 else lg_at[s][r]
            err = float(np.max(np.abs(v[g["logit_idx"][i, j]] - g["logit_val"][i, j])))
            assert err <= 1e-2, f"row {r} step {s}: max |dlogit| {err:.3e}"
            worst = max(worst, err)
    print(f"config 5: fixture rows identical over 16 steps; max |dlogit| at steps {steps} {worst:.2e}")


def test_config5_each_row_equals_a_one_row_batch(c5):
    """Every one of the 64 rows (synthetic contexts up to 4096, and the fixture rows) steps bitwise
    as it does alone in a 1-row batch: the split-K GEMM reduce, the per-row attention splits and the
    per-row GDN do not depend on the batch."""
    g, m = c5
    b, _ = c5_batch(m, g, seed=23)
    with b, Q.Batch(m, max_rows=1, max_context=4096) as one:
        single = []
        for r in range(64):
            one.copy_row(0, b, r)
            single.append(one.step(1, logits=True))
        picks, lg = b.step(64, logits=True)
    bad = [r for r in range(64) if int(single[r][0][0]) != int(picks[r])
           or not np.array_equal(single[r][1][0].view(np.uint32), lg[r].view(np.uint32))]
    assert not bad, f"rows whose 64-row step differs from their 1-row step: {bad}"
