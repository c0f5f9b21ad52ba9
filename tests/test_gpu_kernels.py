"""HIP kernels through the C ABI against the CPU oracle (GPU box only).

Error metric: the reference's rel_err = max|got - want| / max(1e-6, max|want|), any non-finite
value counts as infinite (kernels/src/lib.rs:499-507). The HIP kernels accumulate in f32; the
oracle is the f64 build."""
import ctypes

import numpy as np
import pytest
import cpu_oracle as O
import devmem as D
import qne as Q

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    if got.shape != want.shape or not (np.all(np.isfinite(got)) and np.all(np.isfinite(want))):
        return np.inf
    return np.max(np.abs(got - want)) / max(1e-6, np.max(np.abs(want)))


to_dev = D.to_dev


def q4_matrix(rows, k, group, rng):
    q = rng.integers(0, 16, size=(rows, k), dtype=np.uint32)
    s = rng.uniform(0.002, 0.03, size=(rows, k // group)).astype(np.float16)
    z = rng.uniform(0, 15, size=(rows, k // group)).astype(np.float16)
    b = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    w = np.ascontiguousarray(b).view(np.uint32).reshape(rows, k // 8)
    sz = np.stack([s.view(np.uint16), z.view(np.uint16)], axis=-1).reshape(rows, -1)  # (scale, zero) pairs
    m = O.mat_struct(None, O.OC_Q4G, rows, k, group, w, s.view(np.uint16), z.view(np.uint16))
    return m, w, sz


def f16_matrix(rows, k, rng):
    w = rng.normal(0, 0.02, size=(rows, k)).astype(np.float16)
    return O.mat_struct(None, O.OC_F16, rows, k, 0, w.view(np.uint16)), w.view(np.uint16), None


@pytest.mark.parametrize("k", [512, 1024, 2048, 3584, 4096, 6144])
@pytest.mark.parametrize("kind,group", [(Q.MAT_Q4, 64), (Q.MAT_Q4, 32), (Q.MAT_F16, 0)])
@pytest.mark.parametrize("epi", [Q.EPI_STORE, Q.EPI_ACCUMULATE, Q.EPI_SWIGLU])
@pytest.mark.parametrize("norm", [False, True])
def test_gemv_matches_oracle(k, kind, group, epi, norm):
    rng = np.random.default_rng(k + 7 * epi + 3 * group + norm)
    rows = 2 * 37 if epi == Q.EPI_SWIGLU else 37
    if k == 2048 and epi == Q.EPI_STORE:
        rows = 8224  # the GDN in-projection: many rows per wave, ragged tail
    m, w, sz = q4_matrix(rows, k, group, rng) if kind == Q.MAT_Q4 else f16_matrix(rows, k, rng)
    x = rng.normal(0, 1, size=k).astype(np.float32)
    g = rng.normal(1, 0.2, size=k).astype(np.float32)
    out_rows = rows // 2 if epi == Q.EPI_SWIGLU else rows
    y0 = rng.normal(size=out_rows).astype(np.float32)
    xin = x.copy()
    if norm:
        O.lib("f64").oc_rmsnorm(O.ptr(x), O.ptr(g), O.ptr(xin), k, 1e-6)
    want = y0.copy()
    O.lib("f64").oc_gemv(ctypes.byref(m), O.ptr(xin), O.ptr(want), {0: O.STORE, 1: O.ACCUMULATE, 2: O.SWIGLU}[epi])
    dw, dx, dy, dg = to_dev(w), to_dev(x), to_dev(y0), to_dev(g)
    dsz = to_dev(sz) if sz is not None else None
    Q.gemv(kind, dw.data_ptr(), dsz.data_ptr() if dsz is not None else 0, rows, k, group, dx.data_ptr(), dy.data_ptr(),
           epi, norm=dg.data_ptr() if norm else 0)
    D.sync()
    err = rel_err(dy.numpy(), want)
    assert err < 2e-5, err


def test_gemv_rejects_unsupported_width():
    with pytest.raises(Q.QneError) as e:
        Q.gemv(Q.MAT_F16, 1, 0, 4, 1000, 0, 1, 1)
    assert e.value.code == Q.EINVAL


@pytest.mark.parametrize("batch", [1, 3, 16])
def test_gdn_step_matches_oracle(batch):
    rng = np.random.default_rng(batch)
    H, dk, dv = 16, 128, 128
    q = rng.normal(size=(batch, H, dk)).astype(np.float32)
    k = rng.normal(size=(batch, H, dk)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(batch, H, dv)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.normal(size=(batch, H))))).astype(np.float32)
    g = np.exp(-np.log1p(np.exp(rng.normal(size=(batch, H))))).astype(np.float32)
    S = rng.normal(0, 0.1, size=(batch, H, dk, dv)).astype(np.float32)
    want_S, want_o = S.copy(), np.empty((batch, H, dv), np.float32)
    for b in range(batch):
        for h in range(H):
            O.lib("f64").oc_delta_rule(dk, dv, O.ptr(q[b, h]), O.ptr(k[b, h]), O.ptr(v[b, h]), float(beta[b, h]),
                                       float(g[b, h]), O.ptr(want_S[b, h]), O.ptr(want_o[b, h]))
    d = [to_dev(a) for a in (q, k, v, beta, g, S)]
    out = D.empty((batch, H, dv), np.float32)
    Q.gdn_step(*[t.data_ptr() for t in d], out.data_ptr(), batch, H)
    D.sync()
    assert rel_err(out.numpy(), want_o) < 1e-5
    assert rel_err(d[5].numpy(), want_S) < 1e-5


def test_gdn_multi_token_equals_sequential_oracle():
    rng = np.random.default_rng(44)
    B, T, H, dk = 2, 80, 4, 128
    q = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    k = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(np.float32)
    g = np.exp(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(np.float32)
    S = rng.normal(0, 0.1, size=(B, H, dk, dk)).astype(np.float32)
    want_S, want_o = S.copy(), np.empty_like(v)
    for b in range(B):
        for t in range(T):
            for h in range(H):
                O.lib("f64").oc_delta_rule(dk, dk, O.ptr(q[b, t, h]), O.ptr(k[b, t, h]), O.ptr(v[b, t, h]),
                                           float(beta[b, t, h]), float(g[b, t, h]), O.ptr(want_S[b, h]),
                                           O.ptr(want_o[b, t, h]))
    d = [to_dev(a) for a in (q, k, v, beta, g, S)]
    out = D.empty_like(d[2])
    Q.gdn_prefill_chunked(*[t.data_ptr() for t in d], out.data_ptr(), B, T, H)
    D.sync()
    assert rel_err(out.numpy(), want_o) < 1e-4
    assert rel_err(d[5].numpy(), want_S) < 1e-4


def gdn_inputs(rng, B, T, H, mode="random"):
    dk = 128
    q = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    k = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(np.float32)
    g = np.exp(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(np.float32)
    if mode == "same_k":  # one key repeated, beta = 1, no decay: the WY solve at its least damped
        k[:] = k[:, :1]
        beta[:] = 1.0
        g[:] = 1.0
    elif mode == "tiny_g":  # decays that underflow the chunk's cumulative product
        g[:, ::7] = 1e-30
    elif mode == "beta0":  # no writes: the state only decays
        beta[:] = 0.0
    S = rng.normal(0, 0.1, size=(B, H, dk, dk)).astype(np.float32)
    return q, k, v, beta, g, S


def oracle_gdn_tokens(q, k, v, beta, g, S):
    B, T, H, dk = q.shape
    want_S, want_o = S.copy(), np.empty_like(v)
    L = O.lib("f64")
    for b in range(B):
        for t in range(T):
            for h in range(H):
                L.oc_delta_rule(dk, dk, O.ptr(q[b, t, h]), O.ptr(k[b, t, h]), O.ptr(v[b, t, h]), float(beta[b, t, h]),
                                float(g[b, t, h]), O.ptr(want_S[b, h]), O.ptr(want_o[b, t, h]))
    return want_o, want_S


@pytest.mark.parametrize("B,T,H,mode", [(1, 48, 3, "random"), (1, 64, 2, "random"), (2, 65, 2, "random"),
                                        (1, 200, 2, "tiny_g"), (1, 130, 1, "same_k"), (3, 129, 2, "beta0"),
                                        (2, 300, 5, "random")])
def test_gdn_multi_token_cases(B, T, H, mode):
    """Token-by-token (T < 64) and chunk-64 WY form (T >= 64, ragged last chunks) against the
    oracle's sequential recurrence (f64), including a repeated key with beta = 1 and g = 1,
    decays that underflow, and beta = 0."""
    rng = np.random.default_rng(T * 10 + H)
    q, k, v, beta, g, S = gdn_inputs(rng, B, T, H, mode)
    want_o, want_S = oracle_gdn_tokens(q, k, v, beta, g, S)
    d = [to_dev(a) for a in (q, k, v, beta, g, S)]
    out = D.empty_like(d[2])
    Q.gdn_prefill_chunked(*[t.data_ptr() for t in d], out.data_ptr(), B, T, H)
    D.sync()
    assert rel_err(out.numpy(), want_o) < 1e-4
    assert rel_err(d[5].numpy(), want_S) < 1e-4


def test_gdn_chunked_split_calls_equal_one_call():
    """The state carried between calls: 64 + 136 tokens in two calls (WY, WY) and 40 + 160 (token by
    token, then WY) against one 200-token call, within the f32 tolerance of either form."""
    rng = np.random.default_rng(77)
    B, T, H = 2, 200, 2
    q, k, v, beta, g, S = gdn_inputs(rng, B, T, H)
    whole = [to_dev(a) for a in (q, k, v, beta, g, S)]
    out = D.empty_like(whole[2])
    Q.gdn_prefill_chunked(*[t.data_ptr() for t in whole], out.data_ptr(), B, T, H)
    for cut in (64, 40):
        st = to_dev(S)
        parts = []
        for a, bnd in ((0, cut), (cut, T)):
            sl = [to_dev(np.ascontiguousarray(x[:, a:bnd])) for x in (q, k, v, beta, g)]
            o = D.empty_like(sl[2])
            Q.gdn_prefill_chunked(*[t.data_ptr() for t in sl], st.data_ptr(), o.data_ptr(), B, bnd - a, H)
            parts.append(o)
        D.sync()
        got = np.concatenate([p.numpy() for p in parts], axis=1)
        assert rel_err(got, out.numpy()) < 1e-4, cut
        assert rel_err(st.numpy(), whole[5].numpy()) < 1e-4, cut


@pytest.mark.parametrize("batch,nq,nkv", [(1, 16, 4), (3, 8, 2), (5, 4, 4)])
def test_paged_attention_matches_dense(batch, nq, nkv):
    rng = np.random.default_rng(batch * 100 + nq)
    hd, blk, max_blocks = 256, 16, 64
    pool = batch * max_blocks + 5
    ctx = rng.integers(0, max_blocks * blk - 1, size=batch).astype(np.int32)
    ctx[0] = 0  # first position
    perm = rng.permutation(pool).astype(np.int32)
    bt = perm[: batch * max_blocks].reshape(batch, max_blocks)
    kpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    vpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    q = rng.normal(size=(batch, nq, hd)).astype(np.float32)
    kn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    vn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    want = np.empty((batch, nq, hd), np.float32)
    for b in range(batch):
        n = ctx[b] + 1
        kd = np.empty((nkv, n, hd), np.float16)
        vd = np.empty((nkv, n, hd), np.float16)
        for p in range(ctx[b]):
            kd[:, p] = kpool[bt[b, p // blk], :, p % blk]
            vd[:, p] = vpool[bt[b, p // blk], :, p % blk]
        kd[:, ctx[b]] = kn[b].astype(np.float16)
        vd[:, ctx[b]] = vn[b].astype(np.float16)
        O.lib("f64").oc_attn_dense(nq, nkv, hd, O.ptr(q[b]), O.ptr(kd.view(np.uint16)), O.ptr(vd.view(np.uint16)), n,
                                   1 / 16, O.ptr(want[b]))
    dk, dv = to_dev(kpool.view(np.uint16)), to_dev(vpool.view(np.uint16))
    dq, dkn, dvn, dbt, dctx = to_dev(q), to_dev(kn), to_dev(vn), to_dev(bt), to_dev(ctx)
    out = D.empty((batch, nq, hd), np.float32)
    Q.paged_attn_decode(dq.data_ptr(), dkn.data_ptr(), dvn.data_ptr(), dk.data_ptr(), dv.data_ptr(), dbt.data_ptr(),
                        max_blocks, dctx.data_ptr(), out.data_ptr(), batch, nq, nkv)
    D.sync()
    assert rel_err(out.numpy(), want) < 1e-5
    # the append wrote exactly the new token's f16 k/v and nothing else
    kp = dk.numpy().view(np.float16)
    for b in range(batch):
        p = ctx[b]
        np.testing.assert_array_equal(kp[bt[b, p // blk], :, p % blk], kn[b].astype(np.float16))
        kp[bt[b, p // blk], :, p % blk] = kpool[bt[b, p // blk], :, p % blk]
    np.testing.assert_array_equal(kp, kpool)


def test_paged_attention_config3_shape():
    """Config-3 shape: 64 sequences, 16 q / 4 kv heads of 256, contexts uniform in [256, 4096], a
    randomly permuted block table over the pool, one appended token per sequence; against the dense
    unpaged oracle (f64)."""
    rng = np.random.default_rng(303)
    batch, nq, nkv, hd, blk, max_blocks = 64, 16, 4, 256, 16, 256
    pool = batch * max_blocks
    ctx = rng.integers(256, 4096, size=batch).astype(np.int32)
    bt = rng.permutation(pool).astype(np.int32).reshape(batch, max_blocks)
    kpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    vpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    q = rng.normal(size=(batch, nq, hd)).astype(np.float32)
    kn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    vn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    want = np.empty((batch, nq, hd), np.float32)
    for b in range(batch):
        n = ctx[b] + 1
        pos = np.arange(ctx[b])
        kd = np.empty((nkv, n, hd), np.float16)
        vd = np.empty((nkv, n, hd), np.float16)
        kd[:, :-1] = kpool[bt[b, pos // blk], :, pos % blk].transpose(1, 0, 2)
        vd[:, :-1] = vpool[bt[b, pos // blk], :, pos % blk].transpose(1, 0, 2)
        kd[:, -1] = kn[b].astype(np.float16)
        vd[:, -1] = vn[b].astype(np.float16)
        kd, vd = np.ascontiguousarray(kd), np.ascontiguousarray(vd)
        O.lib("f64").oc_attn_dense(nq, nkv, hd, O.ptr(q[b]), O.ptr(kd.view(np.uint16)), O.ptr(vd.view(np.uint16)), n,
                                   1 / 16, O.ptr(want[b]))
    dk, dv = to_dev(kpool.view(np.uint16)), to_dev(vpool.view(np.uint16))
    dq, dkn, dvn, dbt, dctx = to_dev(q), to_dev(kn), to_dev(vn), to_dev(bt), to_dev(ctx)
    out = D.empty((batch, nq, hd), np.float32)
    Q.paged_attn_decode(dq.data_ptr(), dkn.data_ptr(), dvn.data_ptr(), dk.data_ptr(), dv.data_ptr(), dbt.data_ptr(),
                        max_blocks, dctx.data_ptr(), out.data_ptr(), batch, nq, nkv)
    D.sync()
    assert rel_err(out.numpy(), want) < 1e-5


def test_gdn_step_config4_batch64():
    test_gdn_step_matches_oracle(64)


def test_gdn_prefill_config4_shape():
    """Config-4(b) shape: 2048 tokens per sequence at batch 4, 16 heads, in one call; against the
    sequential recurrence of the oracle (f64)."""
    rng = np.random.default_rng(404)
    B, T, H, dk = 4, 2048, 16, 128
    q = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    k = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(B, T, H, dk)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(np.float32)
    g = np.exp(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(np.float32)
    S = rng.normal(0, 0.1, size=(B, H, dk, dk)).astype(np.float32)
    want_S, want_o = S.copy(), np.empty_like(v)
    L = O.lib("f64")
    for b in range(B):
        for t in range(T):
            for h in range(H):
                L.oc_delta_rule(dk, dk, O.ptr(q[b, t, h]), O.ptr(k[b, t, h]), O.ptr(v[b, t, h]), float(beta[b, t, h]),
                                float(g[b, t, h]), O.ptr(want_S[b, h]), O.ptr(want_o[b, t, h]))
    d = [to_dev(a) for a in (q, k, v, beta, g, S)]
    out = D.empty_like(d[2])
    Q.gdn_prefill_chunked(*[t.data_ptr() for t in d], out.data_ptr(), B, T, H)
    D.sync()
    assert rel_err(out.numpy(), want_o) < 1e-4
    assert rel_err(d[5].numpy(), want_S) < 1e-4


@pytest.mark.parametrize("workgroups,n,rounds", [(2, 2, 5), (8, 2048, 11), (64, 2048, 8)])
def test_exchange_probe_runs_every_round(workgroups, n, rounds):
    """The hand-over probe: every round every workgroup publishes its share and sees everyone's, so
    after the last round its buffer holds every value of that round, tagged with it (value r + o at
    entry o), and the other buffer those of the round before."""
    import ctypes
    lib = Q.load_library()
    buf, ctl = D.zeros(2 * n, np.uint64), D.zeros(2, np.uint64)
    us = ctypes.c_double()
    assert lib.qne_exchange_probe(buf.ptr, n, rounds, workgroups, ctl.ptr, ctypes.byref(us)) == 0
    assert us.value > 0.0
    got = buf.numpy().reshape(2, n)
    for r in (rounds, rounds - 1):
        e = got[r & 1]
        assert np.all((e >> np.uint64(32)) == r)
        vals = (e & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
        np.testing.assert_array_equal(vals, (r + np.arange(n)).astype(np.float32))
    assert lib.qne_exchange_probe(buf.ptr, 3, rounds, workgroups, ctl.ptr, ctypes.byref(us)) == Q.EINVAL


@pytest.mark.parametrize("words,groups", [(4 * 1000003, 64), (4 * 256 * 4, 1), (4 * 7, 3)])
def test_stream_read_probe_reads_every_word_once(words, groups):
    """The streaming-read probe (shaders.rs:701-717) folds every 16-byte word into the sink: the xor
    of all sink words is the xor of all data words (a skipped or doubled word changes it)."""
    lib = Q.load_library()
    data = np.random.default_rng(words).integers(0, 2**32, size=words, dtype=np.uint32)
    d, sink = D.to_dev(data), D.zeros(groups * 256, np.uint32)
    assert lib.qne_stream_read(d.ptr, data.nbytes, sink.ptr, groups, None) == 0
    D.sync()
    assert int(np.bitwise_xor.reduce(sink.numpy())) == int(np.bitwise_xor.reduce(data))
    y = D.zeros(1, np.float32)
    for _ in range(5):
        assert lib.qne_noop_dispatch(y.ptr, None) == 0
    D.sync()
    assert float(y.numpy()[0]) == 5.0
