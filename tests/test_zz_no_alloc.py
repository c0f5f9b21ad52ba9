"""qne_paged_attn_decode_noalloc against qne_paged_attn_decode through the C ABI (GPU): the same
inputs give bitwise the same outputs and the same appended K/V, on two calls in a row (the second
smaller, so the fixed scratch holds the first call's partials when it starts); a call changes the
device's free memory by nothing; the call captured into a HIP graph on a created stream replays to
the same result; and a call whose partials do not fit the fixed scratch is rejected before any
device work."""
import numpy as np
import pytest

import devmem as D
import qne as Q

pytestmark = pytest.mark.gpu


def inputs(rng, batch, nq, nkv, max_blocks, lo, hi):
    hd, blk = 256, 16
    pool = batch * max_blocks
    ctx = rng.integers(lo, hi, size=batch).astype(np.int32)
    bt = rng.permutation(pool).astype(np.int32).reshape(batch, max_blocks)
    kpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    vpool = rng.normal(size=(pool, nkv, blk, hd)).astype(np.float16)
    q = rng.normal(size=(batch, nq, hd)).astype(np.float32)
    kn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    vn = rng.normal(size=(batch, nkv, hd)).astype(np.float32)
    return q, kn, vn, kpool.view(np.uint16), vpool.view(np.uint16), bt, ctx


def run(fn, args, batch, nq, nkv, max_blocks):
    q, kn, vn, kp, vp, bt, ctx = args
    d = [D.to_dev(a) for a in (q, kn, vn, kp, vp, bt, ctx)]
    out = D.empty((batch, nq, 256), np.float32)
    fn(d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, d[4].ptr, d[5].ptr, max_blocks, d[6].ptr, out.ptr, batch, nq, nkv)
    D.sync()
    return out.numpy(), d[3].numpy(), d[4].numpy()


CASES = [(64, 16, 4, 256, 256, 4096),  # config 3: 64 sequences, contexts U[256, 4096)
         (3, 8, 2, 64, 0, 1000)]       # smaller: fewer sequences, other heads, shorter contexts


def test_noalloc_equals_the_allocating_entry_point_on_two_calls():
    for i, (batch, nq, nkv, max_blocks, lo, hi) in enumerate(CASES):
        args = inputs(np.random.default_rng(50 + i), batch, nq, nkv, max_blocks, lo, hi)
        want = run(Q.paged_attn_decode, args, batch, nq, nkv, max_blocks)
        got = run(Q.paged_attn_decode_noalloc, args, batch, nq, nkv, max_blocks)
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), f"call {i}: outputs differ"
        assert np.array_equal(got[1], want[1]) and np.array_equal(got[2], want[2]), f"call {i}: appended K/V differ"


def test_noalloc_allocates_nothing_and_replays_under_graph_capture():
    batch, nq, nkv, max_blocks, lo, hi = CASES[1]
    args = inputs(np.random.default_rng(60), batch, nq, nkv, max_blocks, lo, hi)
    want = run(Q.paged_attn_decode, args, batch, nq, nkv, max_blocks)[0]
    q, kn, vn, kp, vp, bt, ctx = args
    d = [D.to_dev(a) for a in (q, kn, vn, kp, vp, bt, ctx)]
    out = D.empty((batch, nq, 256), np.float32)

    def call(stream=0):
        Q.paged_attn_decode_noalloc(d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, d[4].ptr, d[5].ptr, max_blocks, d[6].ptr,
                                    out.ptr, batch, nq, nkv, stream)

    call()  # warm-up: the runtime's own first-launch state
    D.sync()
    free0 = D.mem_free()
    call()
    D.sync()
    assert D.mem_free() == free0, "the no-allocation entry point changed the device's free memory"
    assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32))
    # captured on a caller's stream (the use it exists for), replayed with eager work between replays
    s = D.Stream()
    g = s.capture(lambda: call(s.ptr))
    try:
        for rep in range(3):
            out.zero()  # eager work on the null stream between replays
            D.sync()
            g.launch(s)
            s.sync()
            got = out.numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"graph replay {rep} differs"
            call()  # an eager call between replays shares the same fixed scratch
            D.sync()
    finally:
        g.destroy()
        s.destroy()


def test_noalloc_rejects_calls_beyond_its_scratch():
    # 2048 sequences x 4 kv heads: one split each, 2048 * 4 * 4 partials of 1032 bytes > 8 MiB
    with pytest.raises(Q.QneError) as e:
        Q.paged_attn_decode_noalloc(1, 1, 1, 1, 1, 1, 16, 1, 1, 2048, 16, 4)
    assert e.value.code == Q.EINVAL and "8388608" in str(e.value)
