"""qne_paged_attn_decode_noalloc against qne_paged_attn_decode through the C ABI (GPU): the same
inputs give bitwise the same outputs and the same appended K/V, on two calls in a row (the second
smaller, so the fixed scratch holds the first call's partials when it starts), and a call whose
partials do not fit the fixed scratch is rejected before any device work."""
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


def test_noalloc_rejects_calls_beyond_its_scratch():
    # 2048 sequences x 4 kv heads: one split each, 2048 * 4 * 4 partials of 1032 bytes > 8 MiB
    with pytest.raises(Q.QneError) as e:
        Q.paged_attn_decode_noalloc(1, 1, 1, 1, 1, 1, 16, 1, 1, 2048, 16, 4)
    assert e.value.code == Q.EINVAL and "8388608" in str(e.value)
