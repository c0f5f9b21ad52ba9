"""Device token sampling (qne_sample) against the oracle's restatement of src/sampling.rs: the same
logits, options and seed must give the same token stream, bit for bit, over greedy and
temperature sampling, top-k up to 1024, top-p, presence penalty, grammar masks, the tool-call
bias, equal logits (taken in increasing token order) and the fail-closed cases."""
import numpy as np
import pytest

import devmem as D
import qne as Q
import weights as W
from cpu_oracle import OracleSampler, bitset

pytestmark = pytest.mark.gpu


def run_both(logits_rows, opts, masks=None, bias=None):
    """Samples each row with a device sampler and the oracle sampler built from the same options;
    returns both token lists (the state advances over the rows)."""
    V = logits_rows[0].size
    got, want = [], []
    with Q.Sampler(V, **opts) as s:
        o = OracleSampler(**opts)
        for r, lg in enumerate(logits_rows):
            m, ml = (masks[r] if masks else (None, 0))
            bt, bv = bias if bias else (0xFFFFFFFF, 0.0)
            host = lg.copy()
            if bias and bt < V:
                host[bt] = np.float32(host[bt] + np.float32(bv))
            d = D.to_dev(np.ascontiguousarray(lg))
            got.append(s.sample(d.data_ptr(), m, ml, bt, bv))
            want.append(o.sample(host, m, ml))
    return got, want


@pytest.mark.parametrize("V", [5, 1000, 151936])
@pytest.mark.parametrize("opts", [
    dict(temperature=0.0),
    dict(temperature=0.6, top_k=20, top_p=0.95, seed=42),
    dict(temperature=1.0, top_k=1024, top_p=1.0, seed=9),
    dict(temperature=2.0, top_k=50, top_p=0.5, seed=3, presence_penalty=1.5),
    dict(temperature=0.3, top_k=0, top_p=0.9, seed=1),
])
def test_device_sampler_matches_oracle(V, opts):
    rng = np.random.default_rng(V + int(opts.get("seed", 0)))
    rows = [rng.normal(0, 3, size=V).astype(np.float32) for _ in range(24)]
    got, want = run_both(rows, opts)
    assert got == want


def test_masks_penalty_and_bias():
    V = 151936
    rng = np.random.default_rng(4)
    rows, masks = [], []
    for r in range(20):
        rows.append(rng.normal(0, 2, size=V).astype(np.float32))
        if r % 3 == 2:
            masks.append((None, 0))
        else:
            n = int(rng.integers(1, 3000))
            allowed = rng.choice(V + 100, size=n, replace=False)  # some past the vocabulary
            ml = int(rng.integers(V // 2, V + 100))
            masks.append((bitset(allowed, ml), ml))
    for opts in (dict(temperature=0.0, presence_penalty=2.0), dict(temperature=0.8, top_k=40, top_p=0.9, seed=5,
                                                                    presence_penalty=1.0)):
        got, want = run_both(rows, opts, masks=masks, bias=(777, 6.5))
        assert got == want


def test_repeated_samples_of_one_row_with_penalty():
    """The presence penalty pushes the greedy pick down the row one token at a time."""
    V = 4096
    lg = np.sort(np.random.default_rng(2).normal(size=V).astype(np.float32))[::-1].copy()
    got, want = run_both([lg] * 40, dict(temperature=0.0, presence_penalty=100.0))
    assert got == want == list(range(40))


@pytest.mark.parametrize("top_k", [1, 20, 1024])
def test_equal_logits_take_the_lowest_tokens(top_k):
    """Thousands of equal values at the top-k boundary: the k-th largest key is shared, and the
    device must take the lowest token ids among the equal ones."""
    V = 151936
    lg = np.zeros(V, np.float32)
    lg[[10, 90000, 151000]] = 1.0  # three above the tie
    rows = [lg, np.full(V, -0.0, np.float32), lg]
    got, want = run_both(rows, dict(temperature=1.0, top_k=top_k, top_p=1.0, seed=8))
    assert got == want


def test_signed_zero_and_extreme_values_use_the_total_order():
    V = 2000
    rng = np.random.default_rng(6)
    lg = rng.choice(np.array([-0.0, 0.0, 1e30, -1e30, 3.4e38, -3.4e38, -np.inf, 1e-40, -1e-40], np.float32), size=V)
    lg = lg.astype(np.float32)
    got, want = run_both([lg] * 10, dict(temperature=1.0, top_k=64, top_p=1.0, seed=12))
    assert got == want
    got, want = run_both([lg] * 3, dict(temperature=0.0))
    assert got == want


def test_fail_closed():
    V = 1000
    with Q.Sampler(V, temperature=0.7) as s:
        host = np.zeros(V, np.float32)
        host[5] = np.nan
        lg = D.to_dev(host)
        with pytest.raises(Q.QneError) as e:
            s.sample(lg.data_ptr())
        assert e.value.code == Q.EINVAL and "non-finite" in str(e.value)
        allowed = [i for i in range(V) if i != 5]
        assert s.sample(lg.data_ptr(), bitset(allowed, V), V) != 5  # NaN outside the mask is ignored
        host[5] = np.inf
        lg.upload(host)
        with pytest.raises(Q.QneError):
            s.sample(lg.data_ptr())
        lg.upload(np.full(V, -np.inf, np.float32))
        with pytest.raises(Q.QneError) as e:
            s.sample(lg.data_ptr())
        assert "no finite token" in str(e.value)
        with pytest.raises(Q.QneError):
            s.sample(D.zeros(V, np.float32).data_ptr(), bitset([], V), V)
    with pytest.raises(Q.QneError):
        Q.Sampler(V, top_k=1025)


def test_sampled_decode_through_the_model_matches_the_oracle():
    """Model::step with the logits left on the device and the device sampler picking every token,
    against the oracle sampler reading the same logits back: identical token streams."""
    index, buf = W.synth_model("tiny", seed=3, body="q4", head="f16")
    m = Q.Model.load(index, buf)
    try:
        prompt = np.random.default_rng(1).integers(0, m.vocab, size=12).astype(np.uint32)
        opts = dict(temperature=0.8, top_k=40, top_p=0.9, seed=77, presence_penalty=0.5)
        m.prefill_chunk(prompt, 0, True)
        o = OracleSampler(**opts)
        with Q.Sampler(m.vocab, **opts) as s:
            pos = len(prompt)
            for _ in range(30):
                want = o.sample(m.logits())
                tok = s.sample(m.logits_device())
                assert tok == want
                m.step_device(tok, pos)
                pos += 1
    finally:
        m.close()
