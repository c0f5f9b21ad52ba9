"""Decode throughput of the Qwen3.5-2B-shaped int4 hybrid decoder at batch 1, context 4096.

Workload (the reference's headline metric on this path): 28 layers [GDN, GDN, GDN, attention] x 7,
hidden 2048, 16 q / 4 kv heads of 256, GDN 16 heads x 128, intermediate 6144, vocab 151936;
int4 body (group 64, f16 scale + f16 zero), f16 embedding and LM head, weights N(0, 0.02) from a
seed; KV cache prefilled with 4000 random ids; then `--steps` greedy decode steps timed as one
GPU-resident submission (each step's pick is fed back on the device).

One step = one decode token. Prints one JSON line. The CPU baseline is the oracle's C
restatement (f32, OpenMP) timed on a bounded sample of the same workload: a few decode steps at
context 4000 with the KV cache and GDN state filled with random values.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "qwen-native-engine_amd"), str(ROOT / "oracle")]

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
PEAK_F32_TFLOPS = 157.3  # MI355X dense f32 MFMA


def algorithmic_bytes_per_token(cfg: dict, mats: dict, ctx: float) -> dict:
    """Bytes one decode token must move at least once, with no cache credit: every weight byte
    read once (embedding: one row), the KV cache over `ctx` positions plus the appended row, the
    GDN recurrent state read and written, the conv state read and written."""
    w = 0
    for name, m in mats.items():
        el = m["rows"] * m["k"]
        if name == "embed":
            el = m["k"]  # one row
        if m["dtype"] == "f16":
            w += el * 2
        else:
            w += el // 2 + 2 * (el // m["group"]) * 2  # nibbles + f16 scale + f16 zero
    lm = mats["lm_head"]["rows"] * mats["lm_head"]["k"] * 2 if mats["lm_head"]["dtype"] == "f16" else 0
    n_attn = sum(1 for i in range(cfg["layers"]) if (i + 1) % cfg["full_attention_every"] == 0)
    n_gdn = cfg["layers"] - n_attn
    kv_row = cfg["n_kv_heads"] * cfg["head_dim"] * 2 * 2  # K and V, f16
    kv = n_attn * kv_row * (ctx + 1)
    gdn = n_gdn * cfg["gdn_heads"] * cfg["gdn_dk"] * cfg["gdn_dv"] * 4 * 2
    conv_ch = 2 * cfg["gdn_heads"] * cfg["gdn_dk"] + cfg["gdn_heads"] * cfg["gdn_dv"]
    conv = n_gdn * conv_ch * (cfg["conv_kernel"] - 1) * 4 * 2
    return {"weights": w - lm, "lm_head": lm, "kv": kv, "gdn_state": gdn, "conv_state": conv,
            "total": w + kv + gdn + conv}


def cpu_baseline(index, buf, cfg, ctx, tokens):
    import cpu_oracle as O
    om = O.OracleModel(index, buf, "f32", max_context=4096)
    L = om.L
    rng = np.random.default_rng(1)
    n_attn = sum(1 for i in range(cfg["layers"]) if (i + 1) % cfg["full_attention_every"] == 0)
    n_gdn = cfg["layers"] - n_attn
    per = cfg["n_kv_heads"] * 4096 * cfg["head_dim"]
    for a in range(n_attn):
        for fn in (L.oc_state_kcache, L.oc_state_vcache):
            arr = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint16 * per).from_address(fn(om.state, a)))
            arr[:] = rng.normal(size=per).astype(np.float16).view(np.uint16)
    rec = cfg["gdn_heads"] * cfg["gdn_dk"] * cfg["gdn_dv"]
    for g in range(n_gdn):
        arr = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_float * rec).from_address(L.oc_state_recurrent(om.state, g)))
        arr[:] = rng.normal(0, 0.05, size=rec).astype(np.float32)
    om.token(1, ctx)  # warm caches and threads
    t0 = time.perf_counter()
    tok = 2
    for i in range(tokens):
        logits = om.token(tok, ctx + 1 + i)
        tok = int(np.argmax(logits))
    dt = time.perf_counter() - t0
    return tokens / dt, L.oc_num_threads()


TRAFFIC_PROFILE = ROOT / "profiles" / "k_decode_2b_int4_ctx4000_hbm_traffic.md"
TRAFFIC_PROFILE_08B = ROOT / "profiles" / "k_decode_08b_f16_ctx128_profile.md"
ATTN_TRAFFIC_PROFILE = ROOT / "profiles" / "paged_attention_b64_hbm_traffic.md"


def _profile_value(path, key):
    """A `key: value` line of a committed profile summary, or None."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


BATCH_PROFILE = ROOT / "profiles" / "batched_decode_2b_int4_b64_counters.md"


def profile_values(path) -> dict:
    """The `key: value` lines a profile summary ends with."""
    vals = {}
    try:
        text = path.read_text()
    except OSError:
        return vals
    for line in text.splitlines():
        if ":" in line and line.split(":", 1)[0].strip().replace("_", "").isalnum() and not line.startswith(("#", "|")):
            k, v = line.split(":", 1)
            try:
                vals[k.strip()] = float(v)
            except ValueError:
                pass
    return vals


def profiled_traffic(steps: int, profile=TRAFFIC_PROFILE):
    """HBM bytes of a `steps`-token decode launch from the FETCH_SIZE / WRITE_SIZE counter passes
    recorded in the profile summary (scaled by a plain copy of known size): the profiled launch's
    bytes per token times `steps`. A token moves the same bytes whatever the window length, except
    for the KV cache's growth with the context (under 0.1 % between a 20- and a 96-token window at
    context 4000). None without the profile."""
    try:
        text = profile.read_text()
    except OSError:
        return None
    vals = {}
    for line in text.splitlines():
        if line.startswith("traffic_") and ":" in line:
            k, v = line.split(":", 1)
            vals[k.strip()] = float(v)
    if "traffic_bytes_per_token" in vals:
        return vals["traffic_bytes_per_token"] * steps
    if vals.get("traffic_steps_per_launch", 0) <= 0 or "traffic_bytes_per_launch" not in vals:
        return None
    return vals["traffic_bytes_per_launch"] / vals["traffic_steps_per_launch"] * steps


def _events_ms(fn, warmup: int, iters: int):
    """Device time per call of fn(stream) from HIP events recorded on the stream it launches on."""
    import torch
    st = torch.cuda.Stream()
    h = st.cuda_stream
    for _ in range(warmup):
        fn(h)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn(h)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def bench_paged_attention(args) -> dict:
    """Paged-KV GQA decode: 16 q / 4 kv heads of 256, f16 K/V N(0, 1) in 16-token blocks behind a
    randomly permuted block table, `--batch` sequences with contexts uniform in [256, 4096], each
    call appending one token per sequence. Algorithmic bytes per call: K and V of every attended
    position (4096 B), the block-table entries, q, the new k/v and the output."""
    import torch
    import qne
    B, nq, nkv, hd, blk, maxb = args.batch, 16, 4, 256, 16, 256
    rng = np.random.default_rng(args.seed)
    ctx = rng.integers(256, 4096, size=B).astype(np.int32)
    pool = B * maxb
    dev = "cuda"
    bt = torch.from_numpy(rng.permutation(pool).astype(np.int32).reshape(B, maxb)).to(dev)
    kp = torch.randn(pool, nkv, blk, hd, dtype=torch.float16, device=dev)
    vp = torch.randn(pool, nkv, blk, hd, dtype=torch.float16, device=dev)
    q = torch.randn(B, nq, hd, device=dev)
    kn, vn = torch.randn(B, nkv, hd, device=dev), torch.randn(B, nkv, hd, device=dev)
    dctx = torch.from_numpy(ctx).to(dev)
    out = torch.empty(B, nq, hd, device=dev)

    def call(stream):
        qne.paged_attn_decode(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kp.data_ptr(), vp.data_ptr(), bt.data_ptr(),
                              maxb, dctx.data_ptr(), out.data_ptr(), B, nq, nkv, stream)

    ms = _events_ms(call, args.warmup, args.steps)
    # HBM bytes of the partial kernel from the committed counter passes, for this workload only
    traffic = _profile_value(ATTN_TRAFFIC_PROFILE, "traffic_bytes_per_call") if (B, args.seed) == (64, 0) else None
    pos = (ctx.astype(np.int64) + 1)
    nbytes = int(pos.sum()) * nkv * hd * 2 * 2 + int(((pos + blk - 1) // blk).sum()) * 4 + B * (2 * nq + 2 * nkv) * hd * 4
    gbs = nbytes / (ms / 1e3) / 1e9
    return {"metric": "paged attention decode GB/s (16q/4kv x 256, 16-token blocks)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": f"{B} sequences, contexts uniform in [256, 4096] (mean {float(ctx.mean()):.0f}), "
                                   f"one appended token each", "batch": B},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                         "traffic_source": ATTN_TRAFFIC_PROFILE.name if traffic else None,
                         "kernel": "k_kv_append + k_attn_partial + k_attn_combine", "bytes_per_step": nbytes},
            "cpu_baseline": None}


def bench_gemv(args) -> dict:
    """The standalone GEMV kernels (qne_gemv, the graph engine's per-matrix launches) on every
    matrix shape of one 2B decode token at batch 1: int4 g64 layer matrices (GDN and attention
    in-projections, out-projections, gate_up with the SwiGLU epilogue, down) and the f16 LM head.
    Each shape rotates over enough copies of its weights (>= 1 GiB) that the 256 MB MALL cannot
    serve them. Algorithmic bytes per call: nibbles + (scale, zero) pairs (or f16 rows), x and y.
    The aggregate weighs each shape by its launches per token (21 GDN and 7 attention layers)."""
    import torch
    import qne
    cfg = {"hidden": 2048, "inter": 6144, "vocab": 151936, "gdn": 2 * 16 * 128 * 2 + 2 * 16, "attn": 2 * 16 * 256 + 2 * 4 * 256}
    h, g64 = cfg["hidden"], 64
    shapes = [  # name, kind, rows, k, epilogue, launches per token
        ("gdn_in", qne.MAT_Q4, cfg["gdn"], h, qne.EPI_STORE, 21),
        ("attn_in", qne.MAT_Q4, cfg["attn"], h, qne.EPI_STORE, 7),
        ("gdn_out", qne.MAT_Q4, h, 16 * 128, qne.EPI_ACCUMULATE, 21),
        ("attn_out", qne.MAT_Q4, h, 16 * 256, qne.EPI_ACCUMULATE, 7),
        ("gate_up", qne.MAT_Q4, 2 * cfg["inter"], h, qne.EPI_SWIGLU, 28),
        ("down", qne.MAT_Q4, h, cfg["inter"], qne.EPI_ACCUMULATE, 28),
        ("lm_head", qne.MAT_F16, cfg["vocab"], h, qne.EPI_STORE, 1),
    ]
    gen = torch.Generator(device="cuda").manual_seed(args.seed)
    rows_out, tot_bytes, tot_ms = [], 0, 0.0
    for name, kind, rows, k, epi, per_tok in shapes:
        if kind == qne.MAT_Q4:
            wbytes = rows * k // 2 + rows * (k // g64) * 4
        else:
            wbytes = rows * k * 2
        copies = max(2, -(-(1 << 30) // wbytes))
        if kind == qne.MAT_Q4:
            w = torch.randint(-2**31, 2**31 - 1, (copies, rows, k // 8), dtype=torch.int32, device="cuda", generator=gen)
            sz = (torch.rand(copies, rows, k // g64, 2, device="cuda", generator=gen) * 0.02).half()
        else:
            w = (torch.randn(copies, rows, k, device="cuda", generator=gen) * 0.02).half()
            sz = None
        x = torch.randn(k, device="cuda", generator=gen)
        y = torch.zeros(rows // 2 if epi == qne.EPI_SWIGLU else rows, device="cuda")
        i = [0]

        def call(stream):
            c = i[0] % copies
            i[0] += 1
            qne.gemv(kind, w[c].data_ptr(), sz[c].data_ptr() if sz is not None else 0, rows, k, g64, x.data_ptr(),
                     y.data_ptr(), epi, stream=stream)

        ms = _events_ms(call, max(args.warmup, copies), max(args.steps, 2 * copies))
        nbytes = wbytes + k * 4 + y.numel() * 4 * (2 if epi == qne.EPI_ACCUMULATE else 1)
        rows_out.append({"matrix": name, "rows": rows, "k": k, "dtype": "q4 g64" if kind == qne.MAT_Q4 else "f16",
                         "us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms / 1e3) / 1e9, 1), "copies": copies})
        tot_bytes += nbytes * per_tok
        tot_ms += ms * per_tok
        del w, sz
        torch.cuda.empty_cache()
    gbs = tot_bytes / (tot_ms / 1e3) / 1e9
    return {"metric": "GEMV kernel GB/s (2B int4 decode matrices + f16 LM head, batch 1)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(tot_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32 accumulate, int4 / f16 weights", "data": "synthetic",
            "config": {"workload": "one decode token's GEMVs as standalone launches (21 GDN + 7 attention layers)"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "k_gemv (qne_gemv)",
                         "bytes_per_step": tot_bytes},
            "detail": rows_out, "cpu_baseline": None}


def bench_gdn(args) -> dict:
    """Gated delta rule, 16 heads, dk = dv = 128, f32 state; q, k L2-normalised N(0, 1), v N(0, 1),
    beta = sigmoid(N(0, 1)), decay g = exp(-softplus(N(0, 1))). (a) one recurrent step at batch 1, 8
    and 64: 133 128 B per (sequence, head) (state read + written, q, k, v, o). (b) 2048 tokens in one
    call at batch 4: 2048 B per (token, head) of q, k, v, o plus the state once per sequence."""
    import torch
    import torch.nn.functional as F
    import qne
    H, dk = 16, 128
    dev = "cuda"
    rng = np.random.default_rng(args.seed)

    def inputs(shape):
        t = lambda *s: torch.from_numpy(rng.normal(size=s).astype(np.float32)).to(dev)
        q, k = F.normalize(t(*shape, dk), dim=-1), F.normalize(t(*shape, dk), dim=-1)
        v = t(*shape, dk)
        beta = torch.sigmoid(t(*shape))
        g = torch.exp(-F.softplus(t(*shape)))
        return q, k, v, beta, g

    steps = {}
    for B in (1, 8, 64):
        q, k, v, beta, g = inputs((B, H))
        # successive calls rotate over states totalling at least 512 MiB (above the 256 MB
        # last-level cache), so every call reads its state from HBM
        nst = max(2, min(512, (512 << 20) // (B * H * dk * dk * 4)))
        S = torch.zeros(nst, B, H, dk, dk, device=dev)
        o = torch.empty(B, H, dk, device=dev)
        turn = [0]

        def step_call(st):
            Si = S[turn[0] % nst]
            turn[0] += 1
            qne.gdn_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), g.data_ptr(), Si.data_ptr(),
                         o.data_ptr(), B, H, st)

        ms = _events_ms(step_call, args.warmup, args.steps)
        nb = B * H * 133128
        steps[B] = {"ms": round(ms, 4), "GB/s": round(nb / (ms / 1e3) / 1e9, 1)}
    B, T = 4, 2048
    q, k, v, beta, g = inputs((B, T, H))
    S = torch.zeros(B, H, dk, dk, device=dev)
    o = torch.empty(B, T, H, dk, device=dev)
    ms = _events_ms(lambda st: qne.gdn_prefill_chunked(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                                                       g.data_ptr(), S.data_ptr(), o.data_ptr(), B, T, H, st),
                    1, max(1, args.steps // 20))
    nb = B * T * H * 2048 + B * H * dk * dk * 4 * 2
    # flops: the sequential-equivalent convention (6 dk dv = 98 304 per token and head), and the MFMA
    # flops the chunk-64 WY form issues (f32 16x16x4 tiles, triangular tiles skipped): per chunk and
    # head 1344 in the prep kernel (K K^T, K Q^T, T off-diagonal blocks, U, W^T) and 8 x 424 in
    # the chain (D, output, state), 2048 flops each
    chunks = B * H * ((T + 63) // 64)
    seq_flop = B * T * H * 98304
    wy_flop = chunks * (1344 + 8 * 424) * 2048
    pre = {"ms": round(ms, 3), "GB/s": round(nb / (ms / 1e3) / 1e9, 1), "tokens_per_s": round(B * T / (ms / 1e3)),
           "form": "chunk-64 WY on f32 MFMA", "seq_equiv_tflops": round(seq_flop / (ms / 1e3) / 1e12, 2),
           "mfma_tflops": round(wy_flop / (ms / 1e3) / 1e12, 2),
           "mfma_frac_f32": round(wy_flop / (ms / 1e3) / 1e12 / PEAK_F32_TFLOPS, 4)}
    gbs = steps[64]["GB/s"]
    return {"metric": "gated delta rule GB/s (16 heads x 128 x 128 state), step at batch 64", "value": gbs,
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": steps[64]["ms"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "recurrent step at batch 1/8/64; 2048-token prefill at batch 4", "batch": 64},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "k_delta_rule",
                         "bytes_per_step": 64 * H * 133128},
            "detail": {"step": steps, "prefill_b4_t2048": pre}, "cpu_baseline": None}


def bench_sample(args) -> dict:
    """Sampled decode (src/sampling.rs Sampler: temperature 0.6, top-k 20, top-p 0.95, presence
    penalty 1.5, the agent's defaults plus a penalty) on the 2B model after a ctx-token prefill:
    the reference's path reads vocab x 4 B of logits back per token and samples on the host (here
    the oracle's C restatement of its sampler, one thread); the device path leaves the logits in HBM
    and runs the O(vocab) part of the sampler on the GPU (qne_step_device + qne_sample), reading
    back only the k best (value, token) pairs. Both paths must produce the same tokens."""
    import torch
    import qne
    import weights as W
    from cpu_oracle import OracleSampler
    # torch's HIP runtime (the event timer below) must be initialised before the library's
    torch.zeros(1, device="cuda")
    opts = dict(temperature=0.6, top_k=20, top_p=0.95, seed=42, presence_penalty=1.5)
    cfg = W.full_config("2b")
    index, buf = W.synth_model("2b", seed=args.seed, body="q4", head="f16", group=64)
    m = qne.Model.load(index, buf, options={"max_context": 4096})
    V = cfg["vocab"]
    prompt = np.random.default_rng(args.seed).integers(0, V, size=args.ctx).astype(np.uint32)
    steps = min(args.steps, 4096 - args.ctx - 1)
    for s0 in range(0, args.ctx, 512):
        m.prefill_chunk(prompt[s0: min(s0 + 512, args.ctx)], s0, s0 + 512 >= args.ctx)
    m.snapshot()
    first, _ = m.last_token()

    def host_path():
        m.restore()
        o = OracleSampler(**opts)
        toks, tok, pos = [], first, args.ctx
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = o.sample(m.step(tok, pos))
            toks.append(tok)
            pos += 1
        return toks, time.perf_counter() - t0

    def device_path():
        m.restore()
        toks, tok, pos = [], first, args.ctx
        with qne.Sampler(V, **opts) as smp:
            ptr = m.logits_device()
            t0 = time.perf_counter()
            for _ in range(steps):
                m.step_device(tok, pos)
                tok = smp.sample(ptr)
                toks.append(tok)
                pos += 1
            return toks, time.perf_counter() - t0

    host_path()
    device_path()  # warm
    host_toks, host_s = host_path()
    dev_toks, dev_s = device_path()
    # the sampler kernel alone: HIP events around repeated calls on one stream over the model's logits
    kernel = {}
    for name, o in (("top_k_20", opts), ("top_k_1024", dict(opts, top_k=1024)), ("greedy", dict(temperature=0.0))):
        with qne.Sampler(V, **o) as smp:
            ptr = m.logits_device()
            ms = _events_ms(lambda s_: smp.sample(ptr, stream=s_), 5, 50)
        kernel[name] = round(ms * 1e3, 1)
    m.close()
    step_ms = dev_s / steps * 1e3
    return {"metric": "sampled decode tok/s (2B int4, ctx %d, device sampler)" % args.ctx,
            "value": round(steps / dev_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": steps,
            "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32", "data": "synthetic",
            "config": {"workload": "2B-shaped int4 decoder, one sequence, sampled with temperature 0.6, top-k 20, "
                                   "top-p 0.95, presence penalty 1.5 after a %d-token prefill" % args.ctx},
            "roofline": None,
            "detail": {"identical_tokens": host_toks == dev_toks, "device_path_ms_per_token": round(step_ms, 4),
                       "host_sampling_path_ms_per_token": round(host_s / steps * 1e3, 4),
                       "readback_bytes_per_token": {"host_path": V * 4, "device_path": 16 + 20 * 8},
                       "sampler_call_us": kernel},
            "cpu_baseline": {"value": round(steps / host_s, 2), "unit": "tok/s", "cores": 1, "kind": "port",
                             "sample": "the same decode with the logits read back and sampled by the oracle's C "
                                       "restatement of src/sampling.rs on one host thread"}}


def bench_batch(args) -> dict:
    """Batched continuous decode on the 2B-shaped int4 model: `--batch` sequences (64) with contexts
    uniform in [256, 4096) on the paged KV cache, all advancing one greedy token per step (each
    row's pick fed back on the device). KV contents and recurrent state are pseudo-random (a fill
    kernel), so no prefill is needed. Algorithmic bytes per step: every weight once (the embedding:
    one row per sequence), each sequence's K and V over its attended positions, GDN and conv state
    read and written per sequence. MFMA work: every GEMM runs two f16 MFMA passes (x split into hi
    and lo halves) over 64 rows."""
    import qne
    import weights as W
    cfg = W.full_config("2b")
    t = time.perf_counter()
    index, buf = W.synth_model("2b", seed=args.seed, body="q4", head="f16", group=64)
    mats = json.loads(index)["matrices"]
    gen_s = time.perf_counter() - t
    m = qne.Model.load(index, buf, options={"max_context": 4096, "engine": "graph"})
    B = args.batch
    rng = np.random.default_rng(args.seed)
    ctx = rng.integers(256, 4096 - args.steps - args.warmup - 1, size=B).astype(np.uint32)
    b = qne.Batch(m, B, 4096)
    b.fill_synthetic(ctx, seed=args.seed)
    if args.warmup:
        b.decode(B, args.warmup)
    _, pos0 = b.row_state(B)
    t0 = time.perf_counter()
    ids = b.decode(B, args.steps)
    wall = time.perf_counter() - t0
    dev_ms, dev_steps = b.last_decode_timing()
    assert dev_steps == args.steps and ids.shape == (args.steps, B)
    tok_s = B * args.steps / wall
    # bytes per step: weights once; per sequence its KV (mean position over the window), GDN, conv
    one = algorithmic_bytes_per_token(cfg, mats, 0.0)
    embed_row = mats["embed"]["k"] * 2
    mean_pos = float(pos0.astype(np.float64).mean()) + (args.steps - 1) / 2
    kv_row = cfg["n_kv_heads"] * cfg["head_dim"] * 2 * 2
    n_attn = sum(1 for i in range(cfg["layers"]) if (i + 1) % cfg["full_attention_every"] == 0)
    kv = B * n_attn * kv_row * (mean_pos + 1)
    weights = one["weights"] - embed_row + one["lm_head"] + B * embed_row
    per_step = weights + kv + B * (one["gdn_state"] + one["conv_state"])
    achieved = per_step / (dev_ms / args.steps / 1e3) / 1e9
    # HBM bytes and MFMA busy cycles per step from the counter passes of this workload (64 rows)
    prof = profile_values(BATCH_PROFILE) if B == 64 else {}
    traffic = prof.get("traffic_bytes_per_step")
    busy = prof.get("mfma_busy_simd_cycles_per_step")
    macs = sum(mm["rows"] * mm["k"] for name, mm in mats.items() if name != "embed")
    mfma_flops = 2 * 2 * 64 * macs  # hi and lo passes over 64 rows
    mfma_tflops = mfma_flops / (dev_ms / args.steps / 1e3) / 1e12
    result = {
        "metric": "batched decode tok/s (64 sequences, 2B int4, ctx U[256,4096]) + % of HBM roofline",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 activations, f16 MFMA (x as hi + lo f16), int4 weights", "data": "synthetic",
        "config": {"workload": f"Qwen3.5-2B-shaped hybrid decoder, int4 g64 body, f16 embed/lm_head, {B} sequences "
                               f"with contexts uniform in [256, 4096) (mean {float(pos0.mean()):.0f}), one greedy "
                               f"token per sequence per step", "batch": B, "layers": cfg["layers"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": BATCH_PROFILE.name if traffic else None,
                     "kernel": "batched decode step (HIP graph: GEMMs, GDN, attention)",
                     "bytes_per_step": int(per_step), "device_ms_per_step": round(dev_ms / args.steps, 4)},
        "mfma": {"flops_per_step": mfma_flops, "achieved_tflops_over_step": round(mfma_tflops, 1),
                 "peak_tflops_f16": 2500.0, "frac_over_step": round(mfma_tflops / 2500.0, 4),
                 # counter-based: busy SIMD-cycles of the MFMA pipes over the step's device time
                 "busy_frac_over_step": round(busy / (dev_ms / args.steps / 1e3 * 2.4e9 * 1024), 4) if busy else None,
                 "busy_source": BATCH_PROFILE.name if busy else None},
        "detail": {"bytes_per_step": {"weights": int(weights), "kv": int(kv),
                                      "gdn_state": int(B * one["gdn_state"]), "conv_state": int(B * one["conv_state"])},
                   "weights_gen_s": round(gen_s, 2), "adapter": m.adapter},
    }
    if not args.no_cpu_baseline:
        mean_ctx = int(pos0.mean())
        v, cores = cpu_baseline(index, buf, cfg, mean_ctx, 2)
        result["cpu_baseline"] = {"value": round(v, 4), "unit": "tok/s", "cores": cores, "kind": "port",
                                  "sample": f"2 greedy decode steps of one sequence of the same model at context "
                                            f"{mean_ctx} (the batch's mean; KV cache and GDN state random), oracle C "
                                            f"restatement, f32, OpenMP; the oracle decodes one sequence at a time"}
    else:
        result["cpu_baseline"] = None
    b.close()
    m.close()
    return result


class _Hip:
    """The few HIP runtime calls the probes need, through the runtime libqne.so itself links."""

    def __init__(self):
        import ctypes
        import qne
        qne.load_library()
        h = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        for name, args in (("hipMalloc", [ctypes.POINTER(vp), sz]), ("hipFree", [vp]),
                           ("hipMemcpy", [vp, vp, sz, ctypes.c_int]), ("hipMemsetD32", [vp, ctypes.c_int, sz]),
                           ("hipDeviceSynchronize", []), ("hipEventCreate", [ctypes.POINTER(vp)]),
                           ("hipEventRecord", [vp, vp]), ("hipEventSynchronize", [vp]),
                           ("hipEventElapsedTime", [ctypes.POINTER(ctypes.c_float), vp, vp])):
            f = getattr(h, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        self.h, self.ct = h, ctypes

    def ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def malloc(self, n):
        p = self.ct.c_void_p()
        self.ck(self.h.hipMalloc(self.ct.byref(p), n), "hipMalloc")
        return p.value

    def free(self, p):
        self.h.hipFree(p)

    def upload(self, p, a, off=0):
        self.ck(self.h.hipMemcpy(p + off, a.ctypes.data, a.nbytes, 1), "hipMemcpy")

    def copy(self, dst, src, n):
        self.ck(self.h.hipMemcpy(dst, src, n, 3), "hipMemcpy")

    def fill32(self, p, v, n_words):
        self.ck(self.h.hipMemsetD32(p, v, n_words), "hipMemsetD32")

    def sync(self):
        self.ck(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def timed(self, fn, n):
        """Device ms per call of fn() (HIP events on the null stream, which fn launches on)."""
        a, b = self.ct.c_void_p(), self.ct.c_void_p()
        self.h.hipEventCreate(self.ct.byref(a))
        self.h.hipEventCreate(self.ct.byref(b))
        self.h.hipEventRecord(a, None)
        for _ in range(n):
            fn()
        self.h.hipEventRecord(b, None)
        self.h.hipEventSynchronize(b)
        ms = self.ct.c_float()
        self.h.hipEventElapsedTime(self.ct.byref(ms), a, b)
        return ms.value / n


def bench_stream(args) -> dict:
    """The reference's two probes on MI355X: the streaming-read bandwidth probe (bandwidth_probe,
    kernels/src/lib.rs:837-863: 64 MB and 400 MB buffers, constant and random data, three runs each)
    and the fixed cost of one dispatch (dispatch_cost, lib.rs:718-724: 2000 no-op dispatches). A
    4 GiB buffer is added: 64 MB fits the 256 MB MALL, 400 MB mostly does not, and 4 GiB measures
    HBM alone. `value` is the 4 GiB random-data read rate: the achievable ceiling a streaming
    kernel (the GEMV, the LM head) can be held against."""
    import qne
    hip = _Hip()
    lib = qne.load_library()
    groups = args.stream_workgroups
    sink = hip.malloc(groups * 256 * 4)
    rng = np.random.default_rng(args.seed)
    block = rng.integers(0, 2**32, size=(64 << 20) // 4, dtype=np.uint32)
    runs = []
    for mb in (64, 400, 4096):
        n = mb << 20
        data = hip.malloc(n)
        for random in (False, True):
            if random:
                hip.upload(data, block)
                for off in range(64 << 20, n, 64 << 20):
                    hip.copy(data + off, data, min(64 << 20, n - off))
            else:
                hip.fill32(data, 0x12345678, n // 4)
            hip.sync()
            call = lambda: lib.qne_stream_read(data, n, sink, groups, None)
            hip.timed(call, 2)
            repeat = 20 if mb <= 100 else 5 if mb <= 1000 else 3
            for run in range(3):
                ms = hip.timed(call, repeat)
                runs.append({"mb": mb, "data": "random" if random else "constant", "run": run,
                             "GB/s": round(n / (ms / 1e3) / 1e9, 1)})
        hip.free(data)
    y = hip.malloc(256)
    hip.fill32(y, 0, 64)
    noop = lambda: lib.qne_noop_dispatch(y, None)
    hip.timed(noop, 10)
    n_disp = 2000
    t0 = time.perf_counter()
    dev_ms = hip.timed(noop, n_disp)
    host_us = (time.perf_counter() - t0) * 1e6 / n_disp
    hip.free(y)
    hip.free(sink)
    best = max(r["GB/s"] for r in runs if r["mb"] == 4096 and r["data"] == "random")
    return {"metric": "streaming read GB/s (16-byte non-temporal loads, 4 GiB random data)", "value": best,
            "unit": "GB/s", "n_gpus": 1, "steps": 3, "warmup": 2, "ms_per_step": round((4096 << 20) / best / 1e6, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32", "data": "synthetic",
            "config": {"workload": "read 64 MB / 400 MB / 4 GiB once, constant and random data; 2000 no-op dispatches",
                       "workgroups": groups, "threads_per_workgroup": 256},
            "roofline": {"bound": "hbm", "achieved": best, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(best / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "k_stream_read"},
            "detail": {"stream": runs, "dispatch_us_device": round(dev_ms * 1e3, 3),
                       "dispatch_us_host": round(host_us, 3), "dispatches": n_disp},
            "cpu_baseline": None}


def bench_exchange(args) -> dict:
    """The hand-over probe (qne_exchange_probe): the all-to-all exchange of a tagged 2048-value
    vector that every phase of the persistent decode kernel pays, without its compute or its weight
    stream, at 8 / 32 / 64 / 128 / 256 co-resident workgroups (256: one per CU, the decode
    kernel's grid). `value` is the time of one exchange round at 256 workgroups. For scale, the
    first line is two workgroups exchanging one value each (a store seen by one other poller)."""
    import ctypes
    import qne
    hip = _Hip()
    lib = qne.load_library()
    n, rounds = 2048, 2002
    buf = hip.malloc(2 * n * 8)
    ctl = hip.malloc(64)
    runs = []
    for wgs, nv in ((2, 2), (8, n), (32, n), (64, n), (128, n), (256, n)):
        for rep in range(2):
            hip.fill32(buf, 0, 2 * n * 2)
            us = ctypes.c_double()
            hip.ck(lib.qne_exchange_probe(buf, nv, rounds, wgs, ctl, ctypes.byref(us)), "qne_exchange_probe")
            runs.append({"workgroups": wgs, "values": nv, "rep": rep, "us_per_round": round(us.value, 3)})
    hip.free(buf)
    hip.free(ctl)
    best = min(r["us_per_round"] for r in runs if r["workgroups"] == 256)
    return {"metric": "hand-over round us (256 workgroups, 2048-value tagged vector)", "value": best, "unit": "us",
            "n_gpus": 1, "steps": rounds - 2, "warmup": 2, "ms_per_step": round(best / 1e3, 6), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "all-to-all exchange of a 2048-value tagged vector, 2000 rounds",
                       "threads_per_workgroup": 512},
            "roofline": None, "detail": {"runs": runs}, "cpu_baseline": None}


def bench_prefill(args) -> dict:
    """Chunked prefill of the 2B-shaped int4 model (Model::prefill_chunk, kernels/src/model.rs:
    349-372, in its prefill_batched form: the whole prompt in one call): a `--ctx`-id prompt (4000),
    which the library runs in passes of up to 2048 tokens, each pass the batched MFMA GEMMs over its
    tokens, the GDN recurrence in its WY form and causal attention over the cache; the call ends with
    the logits. One untimed prefill first (it captures the pass graphs), then the timed one from a
    reset state. MFMA work: every body GEMM runs two f16 MFMA passes (x split into hi and lo halves)
    over every token; the weights stream once per pass."""
    import qne
    import weights as W
    cfg = W.full_config("2b")
    index, buf = W.synth_model("2b", seed=args.seed, body="q4", head="f16", group=64)
    mats = json.loads(index)["matrices"]
    m = qne.Model.load(index, buf, options={"max_context": 4096, "prefill_graphs": not args.prefill_direct})
    n = args.ctx
    prompt = np.random.default_rng(args.seed).integers(0, cfg["vocab"], size=n).astype(np.uint32)

    def run():
        m.reset()
        m.prefill_chunk(prompt, 0, True)

    run()
    t0 = time.perf_counter()
    run()  # prefill_chunk returns after its stream has drained
    wall = time.perf_counter() - t0
    body = sum(mm["rows"] * mm["k"] for name, mm in mats.items() if name not in ("embed", "lm_head"))
    mfma_flops = 2 * 2 * n * body  # hi and lo passes over every token
    passes = (n + 2047) // 2048
    one = algorithmic_bytes_per_token(cfg, mats, 0.0)
    result = {
        "metric": f"chunked prefill tok/s ({n}-id prompt, 2B int4)", "value": round(n / wall, 1), "unit": "tok/s",
        "n_gpus": 1, "prefill_s": round(wall, 4), "higher_is_better": True, "dtype": "f32 activations, f16 MFMA "
        "(x as hi + lo f16), int4 weights", "data": "synthetic",
        "config": {"workload": f"Qwen3.5-2B-shaped hybrid decoder, int4 g64 body, {n}-id prompt in one "
                               f"prefill_chunk call (passes of up to 2048 tokens)",
                   "prefill_graphs": not args.prefill_direct},
        "mfma": {"gemm_flops": mfma_flops, "achieved_tflops_over_prefill": round(mfma_flops / wall / 1e12, 1),
                 "peak_tflops_f16": 2500.0, "frac_over_prefill": round(mfma_flops / wall / 1e12 / 2500.0, 4)},
        "detail": {"passes": passes, "weight_bytes_per_pass": int(one["weights"]), "adapter": m.adapter},
    }
    m.close()
    return result


def copy_calibration(mib: int) -> None:
    """A plain device-to-device copy of a known size: under a hardware-counter profiler its
    FETCH_SIZE / WRITE_SIZE readings per dispatch, divided into the bytes it must move, give the
    scale factor applied to the decode kernel's readings."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "dispatches": 3}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed decode steps (default 96; 128 for --config 0.8b)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps, run as one window (default: as many as --steps, so that "
                         "every decode window a profile sees has the timed length)")
    ap.add_argument("--ctx", type=int, default=None, help="prompt length (default 4000; 128 for --config 0.8b)")
    ap.add_argument("--config", default="2b",
                    help="2b (the decode benchmark), 0.8b (f16 weights, 128-id prompt, 128 steps), batch "
                         "(64-sequence batched decode), prefill (4000-id chunked prefill), sample (sampled decode with the device sampler), stream "
                         "(the read-bandwidth and dispatch-cost probes), exchange (the decode kernel's hand-over "
                         "probe), or the kernel microbenches attn / gdn / gemv")
    ap.add_argument("--batch", type=int, default=64, help="sequences (--config attn / batch)")
    ap.add_argument("--stream-workgroups", type=int, default=2048, help="workgroups of the --config stream probe")
    ap.add_argument("--cpu-tokens", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill", default="chunk", choices=["chunk", "tokens"],
                    help="fill the context with prefill_chunk (batched GEMM passes, the default) or with "
                         "prefill (the persistent token kernel)")
    ap.add_argument("--prefill-direct", action="store_true",
                    help="--config prefill: launch each pass's kernels one by one instead of replaying its graph")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--engine", default="persistent", choices=["persistent", "graph"])
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (scales the HBM byte counters)")
    args = ap.parse_args()
    small = args.config == "0.8b"
    if args.steps is None:
        args.steps = 128 if small else 96
    if args.ctx is None:
        args.ctx = 128 if small else 4000
    if args.warmup is None:
        args.warmup = args.steps
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.config in ("attn", "gdn", "gemv"):
        sys.path[:0] = [str(ROOT / "qwen-native-engine_amd")]
        fn = {"attn": bench_paged_attention, "gdn": bench_gdn, "gemv": bench_gemv}[args.config]
        print(json.dumps(fn(args)))
        return
    if args.config == "batch":
        print(json.dumps(bench_batch(args)))
        return
    if args.config == "prefill":
        print(json.dumps(bench_prefill(args)))
        return
    if args.config == "stream":
        sys.path[:0] = [str(ROOT / "qwen-native-engine_amd")]
        print(json.dumps(bench_stream(args)))
        return
    if args.config == "exchange":
        sys.path[:0] = [str(ROOT / "qwen-native-engine_amd")]
        print(json.dumps(bench_exchange(args)))
        return
    if args.config == "sample":
        sys.path[:0] = [str(ROOT / "qwen-native-engine_amd")]
        print(json.dumps(bench_sample(args)))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this engine runs batch-1 decode on one GPU; --gpus above 1 is not supported "
              "(the decode path is measured on one GPU only)", file=sys.stderr)
        sys.exit(2)
    import qne
    import weights as W

    cfg = W.full_config(args.config)
    t = time.perf_counter()
    # the 0.8B configuration has f16 weights throughout, the 2B one an int4 g64 body
    body = "f16" if small else "q4"
    index, buf = W.synth_model(args.config, seed=args.seed, body=body, head="f16", group=64)
    mats = json.loads(index)["matrices"]
    gen_s = time.perf_counter() - t
    m = qne.Model.load(index, buf, options={"max_context": 4096, "engine": args.engine})
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, cfg["vocab"], size=args.ctx).astype(np.uint32)
    t = time.perf_counter()
    ctx_timed = args.ctx
    if args.prefill == "tokens":
        # the whole prompt through the persistent token kernel (Model::prefill, model.rs:324); the
        # warmup window then runs at ctx and the timed one right after it
        assert args.ctx + args.warmup + args.steps <= 4096, "context + warmup + steps must fit in 4096"
        m.prefill(prompt)
        prefill_s = time.perf_counter() - t
        if args.warmup:
            m.decode(args.warmup + 1, args.warmup, [])
        ctx_timed = args.ctx + args.warmup
    else:
        assert args.ctx + max(args.steps, args.warmup) <= 4096, "context + steps must fit in 4096"
        for s in range(0, args.ctx - 1, 512):
            m.prefill_chunk(prompt[s: min(s + 512, args.ctx - 1)], s, False)
        prefill_s = time.perf_counter() - t
        # Snapshot after ctx - 1 tokens. The last prompt token is replayed before each decode run
        # to set the greedy pick and position, which snapshot/restore do not cover
        # (model.rs:394-414).
        m.snapshot()
        if args.warmup:
            m.prefill_chunk(prompt[-1:], args.ctx - 1, True)
            m.decode(args.warmup + 1, args.warmup, [])
            m.restore()
        m.prefill_chunk(prompt[-1:], args.ctx - 1, True)
    # decode() returns after its stream has drained, so the wall clock brackets the device work
    t0 = time.perf_counter()
    ids = m.decode(args.steps + 1, args.steps, [])
    wall = time.perf_counter() - t0
    dev_ms, dev_steps = m.last_decode_timing()
    assert dev_steps == args.steps and len(ids) == args.steps + 1
    tok_s = args.steps / wall
    bytes_tok = algorithmic_bytes_per_token(cfg, mats, ctx_timed + (args.steps - 1) / 2)
    # one k_decode launch covers the whole timed window: bytes per launch / launch duration
    achieved = bytes_tok["total"] * args.steps / (dev_ms / 1e3) / 1e9
    if args.config == "2b" and args.ctx == 4000:
        traffic_profile = TRAFFIC_PROFILE
    elif args.config == "0.8b" and args.ctx == 128:
        traffic_profile = TRAFFIC_PROFILE_08B
    else:
        traffic_profile = None
    traffic = profiled_traffic(args.steps, traffic_profile) if traffic_profile else None
    result = {
        "metric": ("decode tok/s @ batch 1, 0.8B f16, 128-id prompt" if small else
                   "decode tok/s @ batch 1, ctx 4096 (2B int4) + % of HBM roofline"),
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"Qwen3.5-{args.config.upper()}-shaped hybrid decoder, "
                               f"{'f16' if small else 'int4 g64'} body, f16 embed/lm_head, "
                               f"batch 1 greedy decode after a {args.ctx}-token prefill"
                               + (" (token kernel)" if args.prefill == "tokens" else ""),
                   "layers": cfg["layers"], "hidden": cfg["hidden"], "vocab": cfg["vocab"], "ctx": args.ctx,
                   "batch": 1, "window": args.steps},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_profile.name if traffic else None,
                     "kernel": f"k_decode, one launch per {args.steps}-token window"
                               if args.engine == "persistent" else
                               f"decode step ({m.dispatches_per_token()} kernels per token)",
                     "bytes_per_launch": bytes_tok["total"] * args.steps, "bytes_per_step": bytes_tok["total"],
                     "device_ms_per_launch": round(dev_ms, 3), "device_ms_per_step": round(dev_ms / args.steps, 4)},
        "detail": {"bytes_per_token": bytes_tok, "weights_gen_s": round(gen_s, 2),
                   "context_fill_s": round(prefill_s, 2),
                   "context_fill": (f"{args.ctx - 1} ids through Model::prefill, untimed set-up" if args.prefill == "tokens"
                                    else f"{args.ctx - 1} ids in 512-id prefill_chunk calls, each the first of its "
                                         "shape (pass graphs instantiated), untimed set-up; the prefill rate is "
                                         "bench.py --config prefill"),
                   "adapter": m.adapter},
    }
    if args.engine == "persistent" and args.prefill != "tokens":
        # the token's dependent phases: one profiled token (not timed) from the prompt state, since
        # the timed window may have filled the context
        m.restore()
        m.prefill_chunk(prompt[-1:], args.ctx - 1, True)
        nph = len(m.profile_token_detail()["phases"])
        result["detail"]["phases_per_token"] = nph
        result["detail"]["device_us_per_phase"] = round(dev_ms / args.steps * 1e3 / nph, 3)
    if not args.no_cpu_baseline:
        v, cores = cpu_baseline(index, buf, cfg, args.ctx, args.cpu_tokens)
        result["cpu_baseline"] = {"value": round(v, 4), "unit": "tok/s", "cores": cores, "kind": "port",
                                  "sample": f"{args.cpu_tokens} greedy decode steps of the same model at context "
                                            f"{args.ctx} (KV cache and GDN state filled with random values), "
                                            f"oracle C restatement, f32, OpenMP"}
    else:
        result["cpu_baseline"] = None
    m.close()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
