"""ctypes binding of the CPU oracle (liboracle_f32.so / liboracle_f64.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker (or the timed CPU restatement). The product never loads it.
"""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OC_F16, OC_Q4G, OC_Q4V1 = 0, 1, 2
STORE, ACCUMULATE, SWIGLU = 0, 1, 2


class Mat(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("rows", ctypes.c_int32), ("k", ctypes.c_int32), ("group", ctypes.c_int32),
                ("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("z", ctypes.c_void_p)]


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("hidden", "layers", "full_attention_every", "intermediate", "vocab",
                                               "n_q_heads", "n_kv_heads", "head_dim", "rope_dim", "gdn_heads",
                                               "gdn_dk", "gdn_dv", "conv_kernel", "max_context")] + \
               [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)]


class Layer(ctypes.Structure):
    _fields_ = [("mixer_in", Mat), ("mixer_out", Mat), ("gate_up", Mat), ("down", Mat),
                ("input_norm", ctypes.c_void_p), ("post_norm", ctypes.c_void_p), ("attn_norms", ctypes.c_void_p),
                ("conv_w", ctypes.c_void_p), ("gdn_params", ctypes.c_void_p)]


class ModelS(ctypes.Structure):
    _fields_ = [("c", Config), ("embed", Mat), ("lm_head", Mat), ("final_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(Layer))]


_libs = {}


def lib(precision: str = "f64"):
    if precision not in _libs:
        p = HERE / f"liboracle_{precision}.so"
        if not p.exists():
            raise RuntimeError(f"{p} not built; run make -C {HERE}")
        L = ctypes.CDLL(str(p))
        vp = ctypes.c_void_p
        L.oc_f16_to_f32.argtypes = [ctypes.c_uint16]; L.oc_f16_to_f32.restype = ctypes.c_float
        L.oc_f32_to_f16.argtypes = [ctypes.c_float]; L.oc_f32_to_f16.restype = ctypes.c_uint16
        L.oc_dequant_row.argtypes = [ctypes.POINTER(Mat), ctypes.c_int, vp]
        L.oc_gemv.argtypes = [ctypes.POINTER(Mat), vp, vp, ctypes.c_int]
        L.oc_rmsnorm.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_float]
        L.oc_embed.argtypes = [ctypes.POINTER(Mat), ctypes.c_uint32, vp]
        L.oc_argmax.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_float)]
        L.oc_rope_inv_freq.argtypes = [ctypes.c_int, ctypes.c_float, vp]
        L.oc_gdn_step.argtypes = [ctypes.POINTER(Config), vp, vp, vp, vp, vp, vp]
        L.oc_attention_step.argtypes = [ctypes.POINTER(Config), vp, vp, vp, ctypes.c_uint32, vp, vp]
        L.oc_delta_rule.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_float, ctypes.c_float, vp, vp]
        L.oc_attn_dense.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int,
                                    ctypes.c_float, vp]
        L.oc_state_new.argtypes = [ctypes.POINTER(ModelS)]; L.oc_state_new.restype = vp
        L.oc_state_free.argtypes = [vp]
        L.oc_reset.argtypes = [vp]
        L.oc_token.argtypes = [ctypes.POINTER(ModelS), vp, ctypes.c_uint32, ctypes.c_uint32, vp]
        L.oc_prefill_chunk.argtypes = [ctypes.POINTER(ModelS), vp, vp, ctypes.c_int, ctypes.c_uint32, ctypes.c_int, vp]
        L.oc_copy_state.argtypes = [vp, vp]
        for n in ("oc_state_recurrent", "oc_state_conv", "oc_state_kcache", "oc_state_vcache"):
            getattr(L, n).argtypes = [vp, ctypes.c_int]
            getattr(L, n).restype = vp
        L.oc_num_threads.restype = ctypes.c_int
        L.oc_sampler_seed.argtypes = [ctypes.c_uint64]; L.oc_sampler_seed.restype = ctypes.c_uint64
        L.oc_sampler_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]; L.oc_sampler_next_f32.restype = ctypes.c_float
        L.oc_sample.argtypes = [vp, ctypes.c_uint32, vp, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint32, ctypes.c_float,
                                ctypes.c_float, ctypes.POINTER(ctypes.c_uint64), vp, ctypes.POINTER(ctypes.c_uint32)]
        L.oc_sample.restype = ctypes.c_int
        _libs[precision] = L
    return _libs[precision]


def ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def config_struct(cfg: dict, max_context: int = 4096) -> Config:
    c = Config()
    for n in ("hidden", "layers", "full_attention_every", "intermediate", "vocab", "n_q_heads", "n_kv_heads",
              "head_dim", "rope_dim", "gdn_heads", "gdn_dk", "gdn_dv", "conv_kernel"):
        setattr(c, n, int(cfg[n]))
    c.max_context = max_context
    c.rope_theta = float(cfg["rope_theta"])
    c.eps = float(cfg.get("rms_eps", 1e-6))
    return c


def mat_struct(m: dict | None, kind: int, rows: int, k: int, group: int, w, s=None, z=None) -> Mat:
    out = Mat()
    out.kind, out.rows, out.k, out.group = kind, rows, k, group
    out.w = w.ctypes.data if w is not None else None
    out.s = s.ctypes.data if s is not None else None
    out.z = z.ctypes.data if z is not None else None
    out._keep = (w, s, z)  # the struct holds raw pointers: keep the arrays alive with it
    return out


V1_CONFIG = dict(n_q_heads=8, n_kv_heads=2, head_dim=256, gdn_heads=16, gdn_dk=128, gdn_dv=128, conv_kernel=4,
                 rms_eps=1e-6)


class OracleModel:
    """The oracle's view of a weights.bin / index.json pair (format 1 or 2)."""

    def __init__(self, index_json: str, weights: np.ndarray, precision: str = "f64", max_context: int = 4096):
        self.L = lib(precision)
        ix = json.loads(index_json)
        cfg = dict(ix["config"])
        if ix.get("format_version", 1) == 1:
            cfg.update(V1_CONFIG)
            if not cfg.get("intermediate"):
                cfg["intermediate"] = 3584 if cfg["hidden"] == 1024 else 6144
        cfg.setdefault("rms_eps", 1e-6)
        self.cfg = cfg
        self.max_context = max_context
        self.buf = np.ascontiguousarray(weights.view(np.uint8).reshape(-1))
        self.keep = []

        def tensor(name, dtype):
            t = ix["tensors"][name]
            a = np.frombuffer(self.buf, dtype=dtype, count=t["bytes"] // np.dtype(dtype).itemsize, offset=t["offset"])
            self.keep.append(a)
            return a

        def mat(name):
            m = ix["matrices"][name]
            if ix.get("format_version", 1) == 1:
                return mat_struct(m, OC_Q4V1, m["rows"], m["k"], 32, tensor(name + ".w", np.uint32),
                                  tensor(name + ".s", np.uint16), tensor(name + ".z", np.uint8))
            if m.get("dtype", "q4") == "f16":
                return mat_struct(m, OC_F16, m["rows"], m["k"], 0, tensor(name + ".w", np.uint16))
            kind = OC_Q4V1 if m.get("zero", "f16") == "u4" else OC_Q4G
            return mat_struct(m, kind, m["rows"], m["k"], m.get("group", 64), tensor(name + ".w", np.uint32),
                              tensor(name + ".s", np.uint16),
                              tensor(name + ".z", np.uint8 if kind == OC_Q4V1 else np.uint16))

        self.layers = (Layer * cfg["layers"])()
        for i in range(cfg["layers"]):
            p = f"layer{i}."
            Lr = self.layers[i]
            Lr.mixer_in, Lr.mixer_out = mat(p + "mixer_in"), mat(p + "mixer_out")
            Lr.gate_up, Lr.down = mat(p + "gate_up"), mat(p + "down")
            Lr.input_norm = tensor(p + "input_norm", np.float32).ctypes.data
            Lr.post_norm = tensor(p + "post_norm", np.float32).ctypes.data
            if (i + 1) % cfg["full_attention_every"] == 0:
                Lr.attn_norms = tensor(p + "attn_norms", np.float32).ctypes.data
            else:
                Lr.conv_w = tensor(p + "conv_w", np.float32).ctypes.data
                Lr.gdn_params = tensor(p + "gdn_params", np.float32).ctypes.data
        self.m = ModelS()
        self.m.c = config_struct(cfg, max_context)
        self.m.embed, self.m.lm_head = mat("embed"), mat("lm_head")
        self.m.final_norm = tensor("final_norm", np.float32).ctypes.data
        self.m.layers = self.layers
        self.state = self.L.oc_state_new(ctypes.byref(self.m))

    def __del__(self):
        try:
            self.L.oc_state_free(self.state)
        except Exception:
            pass

    def reset(self):
        self.L.oc_reset(self.state)

    def state_bytes(self) -> bytes:
        """Every recurrent, conv and KV value of the state, concatenated (for bitwise comparisons)."""
        c = self.cfg
        attn = [(i + 1) % c["full_attention_every"] == 0 for i in range(c["layers"])]
        n_gdn, n_attn = attn.count(False), attn.count(True)
        rec = c["gdn_heads"] * c["gdn_dk"] * c["gdn_dv"] * 4
        conv = (2 * c["gdn_heads"] * c["gdn_dk"] + c["gdn_heads"] * c["gdn_dv"]) * (c["conv_kernel"] - 1) * 4
        kv = c["n_kv_heads"] * self.max_context * c["head_dim"] * 2
        out = []
        for i in range(n_gdn):
            out.append(ctypes.string_at(self.L.oc_state_recurrent(self.state, i), rec))
            out.append(ctypes.string_at(self.L.oc_state_conv(self.state, i), conv))
        for i in range(n_attn):
            out.append(ctypes.string_at(self.L.oc_state_kcache(self.state, i), kv))
            out.append(ctypes.string_at(self.L.oc_state_vcache(self.state, i), kv))
        return b"".join(out)

    def token(self, token: int, pos: int, want_logits: bool = True):
        out = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        self.L.oc_token(ctypes.byref(self.m), self.state, token, pos, ptr(out) if want_logits else None)
        return out

    def prefill_chunk(self, ids, start: int, finish_logits: bool = True):
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
        out = np.empty(self.cfg["vocab"], dtype=np.float32)
        self.L.oc_prefill_chunk(ctypes.byref(self.m), self.state, ptr(a), a.size, start, int(finish_logits), ptr(out))
        return out if finish_logits else None

    def greedy(self, prompt, steps: int):
        """Prefill then greedy decode; returns (ids, list of logits per step)."""
        logits = self.prefill_chunk(prompt, 0, True)
        ids, all_logits = [], [logits]
        pos = len(prompt)
        for _ in range(steps):
            t = int(np.argmax(logits))  # lowest index among equal maxima, like oc_argmax
            ids.append(t)
            logits = self.token(t, pos)
            all_logits.append(logits)
            pos += 1
        return ids, all_logits


class OracleSampler:
    """src/sampling.rs Sampler restated in the C oracle (oc_sample), f32 throughout: the checker of
    the device sampler. sample() raises ValueError where the reference's try_sample fails closed."""

    def __init__(self, temperature=0.6, top_k=20, top_p=0.95, seed=42, presence_penalty=0.0):
        self.L = lib("f32")
        self.state = ctypes.c_uint64(self.L.oc_sampler_seed(seed))
        self.opts = (float(temperature), int(top_k), float(top_p), float(presence_penalty))
        self.seen = np.zeros(0, np.uint8)

    def sample(self, logits, mask=None, mask_len=0):
        x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
        V = x.size
        if self.seen.size < max(V, 1):
            self.seen = np.concatenate([self.seen, np.zeros(max(V, 1) - self.seen.size, np.uint8)])
        if mask is not None:
            m = np.ascontiguousarray(np.asarray(mask, dtype=np.uint32))
            mp = m.ctypes.data_as(ctypes.c_void_p)
        else:
            m, mp, mask_len = None, None, 0
        t, k, p, pen = self.opts
        tok = ctypes.c_uint32()
        rc = self.L.oc_sample(x.ctypes.data_as(ctypes.c_void_p) if V else None, V, mp, mask_len, t, k, p, pen,
                              ctypes.byref(self.state), self.seen.ctypes.data_as(ctypes.c_void_p), ctypes.byref(tok))
        if rc:
            raise ValueError("distribution rejected")
        return tok.value


def bitset(allowed, n):
    """uint32 words with bit i%32 of word i/32 set for each allowed token i < n (SimpleVob layout)."""
    w = np.zeros((n + 31) // 32 or 1, np.uint32)
    for i in allowed:
        if i < n:
            w[i >> 5] |= np.uint32(1 << (i & 31))
    return w
