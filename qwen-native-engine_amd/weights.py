"""weights.bin + index.json: writer, format-2 layout and seeded synthetic models.

The file format follows scripts/convert_weights.py of the reference (weights.bin of 256-byte
aligned, content-deduplicated tensors; index.json {format_version, config, matrices, tensors},
convert_weights.py:35-59,134-141). Format 2 adds config-driven shapes and per-matrix encodings:
  config:   layers, full_attention_every, hidden, intermediate, vocab, rope_theta, rope_dim,
            n_q_heads, n_kv_heads, head_dim, gdn_heads, gdn_dk, gdn_dv, conv_kernel, rms_eps
  matrices: name -> {rows, k, dtype: "f16" | "q4", group, zero: "f16" | "u4"}
  tensors:  "<matrix>.w" (f16 [rows][k], or u32 [rows][k/8] nibbles, value c at bits 4*(c%8) of
            word c/8), "<matrix>.s" (f16 [rows][k/group]), "<matrix>.z" (f16 [rows][k/group], or
            u4 zero points two per byte), plus the f32 vectors of the reference
            (layer{i}.input_norm / post_norm / attn_norms / conv_w / gdn_params, final_norm).
Projections are concatenated along rows as in the reference (convert_weights.py:6-12):
GDN mixer_in = q, k, v, z, a, b; attention mixer_in = q, gate, k, v; gate_up = gate, up.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

ALIGN = 256

# Model shapes used by the tests and benches.
CONFIGS = {
    # small enough for the CPU oracle to run whole prompts in a second
    "tiny": dict(layers=4, full_attention_every=4, hidden=512, intermediate=1024, vocab=4096,
                 n_q_heads=2, n_kv_heads=1, head_dim=256, gdn_heads=4),
    # Qwen3.5-0.8B body shapes with fewer layers and a small vocabulary
    "small": dict(layers=8, full_attention_every=4, hidden=1024, intermediate=3584, vocab=8192,
                  n_q_heads=8, n_kv_heads=2, head_dim=256, gdn_heads=16),
    # Qwen3.5-0.8B-shaped hybrid decoder (f16 weights)
    "0.8b": dict(layers=24, full_attention_every=4, hidden=1024, intermediate=3584, vocab=151936,
                 n_q_heads=8, n_kv_heads=2, head_dim=256, gdn_heads=16),
    # Qwen3.5-2B-shaped hybrid decoder (int4 body, f16 embedding and LM head)
    "2b": dict(layers=28, full_attention_every=4, hidden=2048, intermediate=6144, vocab=151936,
               n_q_heads=16, n_kv_heads=4, head_dim=256, gdn_heads=16),
}
COMMON = dict(rope_theta=10000000.0, rope_dim=64, gdn_dk=128, gdn_dv=128, conv_kernel=4, rms_eps=1e-6)


def full_config(name_or_cfg) -> dict:
    cfg = dict(COMMON)
    cfg.update(CONFIGS[name_or_cfg] if isinstance(name_or_cfg, str) else name_or_cfg)
    return cfg


def is_attn(cfg: dict, i: int) -> bool:
    return (i + 1) % cfg["full_attention_every"] == 0


def attn_proj(c):
    return 2 * c["n_q_heads"] * c["head_dim"] + 2 * c["n_kv_heads"] * c["head_dim"]


def gdn_proj(c):
    return 2 * c["gdn_heads"] * c["gdn_dk"] + 2 * c["gdn_heads"] * c["gdn_dv"] + 2 * c["gdn_heads"]


def conv_channels(c):
    return 2 * c["gdn_heads"] * c["gdn_dk"] + c["gdn_heads"] * c["gdn_dv"]


def matrix_shapes(cfg: dict) -> dict:
    """name -> (rows, k) for every matrix of the model (model.rs:72-84 generalised)."""
    c, h = cfg, cfg["hidden"]
    out = {"embed": (c["vocab"], h), "lm_head": (c["vocab"], h)}
    for i in range(c["layers"]):
        a = is_attn(c, i)
        out[f"layer{i}.mixer_in"] = (attn_proj(c) if a else gdn_proj(c), h)
        out[f"layer{i}.mixer_out"] = (h, c["n_q_heads"] * c["head_dim"] if a else c["gdn_heads"] * c["gdn_dv"])
        out[f"layer{i}.gate_up"] = (2 * c["intermediate"], h)
        out[f"layer{i}.down"] = (h, c["intermediate"])
    return out


def vector_shapes(cfg: dict) -> dict:
    """name -> float count of every f32 tensor."""
    c, h = cfg, cfg["hidden"]
    out = {"final_norm": h}
    for i in range(c["layers"]):
        out[f"layer{i}.input_norm"] = h
        out[f"layer{i}.post_norm"] = h
        if is_attn(c, i):
            out[f"layer{i}.attn_norms"] = 2 * c["head_dim"]
        else:
            out[f"layer{i}.conv_w"] = conv_channels(c) * c["conv_kernel"]
            out[f"layer{i}.gdn_params"] = 2 * c["gdn_heads"] + c["gdn_dv"]
    return out


class Writer:
    """Appends tensors to a weights.bin file and builds its index.json "tensors" map.

    Format rules (the reference's scripts/convert_weights.py defines them for format 1 and this
    module keeps them): every tensor starts on a 256-byte boundary, and a tensor whose raw bytes,
    kind and shape equal a tensor written earlier is not stored twice; its index entry names the
    earlier copy's range (a tied LM head, repeated norm gains)."""

    def __init__(self, path):
        self._out = open(path, "wb")
        self._size = 0            # bytes written so far
        self._stored = {}         # content key -> index entry of the stored copy
        self.index = {}           # tensor name -> {"offset", "bytes", "kind", "shape"}

    def _align(self):
        gap = -self._size % ALIGN
        if gap:
            self._out.write(bytes(gap))
            self._size += gap

    def add(self, name, array, kind):
        arr = np.ascontiguousarray(array)
        raw = arr.tobytes()
        key = (hashlib.sha256(raw).hexdigest(), kind, arr.shape)
        entry = self._stored.get(key)
        if entry is None:
            self._align()
            entry = {"offset": self._size, "bytes": arr.nbytes, "kind": kind, "shape": list(arr.shape)}
            self._out.write(raw)
            self._size += arr.nbytes
            self._stored[key] = entry
        self.index[name] = dict(entry)

    def close(self):
        self._out.close()


def split_query_gate_rows(parts, heads, head_dim):
    """The attention in-projection of a Qwen3.5 checkpoint holds, per query head, its head_dim query
    rows followed by its head_dim gate rows; the engine (and the reference's format) wants every
    query row first, then every gate row, head by head. `parts` are arrays over those rows (weights,
    scales, zeros); each is returned in the engine's order."""
    per_head = np.arange(heads * 2 * head_dim).reshape(heads, 2, head_dim)
    order = np.concatenate([per_head[:, 0, :].reshape(-1), per_head[:, 1, :].reshape(-1)])
    return tuple(np.asarray(p)[order] for p in parts)


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


class Layout:
    """In-memory weights.bin: offsets planned first (256-byte aligned), then filled in place."""

    def __init__(self):
        self.tensors = {}
        self.size = 0

    def reserve(self, name, nbytes, kind, shape):
        self.size += (-self.size) % ALIGN
        self.tensors[name] = {"offset": self.size, "bytes": int(nbytes), "kind": kind, "shape": list(shape)}
        self.size += int(nbytes)

    def view(self, buf, name, dtype):
        t = self.tensors[name]
        return np.frombuffer(buf, dtype=dtype, count=t["bytes"] // np.dtype(dtype).itemsize, offset=t["offset"])


def plan(cfg: dict, body: str = "q4", head: str = "f16", group: int = 64, tied: bool = False):
    """Plans every tensor of a format-2 model. body/head: "f16" or "q4" for the layer matrices and
    for the embedding / LM head."""
    lay = Layout()
    mats = {}
    for name, (rows, k) in matrix_shapes(cfg).items():
        dtype = head if name in ("embed", "lm_head") else body
        if name == "lm_head" and tied:
            mats[name] = dict(mats["embed"])
            for suffix in (".w", ".s", ".z"):
                if "embed" + suffix in lay.tensors:
                    lay.tensors[name + suffix] = dict(lay.tensors["embed" + suffix])
            continue
        if dtype == "f16":
            mats[name] = {"rows": rows, "k": k, "dtype": "f16"}
            lay.reserve(name + ".w", rows * k * 2, "f16", (rows, k))
        else:
            mats[name] = {"rows": rows, "k": k, "dtype": "q4", "group": group, "zero": "f16"}
            lay.reserve(name + ".w", rows * k // 2, "q4", (rows, k // 8))
            lay.reserve(name + ".s", rows * k // group * 2, "f16", (rows, k // group))
            lay.reserve(name + ".z", rows * k // group * 2, "f16", (rows, k // group))
    for name, n in vector_shapes(cfg).items():
        lay.reserve(name, n * 4, "f32", (n,))
    return lay, mats


def index_json(cfg: dict, lay: Layout, mats: dict, source: str) -> str:
    keys = ["layers", "full_attention_every", "hidden", "intermediate", "vocab", "rope_theta", "rope_dim",
            "n_q_heads", "n_kv_heads", "head_dim", "gdn_heads", "gdn_dk", "gdn_dv", "conv_kernel", "rms_eps"]
    return json.dumps({"source": source, "format_version": 2, "config": {k: cfg[k] for k in keys},
                       "matrices": mats, "tensors": lay.tensors}, indent=1)


def synth_model(cfg_name_or_dict, seed: int = 0, body: str = "q4", head: str = "f16", group: int = 64,
                std: float = 0.02, norm_jitter: float = 0.0, tied: bool = False, lib=None):
    """Seeded random model: every matrix N(0, std) (SplitMix64 + Box-Muller keyed by tensor name),
    int4 matrices quantised per group (qne_quantize_q4g); norm gains 1 (+ N(0, norm_jitter)),
    conv_w N(0, std), dt_bias 0, A_neg_exp -0.5, GDN norm 1 (the reference's synthetic values,
    kernels/src/lib.rs:777). Returns (index_json, weights as a uint8 numpy array)."""
    from qne import load_library
    lib = lib or load_library()
    cfg = full_config(cfg_name_or_dict)
    lay, mats = plan(cfg, body, head, group, tied)
    buf = np.zeros(lay.size, dtype=np.uint8)
    mem = buf.data
    import ctypes
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    for name, m in mats.items():
        if name == "lm_head" and tied:
            continue
        rows, k, stream = m["rows"], m["k"], fnv1a64(name)
        if m["dtype"] == "f16":
            w = lay.view(mem, name + ".w", np.uint16)
            lib.qne_synth_normal_f16(ctypes.c_uint64(seed), ctypes.c_uint64(stream), ctypes.c_size_t(w.size),
                                     ctypes.c_float(std), ptr(w))
        else:
            tmp = np.empty(rows * k, dtype=np.float32)
            lib.qne_synth_normal_f32(ctypes.c_uint64(seed), ctypes.c_uint64(stream), ctypes.c_size_t(tmp.size),
                                     ctypes.c_float(std), ptr(tmp))
            q = lay.view(mem, name + ".w", np.uint32)
            s = lay.view(mem, name + ".s", np.uint16)
            z = lay.view(mem, name + ".z", np.uint16)
            rc = lib.qne_quantize_q4g(ptr(tmp), ctypes.c_size_t(rows), ctypes.c_size_t(k), ctypes.c_size_t(group),
                                      ptr(q), ptr(s), ptr(z))
            assert rc == 0
            del tmp
    for name, n in vector_shapes(cfg).items():
        v = lay.view(mem, name, np.float32)
        if name.endswith("conv_w"):
            lib.qne_synth_normal_f32(ctypes.c_uint64(seed), ctypes.c_uint64(fnv1a64(name)), ctypes.c_size_t(n),
                                     ctypes.c_float(std), ptr(v))
        elif name.endswith("gdn_params"):
            H = cfg["gdn_heads"]
            v[:H] = 0.0
            v[H:2 * H] = -0.5
            v[2 * H:] = 1.0
        else:
            v[:] = 1.0
            if norm_jitter:
                j = np.empty(n, dtype=np.float32)
                lib.qne_synth_normal_f32(ctypes.c_uint64(seed), ctypes.c_uint64(fnv1a64(name)), ctypes.c_size_t(n),
                                         ctypes.c_float(norm_jitter), ptr(j))
                v += j
    return index_json(cfg, lay, mats, f"synthetic seed {seed}"), buf


def write_files(directory, index: str, weights: np.ndarray):
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    (d / "weights.bin").write_bytes(weights.tobytes())
    (d / "index.json").write_text(index, encoding="utf-8")
