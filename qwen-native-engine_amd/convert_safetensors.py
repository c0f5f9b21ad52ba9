"""Qwen3.5 safetensors checkpoint (Hugging Face layout) -> weights.bin + index.json (format 2).

The reference converts the onnx-community q4f16 export (scripts/convert_weights.py:82-145). This
converter reads the original checkpoint (`model.safetensors` or a sharded
`model.safetensors.index.json`, bf16 / f16 / f32) and writes the same tensor set in format 2
(weights.py), f16 or int4 per matrix. The mapping follows the transformers `qwen3_5` modules
(Qwen3_5DecoderLayer, Qwen3_5GatedDeltaNet, Qwen3_5Attention, Qwen3_5MLP):

  layer{i}.input_norm, post_norm, final_norm = 1 + weight   (Qwen3_5RMSNorm scales by 1 + w; the
      engine's RMSNorm, like the reference's shader, multiplies by the stored gain)
  GDN layers (linear_attn):
      mixer_in   = in_proj_qkv (q, k, v) ; in_proj_z ; in_proj_a ; in_proj_b  (convert_weights.py:121)
      mixer_out  = out_proj
      conv_w     = conv1d.weight [channels, 1, K] as [channels][K]
      gdn_params = dt_bias ; -exp(A_log) ; norm.weight      (convert_weights.py:125: A_neg_exp; the
                   gated norm scales by w itself)
  attention layers (self_attn):
      mixer_in   = q_proj with its rows [h0 q | h0 gate | h1 q | ...] reordered to all queries, then
                   all gates (convert_weights.py:72-78) ; k_proj ; v_proj
      mixer_out  = o_proj
      attn_norms = 1 + q_norm.weight ; 1 + k_norm.weight
  gate_up = mlp.gate_proj ; mlp.up_proj,  down = mlp.down_proj
  embed = embed_tokens, lm_head = lm_head.weight (embed_tokens when tie_word_embeddings)

Tensor names may carry the text model's prefix of the multimodal checkpoint
(`model.language_model.`) or of the text-only one (`model.`); vision-tower and multi-token
prediction tensors are not read.

Run: python qwen-native-engine_amd/convert_safetensors.py --model-dir <hf dir> --out <dir>
     [--body f16|q4] [--head f16|q4] [--group 64]
"""
from __future__ import annotations

import argparse
import json
import struct
from pathlib import Path

import numpy as np

try:
    from . import weights as W  # type: ignore
except ImportError:  # run as a script or imported from the package directory
    import weights as W

_DTYPES = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32}


class SafeTensors:
    """Read-only view of a (possibly sharded) safetensors checkpoint; tensors are memory-mapped
    and converted to float32 one at a time."""

    def __init__(self, model_dir):
        d = Path(model_dir)
        index = d / "model.safetensors.index.json"
        if index.exists():
            files = sorted(set(json.loads(index.read_text(encoding="utf-8"))["weight_map"].values()))
        else:
            files = sorted(p.name for p in d.glob("*.safetensors"))
        if not files:
            raise FileNotFoundError(f"no safetensors files in {d}")
        self.where = {}
        for f in files:
            path = d / f
            with open(path, "rb") as fh:
                n = struct.unpack("<Q", fh.read(8))[0]
                header = json.loads(fh.read(n))
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                self.where[name] = (path, 8 + n, meta)

    def names(self):
        return self.where.keys()

    def has(self, name):
        return name in self.where

    def get(self, name) -> np.ndarray:
        if name not in self.where:
            raise KeyError(f"tensor {name} not in the checkpoint")
        path, base, meta = self.where[name]
        dt = meta["dtype"]
        if dt not in _DTYPES:
            raise ValueError(f"{name}: unsupported dtype {dt}")
        begin, end = meta["data_offsets"]
        shape = tuple(meta["shape"])
        count = int(np.prod(shape)) if shape else 1
        raw = np.memmap(path, dtype=_DTYPES[dt], mode="r", offset=base + begin, shape=(count,))
        if (end - begin) != count * raw.itemsize:
            raise ValueError(f"{name}: data size does not match its shape")
        if dt == "BF16":
            out = (raw.astype(np.uint32) << 16).view(np.float32)
        else:
            out = raw.astype(np.float32)
        return out.reshape(shape)


def read_config(model_dir):
    """(top-level config, text config): the image-text checkpoints nest the text model's config
    under text_config and keep tie_word_embeddings at the top."""
    cfg = json.loads((Path(model_dir) / "config.json").read_text(encoding="utf-8"))
    return cfg, cfg.get("text_config", cfg)


def engine_config(hf: dict) -> dict:
    """Format-2 config from a Qwen3.5 text config; raises ValueError for what the engine cannot run."""
    layers = hf["num_hidden_layers"]
    types = hf.get("layer_types")
    every = hf.get("full_attention_interval", 4)
    if types is not None:
        if "full_attention" not in types:
            raise ValueError("unsupported architecture: no full-attention layer")
        every = types.index("full_attention") + 1
        want = ["full_attention" if (i + 1) % every == 0 else "linear_attention" for i in range(layers)]
        if list(types) != want:
            raise ValueError("unsupported architecture: layer_types is not every-Nth full attention")
    if hf["linear_num_key_heads"] != hf["linear_num_value_heads"]:
        raise ValueError("unsupported architecture: linear_num_key_heads != linear_num_value_heads")
    rope = hf.get("rope_parameters") or {}
    theta = rope.get("rope_theta", hf.get("rope_theta", 10000000.0))
    partial = rope.get("partial_rotary_factor", hf.get("partial_rotary_factor", 1.0))
    head_dim = hf.get("head_dim") or hf["hidden_size"] // hf["num_attention_heads"]
    if hf.get("attention_bias"):
        raise ValueError("unsupported architecture: attention_bias")
    if hf.get("hidden_act", "silu") != "silu":
        raise ValueError("unsupported architecture: hidden_act must be silu")
    return dict(layers=layers, full_attention_every=every, hidden=hf["hidden_size"],
                intermediate=hf["intermediate_size"], vocab=hf["vocab_size"], rope_theta=float(theta),
                rope_dim=int(head_dim * partial), n_q_heads=hf["num_attention_heads"],
                n_kv_heads=hf["num_key_value_heads"], head_dim=head_dim, gdn_heads=hf["linear_num_value_heads"],
                gdn_dk=hf["linear_key_head_dim"], gdn_dv=hf["linear_value_head_dim"],
                conv_kernel=hf["linear_conv_kernel_dim"], rms_eps=float(hf.get("rms_norm_eps", 1e-6)))


def _prefix(st: SafeTensors) -> str:
    for p in ("model.language_model.", "model."):
        if st.has(p + "embed_tokens.weight"):
            return p
    raise ValueError("no embed_tokens.weight under model.language_model. or model.")


def _deinterleave_q_gate(w: np.ndarray, heads: int, head_dim: int) -> np.ndarray:
    """Rows [h0 q | h0 gate | h1 q | ...] -> [all q | all gates] (convert_weights.py:72-78)."""
    r = w.reshape(heads, 2, head_dim, -1)
    return np.concatenate([r[:, 0].reshape(heads * head_dim, -1), r[:, 1].reshape(heads * head_dim, -1)])


def convert(model_dir, out_dir, body: str = "f16", head: str = "f16", group: int = 64, lib=None) -> dict:
    """Writes out_dir/weights.bin and out_dir/index.json; returns the index as a dict."""
    if body not in ("f16", "q4") or head not in ("f16", "q4"):
        raise ValueError("body and head must be f16 or q4")
    top, hf = read_config(model_dir)
    cfg = engine_config(hf)
    st = SafeTensors(model_dir)
    pre = _prefix(st)
    tied = bool(top.get("tie_word_embeddings", hf.get("tie_word_embeddings", False))) or not st.has("lm_head.weight")
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    wr = W.Writer(out / "weights.bin.tmp")
    mats = {}
    if "q4" in (body, head) and lib is None:
        from qne import load_library
        lib = load_library()

    def add_matrix(name, w, dtype):
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, k = w.shape
        if dtype == "f16":
            mats[name] = {"rows": rows, "k": k, "dtype": "f16"}
            wr.add(name + ".w", w.astype(np.float16).view(np.uint16), "f16")
            return
        import ctypes
        if k % group:
            raise ValueError(f"{name}: k={k} is not a multiple of the group {group}")
        q = np.empty((rows, k // 8), dtype=np.uint32)
        s = np.empty((rows, k // group), dtype=np.uint16)
        z = np.empty((rows, k // group), dtype=np.uint16)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        rc = lib.qne_quantize_q4g(p(w), ctypes.c_size_t(rows), ctypes.c_size_t(k), ctypes.c_size_t(group),
                                  p(q), p(s), p(z))
        if rc != 0:
            raise ValueError(f"{name}: quantisation failed ({rc})")
        mats[name] = {"rows": rows, "k": k, "dtype": "q4", "group": group, "zero": "f16"}
        wr.add(name + ".w", q, "q4")
        wr.add(name + ".s", s, "f16")
        wr.add(name + ".z", z, "f16")

    def vec(name, v):
        wr.add(name, np.ascontiguousarray(v, dtype=np.float32).reshape(-1), "f32")

    g = lambda n: st.get(pre + n)
    embed = g("embed_tokens.weight")
    add_matrix("embed", embed, head)
    del embed
    for i in range(cfg["layers"]):
        L = f"layers.{i}."
        vec(f"layer{i}.input_norm", 1.0 + g(L + "input_layernorm.weight"))
        vec(f"layer{i}.post_norm", 1.0 + g(L + "post_attention_layernorm.weight"))
        if W.is_attn(cfg, i):
            A = L + "self_attn."
            q = _deinterleave_q_gate(g(A + "q_proj.weight"), cfg["n_q_heads"], cfg["head_dim"])
            add_matrix(f"layer{i}.mixer_in", np.concatenate([q, g(A + "k_proj.weight"), g(A + "v_proj.weight")]), body)
            add_matrix(f"layer{i}.mixer_out", g(A + "o_proj.weight"), body)
            vec(f"layer{i}.attn_norms", np.concatenate([1.0 + g(A + "q_norm.weight"), 1.0 + g(A + "k_norm.weight")]))
        else:
            D = L + "linear_attn."
            add_matrix(f"layer{i}.mixer_in", np.concatenate([g(D + n + ".weight") for n in
                                                             ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")]), body)
            add_matrix(f"layer{i}.mixer_out", g(D + "out_proj.weight"), body)
            conv = g(D + "conv1d.weight")
            vec(f"layer{i}.conv_w", conv.reshape(conv.shape[0], -1))
            vec(f"layer{i}.gdn_params", np.concatenate([g(D + "dt_bias"), -np.exp(g(D + "A_log").astype(np.float64)),
                                                        g(D + "norm.weight")]))
        M = L + "mlp."
        add_matrix(f"layer{i}.gate_up", np.concatenate([g(M + "gate_proj.weight"), g(M + "up_proj.weight")]), body)
        add_matrix(f"layer{i}.down", g(M + "down_proj.weight"), body)
    vec("final_norm", 1.0 + g("norm.weight"))
    lm = g("embed_tokens.weight") if tied else st.get("lm_head.weight")
    add_matrix("lm_head", lm, head)
    del lm
    wr.close()
    # the shapes the engine expects, checked before the files are published
    for name, (rows, k) in W.matrix_shapes(cfg).items():
        if (mats[name]["rows"], mats[name]["k"]) != (rows, k):
            raise ValueError(f"{name}: shape {mats[name]['rows']}x{mats[name]['k']}, expected {rows}x{k}")
    keys = ["layers", "full_attention_every", "hidden", "intermediate", "vocab", "rope_theta", "rope_dim",
            "n_q_heads", "n_kv_heads", "head_dim", "gdn_heads", "gdn_dk", "gdn_dv", "conv_kernel", "rms_eps"]
    index = {"source": f"{Path(model_dir).name} safetensors", "format_version": 2,
             "config": {k: cfg[k] for k in keys}, "matrices": mats, "tensors": wr.index}
    (out / "index.json.tmp").write_text(json.dumps(index, indent=1), encoding="utf-8")
    (out / "weights.bin.tmp").replace(out / "weights.bin")
    (out / "index.json.tmp").replace(out / "index.json")
    return index


def main():
    ap = argparse.ArgumentParser(description="Convert a Qwen3.5 safetensors checkpoint to weights.bin + index.json")
    ap.add_argument("--model-dir", type=Path, required=True, help="directory with config.json and *.safetensors")
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--body", choices=("f16", "q4"), default="q4", help="layer matrices")
    ap.add_argument("--head", choices=("f16", "q4"), default="f16", help="embedding and LM head")
    ap.add_argument("--group", type=int, default=64, help="int4 quantisation group (64 or 128)")
    a = ap.parse_args()
    ix = convert(a.model_dir, a.out, a.body, a.head, a.group)
    size = (a.out / "weights.bin").stat().st_size
    print(f"wrote {size / 1e6:.0f} MB, {len(ix['tensors'])} tensors to {a.out}")


if __name__ == "__main__":
    main()
