"""A tiny Qwen3.5 text model from transformers' own `qwen3_5` implementation, with seeded random
parameters, saved as a safetensors checkpoint the way the published ones are laid out (matrices
in bf16, the small per-head vectors in f32). Its forward pass is the independent check of the
safetensors converter and of the oracle's model math: transformers computes the hybrid decoder
(chunked gated delta rule, SDPA attention, (1 + w) RMSNorm, interleaved q/gate rows) its own way.

Shapes are the engine's "tiny" test model: 4 layers (3 Gated DeltaNet, 1 attention), hidden 512,
intermediate 1024, vocab 4096, 2 query heads / 1 kv head of 256, 4 GDN heads of 128."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

TINY = dict(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_hidden_layers=4, num_attention_heads=2,
            num_key_value_heads=1, head_dim=256, linear_num_key_heads=4, linear_num_value_heads=4,
            linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4, rms_norm_eps=1e-6,
            rope_parameters={"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25,
                             "mrope_section": [11, 11, 10], "mrope_interleaved": True})


def available() -> bool:
    """Whether safetensors and transformers' qwen3_5 model are installed, found without importing
    either (a GPU test process must not load torch, which carries its own HIP runtime)."""
    import importlib.util
    try:
        st, tf = importlib.util.find_spec("safetensors"), importlib.util.find_spec("transformers")
    except Exception:
        return False
    if st is None or tf is None or importlib.util.find_spec("torch") is None or not tf.submodule_search_locations:
        return False
    return any((Path(d) / "models" / "qwen3_5" / "modeling_qwen3_5.py").exists() for d in tf.submodule_search_locations)


def build_in_subprocess(seed: int, directory, ids) -> tuple[Path, np.ndarray]:
    """build + save + logits(ids) in a child process (for the GPU tests, which keep torch out of
    their own process): returns the checkpoint directory and transformers' logits."""
    import subprocess
    import sys
    d = Path(directory)
    ids = np.asarray(ids, dtype=np.int64)
    np.save(d / "ids.npy", ids)
    subprocess.run([sys.executable, str(Path(__file__).resolve()), str(seed), str(d)], check=True)
    return d / "hf", np.load(d / "logits.npy")


def build(seed: int = 0, tied: bool = False):
    """The model (float32, eval mode) with every parameter drawn from a seeded generator: matrices
    N(0, 0.03), RMSNorm offsets N(0, 0.2) (the stored weight is the offset from 1), gated-norm gains
    1 + N(0, 0.2), conv taps N(0, 0.3), A_log = log U(1, 16), dt_bias N(0, 0.5). Matrices and conv
    taps are rounded to bf16, the precision they are saved in."""
    import torch
    from transformers.models.qwen3_5 import Qwen3_5ForCausalLM, Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(tie_word_embeddings=tied, **TINY)
    torch.manual_seed(seed)
    m = Qwen3_5ForCausalLM(cfg).eval()
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("A_log"):
                v = torch.log(1.0 + 15.0 * torch.rand(p.shape, generator=gen))
            elif name.endswith("dt_bias"):
                v = 0.5 * torch.randn(p.shape, generator=gen)
            elif name.endswith("conv1d.weight"):
                v = 0.3 * torch.randn(p.shape, generator=gen)
            elif name.endswith("linear_attn.norm.weight"):
                v = 1.0 + 0.2 * torch.randn(p.shape, generator=gen)
            elif p.ndim == 1:
                v = 0.2 * torch.randn(p.shape, generator=gen)  # (1 + w) RMSNorm offsets
            else:
                v = 0.03 * torch.randn(p.shape, generator=gen)
            if p.ndim >= 2:  # stored as bf16 in the checkpoint (save): keep the model on those values
                v = v.to(torch.bfloat16).float()
            p.copy_(v)
    return m


def save(m, directory, multimodal: bool = False) -> Path:
    """Writes config.json and model.safetensors. multimodal: the tensor names and config nesting of
    the image-text checkpoints (model.language_model.*, text_config), plus a vision-tower and an
    MTP tensor the converter must skip."""
    import torch
    from safetensors.torch import save_file
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    tensors = {}
    for name, p in m.state_dict().items():
        if name == "lm_head.weight" and m.config.tie_word_embeddings:
            continue
        t = p.detach().to(torch.bfloat16) if p.ndim >= 2 else p.detach().float()
        if multimodal and name.startswith("model."):
            name = "model.language_model." + name[len("model."):]
        tensors[name] = t.contiguous()
    if multimodal:
        tensors["model.visual.patch_embed.proj.weight"] = torch.zeros(8, 3, 2, 2, dtype=torch.bfloat16)
        tensors["mtp.fc.weight"] = torch.zeros(4, 4, dtype=torch.bfloat16)
    save_file(tensors, str(d / "model.safetensors"))
    text = m.config.to_dict()
    cfg = {"model_type": "qwen3_5", "text_config": text,
           "tie_word_embeddings": bool(m.config.tie_word_embeddings)} if multimodal else text
    (d / "config.json").write_text(json.dumps(cfg), encoding="utf-8")
    return d


def logits(m, ids) -> np.ndarray:
    """transformers' logits for every position of the prompt, float32 [len(ids), vocab]."""
    import torch
    with torch.no_grad():
        out = m(torch.as_tensor(np.asarray(ids, dtype=np.int64))[None]).logits[0]
    return out.float().numpy()


if __name__ == "__main__":
    import sys
    seed, out = int(sys.argv[1]), Path(sys.argv[2])
    model = build(seed=seed)
    save(model, out / "hf")
    np.save(out / "logits.npy", logits(model, np.load(out / "ids.npy")))
