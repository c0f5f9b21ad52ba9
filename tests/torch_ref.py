"""An independent float64 formulation of the hybrid decoder in torch, used only to pin the oracle.

It is written from the mathematics with library routines instead of the oracle's loops:
F.rms_norm, F.silu, F.softplus, F.conv1d for the causal convolution, the delta rule in matrix
form S' = g (I - beta k k^T) S + beta k v^T with out = S'^T q, RoPE as a complex rotation, and
F.scaled_dot_product_attention for GQA attention. Weights are dequantised with numpy bit
operations on the packed words.
"""
from __future__ import annotations

import json

import numpy as np
import torch
import torch.nn.functional as F

D = torch.float64


def dequant(ix, buf, name):
    m = ix["matrices"][name]
    rows, k = m["rows"], m["k"]

    def t(n, dt):
        e = ix["tensors"][n]
        return np.frombuffer(buf, dtype=dt, count=e["bytes"] // np.dtype(dt).itemsize, offset=e["offset"])

    if ix.get("format_version", 1) == 2 and m.get("dtype") == "f16":
        return torch.from_numpy(t(name + ".w", np.float16).astype(np.float64).reshape(rows, k))
    words = t(name + ".w", np.uint32).reshape(rows, k // 8)
    shifts = np.arange(8, dtype=np.uint32) * 4
    q = ((words[:, :, None] >> shifts) & 15).reshape(rows, k).astype(np.float64)
    g = m.get("group", 32) if ix.get("format_version", 1) == 2 else 32
    s = t(name + ".s", np.float16).astype(np.float64).reshape(rows, k // g)
    if ix.get("format_version", 1) == 2 and m.get("zero", "f16") == "f16":
        z = t(name + ".z", np.float16).astype(np.float64).reshape(rows, k // g)
    else:
        zb = t(name + ".z", np.uint8).reshape(rows, -1)
        z = np.stack([zb & 15, zb >> 4], axis=-1).reshape(rows, -1)[:, : k // g].astype(np.float64)
    w = (q - np.repeat(z, g, axis=1)) * np.repeat(s, g, axis=1)
    return torch.from_numpy(w)


class TorchModel:
    def __init__(self, index_json: str, weights: np.ndarray, max_context: int = 4096):
        ix = json.loads(index_json)
        self.ix, self.buf = ix, weights.tobytes()
        c = dict(ix["config"])
        self.c = c
        self.W = {n: dequant(ix, self.buf, n) for n in ix["matrices"]}

        def vec(n):
            e = ix["tensors"][n]
            return torch.from_numpy(np.frombuffer(self.buf, dtype=np.float32, count=e["bytes"] // 4,
                                                  offset=e["offset"]).astype(np.float64))

        self.V = {n: vec(n) for n in ix["tensors"] if ix["tensors"][n]["kind"] == "f32"}
        self.max_context = max_context
        self.reset()

    def reset(self):
        c = self.c
        H, dk, dv = c["gdn_heads"], c["gdn_dk"], c["gdn_dv"]
        ch = 2 * H * dk + H * dv
        self.conv = {}
        self.S = {}
        self.K = {}
        self.Vc = {}
        for i in range(c["layers"]):
            if (i + 1) % c["full_attention_every"] == 0:
                self.K[i], self.Vc[i] = [], []
            else:
                self.conv[i] = torch.zeros(ch, c["conv_kernel"] - 1, dtype=D)
                self.S[i] = torch.zeros(H, dk, dv, dtype=D)

    def rms(self, x, w):
        return F.rms_norm(x, (x.shape[-1],), weight=w, eps=self.c.get("rms_eps", 1e-6))

    def gdn(self, i, proj):
        c = self.c
        H, dk, dv = c["gdn_heads"], c["gdn_dk"], c["gdn_dv"]
        ch = 2 * H * dk + H * dv
        w = self.V[f"layer{i}.conv_w"].reshape(ch, 1, c["conv_kernel"])
        seq = torch.cat([self.conv[i], proj[:ch, None]], dim=1)  # [ch, K]
        y = F.conv1d(seq[None], w, groups=ch)[0, :, -1]
        self.conv[i] = seq[:, 1:]
        y = F.silu(y)
        q = y[: H * dk].reshape(H, dk)
        k = y[H * dk: 2 * H * dk].reshape(H, dk)
        v = y[2 * H * dk:].reshape(H, dv)
        z = proj[ch: ch + H * dv].reshape(H, dv)
        a = proj[ch + H * dv: ch + H * dv + H]
        b = proj[ch + H * dv + H: ch + H * dv + 2 * H]
        prm = self.V[f"layer{i}.gdn_params"]
        dt, A, nw = prm[:H], prm[H:2 * H], prm[2 * H:]
        # L2 normalisation with the reference's 1e-6 inside the root (shaders.rs:489-492)
        nq = torch.linalg.vector_norm(q, dim=-1, keepdim=True)
        nk = torch.linalg.vector_norm(k, dim=-1, keepdim=True)
        q = q / torch.sqrt(nq * nq + 1e-6) / dk ** 0.5
        k = k / torch.sqrt(nk * nk + 1e-6)
        g = torch.exp(A * F.softplus(a + dt))
        beta = torch.sigmoid(b)
        out = torch.empty(H, dv, dtype=D)
        for h in range(H):
            S = self.S[i][h]
            kk = k[h][:, None]
            S = g[h] * (torch.eye(dk, dtype=D) - beta[h] * kk @ kk.T) @ S + beta[h] * kk @ v[h][None, :]
            self.S[i][h] = S
            out[h] = S.T @ q[h]
        o = F.rms_norm(out, (dv,), weight=nw, eps=1e-6) * F.silu(z)
        return o.reshape(-1)

    def rope(self, x, pos):
        c = self.c
        half = c["rope_dim"] // 2
        inv = np.array([np.float32(c["rope_theta"] ** (-(2 * j) / c["rope_dim"])) for j in range(half)], dtype=np.float32)
        ang = torch.from_numpy((np.float32(pos) * inv).astype(np.float64))
        zc = torch.complex(x[..., :half], x[..., half: 2 * half]) * torch.polar(torch.ones_like(ang), ang)
        y = x.clone()
        y[..., :half], y[..., half: 2 * half] = zc.real, zc.imag
        return y

    def attention(self, i, proj, pos):
        c = self.c
        nq, nkv, hd = c["n_q_heads"], c["n_kv_heads"], c["head_dim"]
        q = proj[: nq * hd].reshape(nq, hd)
        gate = proj[nq * hd: 2 * nq * hd].reshape(nq, hd)
        k = proj[2 * nq * hd: 2 * nq * hd + nkv * hd].reshape(nkv, hd)
        v = proj[2 * nq * hd + nkv * hd:].reshape(nkv, hd)
        norms = self.V[f"layer{i}.attn_norms"]
        q = self.rope(self.rms(q, norms[:hd]), pos)
        k = self.rope(self.rms(k, norms[hd:]), pos)
        # the cache holds f16 keys and values
        k16 = torch.from_numpy(k.numpy().astype(np.float32).astype(np.float16).astype(np.float64))
        v16 = torch.from_numpy(v.numpy().astype(np.float32).astype(np.float16).astype(np.float64))
        self.K[i].append(k16)
        self.Vc[i].append(v16)
        Kc = torch.stack(self.K[i], dim=1)  # [nkv, len, hd]
        Vc = torch.stack(self.Vc[i], dim=1)
        rep = nq // nkv
        Kq = Kc.repeat_interleave(rep, dim=0)
        Vq = Vc.repeat_interleave(rep, dim=0)
        o = F.scaled_dot_product_attention(q[:, None, :], Kq, Vq, scale=1.0 / hd ** 0.5)[:, 0, :]
        return (o * torch.sigmoid(gate)).reshape(-1)

    def token(self, tok, pos):
        c = self.c
        h = self.W["embed"][tok].clone()
        for i in range(c["layers"]):
            x = self.rms(h, self.V[f"layer{i}.input_norm"])
            proj = self.W[f"layer{i}.mixer_in"] @ x
            if (i + 1) % c["full_attention_every"] == 0:
                mixed = self.attention(i, proj, pos)
            else:
                mixed = self.gdn(i, proj)
            h = h + self.W[f"layer{i}.mixer_out"] @ mixed
            x = self.rms(h, self.V[f"layer{i}.post_norm"])
            gu = self.W[f"layer{i}.gate_up"] @ x
            I = c["intermediate"]
            h = h + self.W[f"layer{i}.down"] @ (F.silu(gu[:I]) * gu[I:])
        x = self.rms(h, self.V["final_norm"])
        return (self.W["lm_head"] @ x).numpy()
