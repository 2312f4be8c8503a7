"""Torch CPU restatement of the reference's CPU path -- TEST / BASELINE INFRASTRUCTURE ONLY.

Used by tests/ and by bench.py's cpu_baseline leg (timed on the host cores); never by the
product path. It restates PalettizedLinear's PyTorch fallback (qwen_model.py:183-192):
    flat_palette = palette.reshape(-1).to(x.dtype); gathered = flat_palette[_flat_idx]
    y = x_flat @ gathered (+ bias)
with _flat_idx = (n // group_size) * 4 + idx (qwen_model.py:97-102), plus QwenLoRA's
y += (x @ A) @ B^T * scaling (qwen_model.py:291-304); backward by torch autograd.
In the native layout ([N, K] weights, palette [N, K/256, 4]) the flat index is
group_id * 4 + idx with group_id = n * (K/256) + k // 256.
"""
from __future__ import annotations

import torch


def native_flat_idx(idx_nk: torch.Tensor) -> torch.Tensor:
    """idx [N, K] -> flat palette index for palette.reshape(-1) of a [N, K/256, 4] palette."""
    N, K = idx_nk.shape
    gid = torch.arange(N)[:, None] * (K // 256) + (torch.arange(K) // 256)[None, :]
    return (gid * 4 + idx_nk.long()).contiguous()


def palettized_linear_cpu(x, palette, flat_idx, bias=None, lora_a=None, lora_b=None,
                          scaling=1.0):
    """y = x @ W^T (+bias) (+ (x A^T) B^T * scaling), W = palette.flat[flat_idx] in x.dtype.
    x [M, K]; palette [N, K/256, 4]; flat_idx [N, K]; lora_a [r, K]; lora_b [N, r]."""
    flat_palette = palette.reshape(-1).to(x.dtype)
    gathered = flat_palette[flat_idx]          # [N, K]
    y = x @ gathered.t()
    if bias is not None:
        y = y + bias.to(x.dtype)
    if lora_a is not None:
        y = y + ((x @ lora_a.t()) @ lora_b.t()) * scaling
    return y


# ---- decoder-layer training step (CPU, fp32) -------------------------------------------------
import math as _math

import torch.nn.functional as _F


def _bf16(t):
    return t.to(torch.bfloat16).to(torch.float32)


class SoftLinearRef(torch.autograd.Function):
    """Reference soft palettized linear (fused_lut_linear_cuda.py:880-970 semantics) in the
    native layout: forward y = x W_hard^T with W_hard = pal[argmax_c P_c] (first max), P =
    softmax((logits + noise) / tau); backward grad_x = gy W_hard, grad_logits = dW P (pal -
    W_soft) (no 1/tau), grad_pal = sum over the 256-k group of dW P, dW = gy^T x."""

    @staticmethod
    def forward(ctx, x, palette, logits, noise, tau):
        N, K, _ = logits.shape
        P = torch.softmax((logits.float() + noise.float()) / tau, dim=-1)
        pw = palette.float().repeat_interleave(256, dim=1)[:, :K, :]
        am = torch.argmax(P, dim=-1, keepdim=True)
        w_hard = _bf16(torch.gather(pw, -1, am)[..., 0])
        ctx.save_for_backward(x, P, pw, w_hard)
        return x @ w_hard.t()

    @staticmethod
    def backward(ctx, gy):
        x, P, pw, w_hard = ctx.saved_tensors
        N, K, _ = P.shape
        dW = gy.t() @ x
        w_soft = (P * pw).sum(-1, keepdim=True)
        g_logits = dW[..., None] * P * (pw - w_soft)
        g_pal = (dW[..., None] * P).reshape(N, K // 256, 256, 4).sum(2)
        return gy @ w_hard, g_pal, g_logits, None, None


def rmsnorm_ref(x, w, eps):
    """HF Qwen3RMSNorm with bf16 storage of the normalised value and of the output."""
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return _bf16(w * _bf16(x * r))


def rope_ref(x, seq, theta):
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    f = torch.outer(torch.arange(seq, dtype=torch.float32), inv)
    emb = torch.cat([f, f], -1)
    c, s = emb.cos()[None, :, None, :], emb.sin()[None, :, None, :]
    rot = torch.cat([-x[..., d // 2:], x[..., : d // 2]], -1)
    return _bf16(x * c + rot * s)


def layer_forward_ref(p, hs, noises, tau, cfg):
    """Student layer forward on CPU. p: dict of fp32 tensors (requires_grad where trained):
    for each linear name: palette, logits, lora_a, lora_b, lora_scale; norm weights."""
    B, S, H = hs.shape

    def lin(name, x):
        q = p[name]
        x2 = x.reshape(-1, x.shape[-1])
        y = SoftLinearRef.apply(x2, q["palette"], q["logits"], noises[name], tau)
        t = _bf16(q["lora_scale"] * (x2 @ q["lora_a"].t()))
        return _bf16(y + t @ q["lora_b"].t()).reshape(*x.shape[:-1], -1)

    x = rmsnorm_ref(hs, p["input_layernorm"], cfg.eps)
    q = rmsnorm_ref(lin("q_proj", x).view(B, S, cfg.heads, cfg.head_dim), p["q_norm"], cfg.eps)
    k = rmsnorm_ref(lin("k_proj", x).view(B, S, cfg.kv_heads, cfg.head_dim), p["k_norm"], cfg.eps)
    v = lin("v_proj", x).view(B, S, cfg.kv_heads, cfg.head_dim)
    q, k = rope_ref(q, S, cfg.rope_theta), rope_ref(k, S, cfg.rope_theta)
    rep = cfg.heads // cfg.kv_heads
    o = _F.scaled_dot_product_attention(q.transpose(1, 2), k.repeat_interleave(rep, 2).transpose(1, 2),
                                        v.repeat_interleave(rep, 2).transpose(1, 2), is_causal=True)
    o = _bf16(o.transpose(1, 2).reshape(B, S, -1))
    hs = _bf16(hs + lin("o_proj", o))
    x = rmsnorm_ref(hs, p["post_attention_layernorm"], cfg.eps)
    g, u = lin("gate_proj", x), lin("up_proj", x)
    h = _bf16(_bf16(_F.silu(g)) * u)
    return _bf16(hs + lin("down_proj", h))


def teacher_forward_ref(w, hs, cfg):
    B, S, H = hs.shape

    def lin(name, x):
        return _bf16(x @ w[name].t())

    x = rmsnorm_ref(hs, w["input_layernorm"], cfg.eps)
    q = rmsnorm_ref(lin("q_proj", x).view(B, S, cfg.heads, cfg.head_dim), w["q_norm"], cfg.eps)
    k = rmsnorm_ref(lin("k_proj", x).view(B, S, cfg.kv_heads, cfg.head_dim), w["k_norm"], cfg.eps)
    v = lin("v_proj", x).view(B, S, cfg.kv_heads, cfg.head_dim)
    q, k = rope_ref(q, S, cfg.rope_theta), rope_ref(k, S, cfg.rope_theta)
    rep = cfg.heads // cfg.kv_heads
    o = _F.scaled_dot_product_attention(q.transpose(1, 2), k.repeat_interleave(rep, 2).transpose(1, 2),
                                        v.repeat_interleave(rep, 2).transpose(1, 2), is_causal=True)
    hs = _bf16(hs + lin("o_proj", _bf16(o.transpose(1, 2).reshape(B, S, -1))))
    x = rmsnorm_ref(hs, w["post_attention_layernorm"], cfg.eps)
    return _bf16(hs + lin("down_proj", _bf16(_bf16(_F.silu(lin("gate_proj", x))) * lin("up_proj", x))))


def compute_loss_ref(s, t):
    """train_qwen.py:229-249, weights 0.5 / 0.5."""
    cos_per = _F.cosine_similarity(s.flatten(0, 1), t.flatten(0, 1), dim=-1, eps=1e-4)
    l_cos = (1 - cos_per).mean()
    l_mse = ((s - t) ** 2).mean() / (t * t).mean().clamp(min=1e-6)
    return 0.5 * l_cos + 0.5 * l_mse
