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
