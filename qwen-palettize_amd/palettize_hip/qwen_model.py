"""PalettizedLinear and QwenLoRA with the reference's constructor API and attributes
(qwen_model.py:65-304), running on the MI355X kernels.

PalettizedLinear keeps the reference's buffers and parameters -- indices (in, out) int64
((out, in) when pre_transposed), indices_int8, _flat_idx, palette (G, 4) bf16, index_logits
(4, in, out) fp16 (+-10 one-hot, only with use_soft_indices), tau, group_size, n_groups,
palette_size, pre_transposed, in_features, out_features, bias -- and dispatches like
qwen_model.py:147-196: soft (Gumbel-softmax, straight-through) in training mode with soft
indices, hard otherwise. soft_semantics picks which of the reference's soft implementations
the soft forward follows: "cuda" (its CUDA-C kernels) or "triton" (its Triton kernels).
Palette groups run along the stored indices' second dimension: the output dimension
normally, the input dimension when pre_transposed (qwen_model.py:97-102).
Both dispatch to the drop-in fused_lut_linear_cuda functions; there is no CPU fallback
(a CPU input raises).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import fused_lut_linear_cuda as FL


class PalettizedLinear(nn.Module):
    def __init__(self, original_linear, indices, n_groups, palette_size, group_size,
                 pre_transposed, initial_palette=None, use_soft_indices=False,
                 soft_semantics="cuda"):
        super().__init__()
        if soft_semantics not in FL.SEMANTICS:
            raise ValueError(f"soft_semantics must be one of {FL.SEMANTICS}")
        # which of the reference's soft implementations this module follows: its CUDA-C one
        # ("cuda") or its Triton one ("triton", which the reference prefers when triton
        # imports, qwen_model.py:111-128); the flags mirror the reference's attributes
        self.soft_semantics = soft_semantics
        self._use_triton = not pre_transposed and soft_semantics == "triton"
        self._use_cuda = not pre_transposed and soft_semantics == "cuda"
        self.register_buffer("indices", indices.long())
        self.register_buffer("indices_int8", indices.to(torch.int8).contiguous())
        self.palette = nn.Parameter(
            initial_palette.clone().to(torch.bfloat16) if initial_palette is not None
            else torch.zeros(n_groups, palette_size, dtype=torch.bfloat16, device=indices.device))
        self.group_size = group_size
        self.n_groups = n_groups
        self.palette_size = palette_size
        self.pre_transposed = pre_transposed
        self.in_features = original_linear.in_features
        self.out_features = original_linear.out_features
        if original_linear.bias is not None:
            self.register_buffer("bias", original_linear.bias.data.clone().to(torch.bfloat16))
        else:
            self.register_buffer("bias", None)
        si, so = indices.shape
        group_idx = torch.arange(so, device=indices.device) // group_size
        self.register_buffer("_flat_idx",
                             (group_idx.unsqueeze(0).expand(si, so) * palette_size + indices).contiguous())
        self.use_soft_indices = use_soft_indices
        self.tau = 1.0
        if use_soft_indices and not pre_transposed:
            K_dim, N_dim = indices.shape
            logits = torch.full((4, K_dim, N_dim), -10.0, dtype=torch.float16, device=indices.device)
            for k in range(4):
                logits[k][indices == k] = 10.0
            self.index_logits = nn.Parameter(logits)
        else:
            self.index_logits = None

    def forward(self, x):
        if not x.is_cuda:
            raise RuntimeError("PalettizedLinear: palettize_hip runs on the GPU only (no CPU path)")
        orig_ndim = x.ndim
        x_flat = x.reshape(-1, x.shape[-1]) if x.ndim == 3 else x
        if self.training and self.use_soft_indices and self.index_logits is not None:
            y = FL.fused_lut_linear_soft(x_flat, self.palette, self.index_logits, self.bias,
                                         self.group_size, self.tau,
                                         semantics=self.soft_semantics)
        elif self.pre_transposed:
            # indices (out, in), palette groups along the input dimension (qwen_model.py:187-190)
            y = FL.fused_lut_linear_pre_transposed(x_flat, self.palette, self.indices_int8,
                                                   self.bias, self.group_size)
        else:
            y = FL.fused_lut_linear(x_flat, self.palette, self.indices_int8, self.bias,
                                    self.group_size)
        if orig_ndim == 3:
            y = y.reshape(x.shape[0], x.shape[1], -1)
        return y

    def extract_hard_indices(self):
        """argmax over the 4 logit planes -> frozen indices (qwen_model.py:198-209)."""
        if self.index_logits is not None:
            with torch.no_grad():
                self.indices = self.index_logits.argmax(dim=0).long()
                self.indices_int8 = self.indices.to(torch.int8).contiguous()
                del self.index_logits
                self.index_logits = None
                self.use_soft_indices = False


class QwenLoRA(nn.Module):
    """y = base(x) + (alpha / r) * (x @ A) @ B^T with A (in, r), B (out, r) bf16
    (qwen_model.py:213-304). init 'loftq' uses the SVD of the palettization residual."""

    def __init__(self, base_module, rank=32, alpha=64, init="loftq", original_weight=None):
        super().__init__()
        self.base = base_module
        self.rank = rank
        self.alpha = alpha
        self.scaling = alpha / rank
        if hasattr(base_module, "in_features"):
            in_dim, out_dim = base_module.in_features, base_module.out_features
        else:
            out_dim, in_dim = base_module.weight.shape
        if hasattr(base_module, "weight"):
            device = base_module.weight.device
        elif hasattr(base_module, "palette"):
            device = base_module.palette.device
        else:
            device = next(base_module.parameters()).device
        if init == "loftq" and original_weight is not None:
            with torch.no_grad():
                if hasattr(base_module, "palette"):
                    # (in, out) for either orientation; the residual is taken as (out, in)
                    w_oi = self._reconstruct_base_weight(base_module).float().t()
                else:
                    w_oi = base_module.weight.data.float()
                R = original_weight.float().to(w_oi.device) - w_oi
                U, S, Vh = torch.linalg.svd(R, full_matrices=False)
                B_init = (U[:, :rank] * S[:rank].sqrt().unsqueeze(0)).contiguous()
                A_init = (Vh[:rank, :].T * S[:rank].sqrt().unsqueeze(0)).contiguous()
                A_init = A_init / math.sqrt(self.scaling)
                B_init = B_init / math.sqrt(self.scaling)
        else:
            A_init = torch.randn(in_dim, rank) * 0.01
            B_init = torch.zeros(out_dim, rank)
        self.lora_A = nn.Parameter(A_init.to(torch.bfloat16).to(device))
        self.lora_B = nn.Parameter(B_init.to(torch.bfloat16).to(device))

    @staticmethod
    def _reconstruct_base_weight(pal_module):
        """The palettized weight as (in, out): the flat gather palette[(c // GS) * 4 + idx]
        over the stored (rows, cols) indices, transposed back when they are (out, in)
        (qwen_model.py:278-289)."""
        gathered = pal_module.palette.reshape(-1)[pal_module._flat_idx]
        return gathered if not pal_module.pre_transposed else gathered.T

    def forward(self, x):
        if not x.is_cuda:
            raise RuntimeError("QwenLoRA: palettize_hip runs on the GPU only (no CPU path)")
        from . import ops
        y_base = self.base(x)
        lead = x.shape[:-1]
        x_flat = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()
        lora = _LoRAFunction.apply(x_flat, self.lora_A, self.lora_B, self.scaling)
        return y_base + lora.reshape(*lead, -1).to(y_base.dtype)


class _LoRAFunction(torch.autograd.Function):
    """scale * (x A) B^T with A (in, r), B (out, r) on the skinny HIP GEMMs."""

    @staticmethod
    def forward(ctx, x, A, B, scale):
        from . import ops
        a_rk = A.t().contiguous()          # [r, K]
        b_nr = B.contiguous()              # [N, r]
        t = ops.lora_project(x, a_rk, scale)   # s * x A   [M, r]
        y = ops.linear_fwd_dense(t, b_nr)      # t B^T     [M, N]
        ctx.save_for_backward(x, a_rk, b_nr, t)
        ctx.scale = scale
        return y

    @staticmethod
    def backward(ctx, gy):
        from . import ops
        x, a_rk, b_nr, t = ctx.saved_tensors
        gy = gy.contiguous()
        gt = ops.lora_grad_t(gy, b_nr, ctx.scale)            # s * gy B   [M, r]
        gx = ops.linear_bwd_x_dense(gt, a_rk) if ctx.needs_input_grad[0] else None  # gt A^T
        ga, gb = ops.lora_weight_grads(x, gy, t, gt, 1.0, out_dtype=torch.bfloat16)
        return gx, ga.t(), gb, None
