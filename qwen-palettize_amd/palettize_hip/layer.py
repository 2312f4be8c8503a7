"""One palettized Qwen3-shaped decoder layer and its distillation training step.

The layer is HF Qwen3DecoderLayer's math (transformers models/qwen3/modeling_qwen3.py:
RMSNorm :50-64, MLP :70-83, attention with per-head q/k RMSNorm and RoPE :140-160,211-318)
with every linear replaced by a Gumbel-softmax palettized linear + LoRA, as the reference
trains it (train_qwen.py:993-1414, qwen_model.py:65-304):

  * linears: SoftPalettizedLinear -- logits [N, K, 4] (bf16), palette fp32 [N, K/256, 4],
    LoRA A [r, K] / B [N, r] (bf16), straight-through forward through W_hard;
    HIP kernels for build-W, the GEMMs and the fused soft backward;
  * RMSNorm and SwiGLU: HIP kernels (plz_rmsnorm_*, plz_swiglu_*);
  * RoPE and causal grouped-query attention: HIP kernels (plz_rope_*, plz_attn_*; head_dim
    128 and sequences a multiple of 128 -- other attention shapes run torch's flash /
    memory-efficient SDPA kernels on the GPU);
  * loss: 0.5 * (1 - cos) + 0.5 * norm_mse against a dense bf16 teacher layer
    (compute_loss, train_qwen.py:229-249), HIP kernels (plz_distill_loss_*); the teacher's
    projections run on the same MFMA GEMM core (plz_linear_fwd_dense, gate/up with the SwiGLU
    in the epilogue);
  * optimizer: AdamW (betas 0.9/0.95, eps 1e-8, wd 0) on fp32 masters of palettes, LoRA and
    logits (FP32MasterOptimizer, train_qwen.py:154-221), two-tier gradient clipping
    (logits 1.0, others 0.3; train_qwen.py:1303-1319), logits clamp +-5 tau after the step
    (train_qwen.py:1343-1348), tau schedule of train_qwen.py:1176-1192.
Everything runs on the GPU: CPU tensors (or non-bf16 activations) raise, there is no CPU
path.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from ._lib import PLZ_W_HARD_NOISY
from .functional import SoftLUTLinearFunction
from .optim import FusedAdamW, NextBuild


def _gpu_bf16(t, what):
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.bfloat16):
        raise RuntimeError(f"{what} must be a bf16 GPU tensor (palettize_hip has no CPU path)")


@dataclass
class LayerConfig:
    hidden: int = 2560
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    eps: float = 1e-6
    rope_theta: float = 1e6
    lora_rank: int = 16
    lora_alpha: float = 16.0   # scaling alpha / r = 1 (y += x A^T B^T)


# ---- fused kernels as autograd Functions ----------------------------------------------
class RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        y, rstd = ops.rmsnorm_fwd(x2, weight.contiguous(), eps)
        ctx.save_for_backward(x2, weight, rstd)
        ctx.shape = shape
        return y.reshape(shape)

    @staticmethod
    def backward(ctx, gy):
        x2, weight, rstd = ctx.saved_tensors
        gx, gw = ops.rmsnorm_bwd(x2, weight.contiguous(), rstd,
                                 gy.reshape(x2.shape).contiguous())
        return gx.reshape(ctx.shape), (gw.to(weight.dtype) if ctx.needs_input_grad[1] else None), None


class AddRMSNormFunction(torch.autograd.Function):
    """(s, norm(s)) with s = a + b (a residual add and the RMSNorm after it, frozen weight):
    plz_add_rmsnorm_fwd, and plz_rmsnorm_bwd_add for the gradient of s along both uses."""

    @staticmethod
    def forward(ctx, a, b, weight, eps):
        shape = a.shape
        s, y, rstd = ops.add_rmsnorm_fwd(a.reshape(-1, shape[-1]).contiguous(),
                                         b.reshape(-1, shape[-1]).contiguous(), weight, eps)
        ctx.save_for_backward(s, weight, rstd)
        ctx.shape = shape
        return s.view(shape), y.view(shape)

    @staticmethod
    def backward(ctx, gs, gy):
        s, weight, rstd = ctx.saved_tensors
        if gy is None:
            g = gs
        else:
            gy2 = gy.reshape(s.shape).contiguous()
            if gs is None:
                g, _ = ops.rmsnorm_bwd(s, weight, rstd, gy2)
            else:
                g = ops.rmsnorm_bwd_add(s, weight, rstd, gy2, gs.reshape(s.shape).contiguous())
            g = g.view(ctx.shape)
        return g, g, None, None


def add_rmsnorm(norm, a, b):
    """(a + b, norm(a + b)): one fused pass for a frozen norm weight on bf16 GPU tensors."""
    if (not norm.weight.requires_grad and a.is_cuda and a.dtype == torch.bfloat16
            and b.dtype == torch.bfloat16 and a.shape == b.shape):
        return AddRMSNormFunction.apply(a, b, norm.weight, norm.eps)
    s = a + b
    return s, norm(s)


class RMSNorm(nn.Module):
    def __init__(self, dim, eps, device=None):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, dtype=torch.bfloat16, device=device),
                                   requires_grad=False)
        self.eps = eps

    def forward(self, x):
        return RMSNormFunction.apply(x, self.weight, self.eps)


class SwiGLUCatFunction(torch.autograd.Function):
    """h = silu(gate) * up from a fused projection's output [..., 2F] = [gate | up]."""

    @staticmethod
    def forward(ctx, gate_up):
        gate_up = gate_up.contiguous()
        ctx.save_for_backward(gate_up)
        return ops.swiglu_fwd_cat(gate_up)

    @staticmethod
    def backward(ctx, gh):
        (gate_up,) = ctx.saved_tensors
        return ops.swiglu_bwd_cat(gate_up, gh.contiguous())


class SwiGLUFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        gate, up = gate.contiguous(), up.contiguous()
        ctx.save_for_backward(gate, up)
        return ops.swiglu_fwd(gate, up)

    @staticmethod
    def backward(ctx, gh):
        gate, up = ctx.saved_tensors
        return ops.swiglu_bwd(gate, up, gh.contiguous())


class RopeFunction(torch.autograd.Function):
    """apply_rope on the GPU: plz_rope_fwd / plz_rope_bwd (bit-exact with the torch expression)."""

    @staticmethod
    def forward(ctx, x, cos, sin):
        ctx.save_for_backward(cos, sin)
        return ops.rope_fwd(x.contiguous(), cos, sin)

    @staticmethod
    def backward(ctx, gy):
        cos, sin = ctx.saved_tensors
        return ops.rope_bwd(gy.contiguous(), cos, sin), None, None


class DistillLossFunction(torch.autograd.Function):
    """compute_loss on the GPU: one pass for the per-row sums, one for grad_student."""

    @staticmethod
    def forward(ctx, s, t, w_cos, w_mse):
        s, t = s.contiguous(), t.contiguous()
        out, ws = ops.distill_loss_fwd(s, t, w_cos, w_mse, 1e-4)
        ctx.save_for_backward(s, t, out, ws)
        ctx.w = (w_cos, w_mse)
        ctx.mark_non_differentiable(out)
        return out[0], out

    @staticmethod
    def backward(ctx, g_loss, _g_out):
        s, t, out, ws = ctx.saved_tensors
        gs = ops.distill_loss_bwd(s, t, out, ws, g_loss, ctx.w[0], ctx.w[1], 1e-4)
        return gs, None, None, None


# ---- palettized linear (native layout, soft path) ----------------------------------------
NOISE_STRIDE = 1 << 32  # Philox counters consumed per forward of a soft linear (> N * K)


class GradSq:
    """The squared-gradient sums of a soft linear's (or a group's) logits, one fp32 per 512
    consecutive gradient values (row n, 128 k), written by its backward's soft dW
    (ops.soft_bwd_lora grad_sq) for the optimizer's clip norm; ``writes`` counts the backward
    passes that wrote it since it was last reset, so a reader knows the sums are those of one
    gradient."""

    def __init__(self, rows, K, device):
        self.buf = torch.empty(rows * (K // 128), dtype=torch.float32, device=device)
        self.writes = 0

    def rows(self, r0, n, K):
        return self.buf[r0 * (K // 128):(r0 + n) * (K // 128)]


class SoftPalettizedLinear(nn.Module):
    """y = x W_ste^T + s (x A^T) B^T with W from logits + Gumbel noise + palette.

    Parameters: logits bf16 [N, K, 4] (initialised one-hot +-10 from `indices`, like
    qwen_model.py:135-143), palette fp32 [N, K/256, 4], lora_a bf16 [r, K] ~ N(0, 0.01),
    lora_b bf16 [N, r] (zeros unless given). The noise is regenerated every forward from a
    Philox stream (seed, counter) so steps are reproducible."""

    def __init__(self, in_features, out_features, indices=None, palette=None, rank=16,
                 lora_scale=1.0, seed=0, device=None, lora_b_std=0.0):
        super().__init__()
        N, K = out_features, in_features
        self.in_features, self.out_features = K, N
        g = torch.Generator(device="cpu").manual_seed(seed)
        if indices is None:
            indices = torch.randint(0, 4, (N, K), generator=g, dtype=torch.uint8)
        if palette is None:
            palette = torch.sort(torch.randn(N, K // 256, 4, generator=g) * 0.02, -1).values
        onehot = F.one_hot(indices.long(), 4).bool()
        logits = torch.where(onehot, torch.tensor(10.0), torch.tensor(-10.0))
        self.index_logits = nn.Parameter(logits.to(torch.bfloat16).to(device).contiguous())
        self.palette = nn.Parameter(palette.float().to(device).contiguous())
        self.lora_a = nn.Parameter((torch.randn(rank, K, generator=g) * 0.01)
                                   .to(torch.bfloat16).to(device))
        self.lora_b = nn.Parameter((torch.randn(N, rank, generator=g) * lora_b_std)
                                   .to(torch.bfloat16).to(device))
        self.lora_scale = lora_scale
        self.tau = 1.0
        self.noise_seed = seed
        self.noise_counter = 0
        self.mode = PLZ_W_HARD_NOISY
        self.grad_sq = None  # a GradSq: the backward writes the logits' squared-gradient sums

    def next_noise_spec(self):
        """The next forward's noise as a Philox descriptor (drawn inside the kernels): key
        noise_seed, counters noise_counter + n*K + k. The counter advances by NOISE_STRIDE per
        forward (more than any N*K), so linears that start together stay on the same offset and
        one batched build serves them all, decorrelated by their keys."""
        off = self.noise_counter
        self.noise_counter += NOISE_STRIDE
        return ops.PhiloxNoise(self.noise_seed, off)

    def forward(self, x, prebuilt=None, residual=None, swiglu=None):
        """prebuilt: (w, group) from the layer's batched build of this forward (the noise
        counter has then been advanced by the layer). residual (optional, bf16 [..., N]): added
        to the output in the GEMM's epilogue (the layer's residual add after its down
        projection). swiglu (optional SwiGLULink): x is that SwiGLU's output, and the grad_x
        GEMM runs its backward in the epilogue."""
        _gpu_bf16(x, "SoftPalettizedLinear input")
        lead = x.shape[:-1]
        if prebuilt is None:
            noise = self.next_noise_spec()
        else:
            w, group, noise = prebuilt[:3]
            probs = prebuilt[3] if len(prebuilt) > 3 else None
            prebuilt = (w, group, self.grad_sq, probs)
        res = None if residual is None else residual.reshape(-1, self.out_features)
        y = SoftLUTLinearFunction.apply(x.reshape(-1, x.shape[-1]), self.palette, self.index_logits,
                                        noise, self.tau, None, self.lora_a, self.lora_b,
                                        self.lora_scale, self.mode, False, prebuilt, res,
                                        swiglu)
        return y.reshape(*lead, self.out_features)


class SoftLinearGroup:
    """Sibling soft linears on the same input (the MLP's gate and up) run as one soft linear over
    their concatenated output rows: one build-W descriptor, one dense GEMM whose LoRA stage takes
    the parts' A stacked ([sum r, K]) and their B block-diagonal ([sum N, sum r], zeros off the
    blocks), and one soft backward whose LoRA weight gradients come out of the same dW tiles.
    Row n of the group is row n of its part, with that part's logits, palette and LoRA, so the
    result is the parts' own linears; the difference is scheduling: the fused dW GEMM has
    enough output tiles to fill the GPU without splitting its reduction (for gate and up at
    hidden 2560: 760 tiles instead of twice 380), which saves the split's fp32 partials and
    second pass, and the LoRA and grad_x work runs once.

    The parts keep their parameters (state_dict names, optimizer groups), re-homed as row
    slices of one storage each for the logits, the palettes and the LoRA A, so the group reads
    them without copies; a part whose parameter was replaced rather than written in place is
    concatenated instead. The noise is one Philox stream over the group's rows (part 0's key at
    the shared counter offset): part p's rows continue part p-1's counters, which each part's
    noise_seed / noise_counter report, so part p alone would draw the same values.
    """

    def __init__(self, parts):
        if len(parts) < 2:
            raise ValueError("a group needs at least two linears")
        K = parts[0].in_features
        if any(p.in_features != K for p in parts):
            raise ValueError("grouped linears must share their input")
        self.parts = list(parts)
        self.rows = [p.out_features for p in parts]
        self.ranks = [p.lora_a.shape[0] for p in parts]
        self.N, self.K, self.R = sum(self.rows), K, sum(self.ranks)
        if len({p.lora_scale for p in parts}) != 1:
            raise ValueError("grouped linears must share the LoRA scale")
        if any(n % 256 for n in self.rows[:-1]):
            raise ValueError("every part but the last must have a multiple of 256 rows")
        for attr in ("index_logits", "palette", "lora_a"):
            base = torch.cat([getattr(p, attr).detach() for p in parts], 0).contiguous()
            r = 0
            for p in parts:
                n = getattr(p, attr).shape[0]
                setattr(p, attr, nn.Parameter(base[r:r + n]))
                r += n
        seed = parts[0].noise_seed
        for p in parts:
            p.noise_seed = seed
        self._sync_counters()
        dev = parts[0].lora_b.device
        self._b_bd = torch.zeros(self.N, self.R, dtype=torch.bfloat16, device=dev)
        self.grad_sq = None  # a GradSq over the group's rows, as SoftPalettizedLinear.grad_sq

    def _sync_counters(self):
        c = self.parts[0].noise_counter
        for p, n in zip(self.parts, self.rows):
            p.noise_counter = c
            c += n * self.K

    @property
    def lora_scale(self):
        return self.parts[0].lora_scale

    @staticmethod
    def _rows_of(tensors):
        """The row-stacked tensor of `tensors`: a view when they are consecutive row slices of
        one storage, else a copy."""
        t0 = tensors[0]
        es = t0.element_size()
        ptr = t0.data_ptr()
        for t in tensors:
            if not t.is_contiguous() or t.data_ptr() != ptr or t.dtype != t0.dtype:
                return torch.cat([x.detach() for x in tensors], 0)
            ptr += t.numel() * es
        rows = sum(t.shape[0] for t in tensors)
        return torch.as_strided(t0.detach(), (rows,) + tuple(t0.shape[1:]), t0.stride())

    def logits(self):
        return self._rows_of([p.index_logits for p in self.parts])

    def palette(self):
        return self._rows_of([p.palette for p in self.parts])

    def lora_a(self):
        return self._rows_of([p.lora_a for p in self.parts])

    def lora_b(self):
        """The block-diagonal B [sum N, sum r] of this forward (its own buffer, off-block zeros)."""
        r0 = c0 = 0
        for p, n, r in zip(self.parts, self.rows, self.ranks):
            self._b_bd[r0:r0 + n, c0:c0 + r].copy_(p.lora_b.detach())
            r0 += n
            c0 += r
        return self._b_bd

    def next_noise_spec(self):
        spec = self.parts[0].next_noise_spec()
        for p in self.parts[1:]:
            p.next_noise_spec()
        self._sync_counters()
        return spec

    def _params(self):
        params = []
        for p in self.parts:
            params += [p.palette, p.index_logits, p.lora_a, p.lora_b]
        return params

    def forward(self, x, prebuilt):
        _gpu_bf16(x, "SoftLinearGroup input")
        lead = x.shape[:-1]
        y = SoftLinearGroupFunction.apply(x.reshape(-1, x.shape[-1]), self, prebuilt,
                                          *self._params())
        return y.reshape(*lead, self.N)

    def forward_swiglu(self, x, prebuilt, link=None):
        """silu(gate) * up of a [gate | up] group from one GEMM (the SwiGLU in its epilogue):
        the same values as SwiGLUCatFunction over forward(x, prebuilt), bit for bit. link
        (optional SwiGLULink): receives the pre-activations, so that the consumer's grad_x GEMM
        can run the SwiGLU backward."""
        _gpu_bf16(x, "SoftLinearGroup input")
        if len(self.parts) != 2 or self.rows[0] != self.rows[1] or self.rows[0] % 128:
            raise ValueError("forward_swiglu needs two parts of equal rows, a multiple of 128")
        lead = x.shape[:-1]
        h = SoftGateUpSwiGLUFunction.apply(x.reshape(-1, x.shape[-1]), self, prebuilt, link,
                                           *self._params())
        return h.reshape(*lead, self.N // 2)


class SoftLinearGroupFunction(torch.autograd.Function):
    """Autograd of SoftLinearGroup: inputs x, the group, the prebuilt (w, build group, noise) of
    this forward, then per part palette, logits, lora_a, lora_b; every part's gradients are row
    slices of the fused ones (grad_B the part's diagonal block)."""

    @staticmethod
    def _setup(ctx, x, grp, prebuilt):
        """(x, w, t, b) of this forward; records what the backward needs besides the saved
        tensors."""
        x = x.contiguous()
        w, build, noise = prebuilt[:3]
        ctx.probs = prebuilt[3] if len(prebuilt) > 3 else None
        ctx.guard = (build, build.generation)
        a, b = grp.lora_a(), grp.lora_b()
        t = ops.lora_project(x, a, grp.lora_scale)
        ctx.grp, ctx.noise, ctx.tau = grp, noise, float(grp.parts[0].tau)
        return x, w, a, b, t

    @staticmethod
    def forward(ctx, x, grp, prebuilt, *params):
        x, w, a, b, t = SoftLinearGroupFunction._setup(ctx, x, grp, prebuilt)
        y = ops.linear_fwd_dense(x, w, None, t, b)
        ctx.save_for_backward(x, grp.palette(), grp.logits(), w, a, b.clone())
        return y

    @staticmethod
    def backward(ctx, gy):
        return SoftLinearGroupFunction._backward(ctx, gy, *ctx.saved_tensors)

    @staticmethod
    def _backward(ctx, gy, x, pal, logits, w, a, b):
        grp = ctx.grp
        if ctx.guard[0].generation != ctx.guard[1]:
            raise RuntimeError("the prebuilt soft weight of this forward was rebuilt by a later "
                               "forward before this backward ran")
        gy = gy.contiguous()
        scale = grp.lora_scale
        grad_x = None
        if ctx.needs_input_grad[0]:
            gt = ops.lora_grad_t(gy, b, scale)
            grad_x = ops.linear_bwd_x_dense(gy, w, gt, a)
        sq = grp.grad_sq
        gl, gp, ga, gb = ops.soft_bwd_lora(x, gy, logits, ctx.noise, pal, ctx.tau, a, b, scale,
                                           False, out_dtype=a.dtype,
                                           grad_sq=sq.buf if sq is not None else None,
                                           probs=ctx.probs)
        if sq is not None:
            sq.writes += 1
        grads = []
        r0 = c0 = 0
        for n, r in zip(grp.rows, grp.ranks):
            grads += [gp[r0:r0 + n], gl[r0:r0 + n], ga[c0:c0 + r], gb[r0:r0 + n, c0:c0 + r].contiguous()]
            r0 += n
            c0 += r
        return (grad_x, None, None, *grads)


class SwiGLULink:
    """Hands the SwiGLU's backward to the grad_x GEMM of the linear that consumes its output
    (plz_linear_bwd_x_dense_swiglu): the SwiGLU's forward sets ``pre`` ([gate | up]
    pre-activations), that linear's backward sets ``grad`` ([grad_gate | grad_up]) and returns a
    placeholder grad_h whose data_ptr is ``marker``; the SwiGLU's backward takes ``grad`` when it
    receives that placeholder and raises if it receives anything else (grad_h accumulated from
    another consumer), since the placeholder holds no values."""

    def __init__(self):
        self.pre = self.grad = self.marker = None


class SoftGateUpSwiGLUFunction(torch.autograd.Function):
    """A [gate | up] SoftLinearGroup followed by the SwiGLU, as one GEMM whose epilogue writes
    both the pre-activations (kept for the backward) and h (plz_linear_fwd_dense_swiglu_cat).
    The backward is the SwiGLU's (plz_swiglu_bwd_rows) and then the group's own."""

    @staticmethod
    def forward(ctx, x, grp, prebuilt, link, *params):
        x, w, a, b, t = SoftLinearGroupFunction._setup(ctx, x, grp, prebuilt)
        y, h = ops.linear_fwd_dense_swiglu_cat(x, w, t, b)
        ctx.save_for_backward(x, grp.palette(), grp.logits(), w, a, b.clone(), y)
        ctx.link = link
        if link is not None:
            link.pre, link.grad, link.marker = y, None, None
        return h

    @staticmethod
    def backward(ctx, gh):
        x, pal, logits, w, a, b, y = ctx.saved_tensors
        link = ctx.link
        if link is not None and link.grad is not None:
            if gh.data_ptr() != link.marker:
                raise RuntimeError("the SwiGLU's output gradient did not come only from the linear "
                                   "that computed its backward (SwiGLULink)")
            gy = link.grad
            link.pre = link.grad = link.marker = None
        else:
            gy = ops.swiglu_bwd_cat(y, gh.contiguous())
        del y
        r = SoftLinearGroupFunction._backward(ctx, gy, x, pal, logits, w, a, b)
        return (*r[:3], None, *r[3:])  # no gradient for the link


# ---- RoPE / attention -------------------------------------------------------------------------
def rope_tables(seq, head_dim, theta, device):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    t = torch.arange(seq, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


class HeadNormRopeFunction(torch.autograd.Function):
    """apply_rope(norm(x)) for a per-head RMSNorm with a frozen weight: plz_head_norm_rope_fwd /
    _bwd, bit-identical to RMSNormFunction followed by RopeFunction."""

    @staticmethod
    def forward(ctx, x, weight, eps, cos, sin):
        x = x.contiguous()
        y, rstd = ops.head_norm_rope_fwd(x, weight, cos, sin, eps)
        ctx.save_for_backward(x, weight, rstd, cos, sin)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight, rstd, cos, sin = ctx.saved_tensors
        return ops.head_norm_rope_bwd(x, weight, rstd, cos, sin, gy.contiguous()), None, None, None, None


def norm_rope(norm, x, cos, sin):
    """apply_rope(norm(x)): one fused pass for a frozen 128-wide per-head norm, else the two."""
    if (not norm.weight.requires_grad and x.shape[-1] == 128 and x.is_cuda
            and x.dtype == torch.bfloat16):
        return HeadNormRopeFunction.apply(x, norm.weight, norm.eps, cos, sin)
    return apply_rope(norm(x), cos, sin)


def apply_rope(x, cos, sin):
    """x bf16 [B, S, H, D] on the GPU: HF's rotate_half embedding (x cos + rotate_half(x) sin),
    computed in fp32 with fp32 tables, rounded once to bf16 (plz_rope_fwd / plz_rope_bwd)."""
    _gpu_bf16(x, "apply_rope input")
    return RopeFunction.apply(x, cos, sin)


_GQA_NATIVE = [True]  # cleared when the SDPA backend refuses enable_gqa


class AttentionFunction(torch.autograd.Function):
    """Causal grouped-query attention on the GPU: plz_attn_fwd (o and the row log-sum-exp) and
    plz_attn_bwd (dQ, and dK / dV summed over the query heads of each kv head)."""

    @staticmethod
    def forward(ctx, q, k, v):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        o, lse = ops.attn_fwd(q, k, v)
        ctx.save_for_backward(q, k, v, o, lse)
        return o

    @staticmethod
    def backward(ctx, go):
        q, k, v, o, lse = ctx.saved_tensors
        return ops.attn_bwd(q, k, v, o, lse, go.contiguous())


def native_attention_ok(q, k):
    """The attention kernels' shapes: bf16 GPU tensors, head_dim 128, seq a multiple of 128."""
    return (q.is_cuda and q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
            and q.shape[-1] == 128 and q.shape[1] % 128 == 0)


def attention(q, k, v, heads, kv_heads):
    """q [B,S,H,D], k/v [B,S,Hkv,D] -> [B,S,H*D]; causal, grouped-query (kv repeated).
    The HIP kernels run where their shape constraints hold; torch SDPA otherwise."""
    B, S, H, D = q.shape
    rep = heads // kv_heads
    if native_attention_ok(q, k):
        if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
            o = AttentionFunction.apply(q, k, v)
        else:
            o, _ = ops.attn_fwd(q.contiguous(), k.contiguous(), v.contiguous())
        return o.view(B, S, H * D)
    _gpu_bf16(q, "attention query")
    qt = q.transpose(1, 2)
    # other shapes: torch's flash / memory-efficient kernels on the GPU only (the math
    # fallback issues bf16 batched products on transposed operands, which this pool does not
    # run reliably)
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        o = None
        if _GQA_NATIVE[0]:
            try:  # grouped-query heads without materialising the repeated k / v
                o = F.scaled_dot_product_attention(qt, k.transpose(1, 2), v.transpose(1, 2),
                                                   is_causal=True, enable_gqa=True)
            except RuntimeError:
                _GQA_NATIVE[0] = False
        if o is None:
            kt = k.repeat_interleave(rep, dim=2).transpose(1, 2)
            vt = v.repeat_interleave(rep, dim=2).transpose(1, 2)
            o = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
    return o.transpose(1, 2).reshape(B, S, H * D)


# ---- the layers -------------------------------------------------------------------------------
class PalettizedDecoderLayer(nn.Module):
    NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, cfg: LayerConfig, seed=0, device=None, lora_b_std=0.0, fuse_gate_up=True):
        super().__init__()
        self.cfg = cfg
        h, hd = cfg.hidden, cfg.head_dim
        shapes = {"q_proj": (h, cfg.heads * hd), "k_proj": (h, cfg.kv_heads * hd),
                  "v_proj": (h, cfg.kv_heads * hd), "o_proj": (cfg.heads * hd, h),
                  "gate_proj": (h, cfg.intermediate), "up_proj": (h, cfg.intermediate),
                  "down_proj": (cfg.intermediate, h)}
        scale = cfg.lora_alpha / cfg.lora_rank
        for i, name in enumerate(self.NAMES):
            K, N = shapes[name]
            self.add_module(name, SoftPalettizedLinear(K, N, rank=cfg.lora_rank, lora_scale=scale,
                                                       seed=seed * 7 + i, device=device,
                                                       lora_b_std=lora_b_std))
        self.input_layernorm = RMSNorm(h, cfg.eps, device)
        self.post_attention_layernorm = RMSNorm(h, cfg.eps, device)
        self.q_norm = RMSNorm(hd, cfg.eps, device)
        self.k_norm = RMSNorm(hd, cfg.eps, device)
        # gate and up as one soft linear over their concatenated rows (SoftLinearGroup): its LoRA
        # weight gradients come from the soft backward's dW tiles, which take ranks up to 32
        self.gate_up = None
        if fuse_gate_up and cfg.intermediate % 256 == 0 and 2 * cfg.lora_rank in (8, 16, 24, 32):
            self.gate_up = SoftLinearGroup([self.gate_proj, self.up_proj])
        self._wgroup = None
        self._wgroup_key = None
        self._pending = None  # weights built by the last optimizer step (commit_next_build)
        # the build also keeps each weight's P (fp16), which the soft backward then reads instead
        # of drawing the noise again, as the reference's backward reads its saved P_aos
        self.save_probs = True
        # the SwiGLU backward in the epilogue of the down projection's grad_x GEMM (SwiGLULink)
        self.swiglu_bwd_in_down = True

    def linears(self):
        return [getattr(self, n) for n in self.NAMES]

    def _units(self):
        """(name, linear or group) in build order: the gate/up group stands for both."""
        out = []
        for n in self.NAMES:
            if self.gate_up is not None and n in ("gate_proj", "up_proj"):
                if n == "gate_proj":
                    out.append(("gate_up", self.gate_up))
                continue
            out.append((n, getattr(self, n)))
        return out

    def _build_group(self):
        """(units, the batched build group of their weights), the group rebuilt when a
        parameter has been replaced rather than written in place (module.to(),
        load_state_dict(assign=True), param.data = ...): its descriptor table holds the
        parameters' device addresses."""
        units = self._units()
        items = []
        for _, u in units:
            if isinstance(u, SoftLinearGroup):
                items.append((u.logits(), ops.PhiloxNoise(u.parts[0].noise_seed, 0), u.palette()))
            else:
                items.append((u.index_logits, ops.PhiloxNoise(u.noise_seed, 0), u.palette))
        key = tuple((t.data_ptr(), t.device) for lg, _, pal in items for t in (lg, pal))
        if self._wgroup is None or self._wgroup_key != key:
            self._wgroup = ops.SoftBuildGroup(items, PLZ_W_HARD_NOISY,
                                              want_probs=self.save_probs)
            self._wgroup_key = key
        return units, self._wgroup

    def _next_offset(self, units, check_tau=True):
        lins = self.linears()
        first = [u.parts[0] if isinstance(u, SoftLinearGroup) else u for _, u in units]
        offset = first[0].noise_counter
        if any(l.noise_counter != offset for l in first) or any(
                l.mode != PLZ_W_HARD_NOISY or (check_tau and l.tau != lins[0].tau) for l in lins):
            raise RuntimeError("batched build: the linears must share noise offset, mode and tau")
        return offset

    def _weight_params(self):
        return [t for l in self.linears() for t in (l.index_logits, l.palette)]

    def build_weights(self):
        """The linears' forward weights in one launch (plz_soft_build_w_batched_philox): each
        linear's (or group's) own Philox key at the shared counter offset of this forward, the
        same tau. Returns {name: (w, group, noise)} for the forward, with "gate_up" for the
        grouped gate and up. When the last optimizer step has already built them
        (plan_next_build / commit_next_build) and no logits, palette or tau has changed since,
        those weights are used as they are."""
        pend, self._pending = self._pending, None
        units, grp = self._build_group()
        tau = self.linears()[0].tau
        if pend is not None:  # the noise counters have advanced already
            self._next_offset(units)
            if (pend["key"] == self._wgroup_key and pend["complete"] and pend["tau"] == tau and
                    all(p._version == v for p, v in pend["versions"])):
                outs = grp.outputs
            else:  # built from values that have changed since: build again, same noise
                outs = grp.run(tau, pend["offset"])
            return {n: (w, grp, sp, pr) for (n, _), (w, _), sp, pr in
                    zip(units, outs, pend["specs"], grp.probs)}
        offset = self._next_offset(units)
        specs = [u.next_noise_spec() for _, u in units]
        outs = grp.run(tau, offset)
        return {n: (w, grp, sp, pr) for (n, _), (w, _), sp, pr in zip(units, outs, specs, grp.probs)}

    def plan_next_build(self, tau):
        """The next forward's weights as an optimizer-step build (optim.NextBuild): every
        linear's logits, palette and output rows of the batched build group, with the noise of
        the next forward (the counters advance now instead of in that forward). Pass it to
        FusedAdamW.step(build=...), then to commit_next_build."""
        units, grp = self._build_group()
        offset = self._next_offset(units, check_tau=False)
        specs = [u.next_noise_spec() for _, u in units]
        items = []
        for (_, u), (w, _), pr in zip(units, grp.outputs, grp.probs):
            if isinstance(u, SoftLinearGroup):
                r0 = 0
                for p, n in zip(u.parts, u.rows):
                    items.append((p.index_logits, p.palette, w[r0:r0 + n], u.parts[0].noise_seed,
                                  r0 * u.K, None if pr is None else pr[r0:r0 + n]))
                    r0 += n
            else:
                items.append((u.index_logits, u.palette, w, u.noise_seed, 0, pr))
        nb = NextBuild(items, offset, tau, PLZ_W_HARD_NOISY)
        nb.specs = specs
        return nb

    def commit_next_build(self, nb):
        """After the optimizer step that ran ``nb``: its weights (complete when every linear's
        logits were updated and built) serve the next forward unless a parameter or tau
        changes first; an incomplete build is redone there with the same noise."""
        self._wgroup.generation += 1  # the weights were rewritten
        self._pending = dict(key=self._wgroup_key, tau=nb.tau, offset=nb.offset, specs=nb.specs,
                             complete=all(id(it[0]) in nb.built for it in nb.items),
                             versions=[(p, p._version) for p in self._weight_params()])

    def forward(self, hs, cos, sin):
        cfg = self.cfg
        B, S, _ = hs.shape
        pw = self.build_weights()
        x = self.input_layernorm(hs)
        q = norm_rope(self.q_norm, self.q_proj(x, pw["q_proj"]).view(B, S, cfg.heads, cfg.head_dim),
                      cos, sin)
        k = norm_rope(self.k_norm, self.k_proj(x, pw["k_proj"]).view(B, S, cfg.kv_heads, cfg.head_dim),
                      cos, sin)
        v = self.v_proj(x, pw["v_proj"]).view(B, S, cfg.kv_heads, cfg.head_dim)
        hs, x = add_rmsnorm(self.post_attention_layernorm, hs,
                            self.o_proj(attention(q, k, v, cfg.heads, cfg.kv_heads), pw["o_proj"]))
        link = None
        if self.gate_up is not None:
            # the SwiGLU backward runs in the down projection's grad_x GEMM epilogue
            link = SwiGLULink() if self.swiglu_bwd_in_down else None
            h = self.gate_up.forward_swiglu(x, pw["gate_up"], link)
        else:
            h = SwiGLUFunction.apply(self.gate_proj(x, pw["gate_proj"]), self.up_proj(x, pw["up_proj"]))
        # the residual add in the down GEMM's epilogue
        return self.down_proj(h, pw["down_proj"], residual=hs, swiglu=link)


class DenseDecoderLayer(nn.Module):
    """bf16 teacher with the same architecture (random init), forward only."""

    def __init__(self, cfg: LayerConfig, seed=1, device=None):
        super().__init__()
        self.cfg = cfg
        g = torch.Generator(device="cpu").manual_seed(seed)
        h, hd = cfg.hidden, cfg.head_dim
        dims = {"q_proj": (cfg.heads * hd, h), "k_proj": (cfg.kv_heads * hd, h),
                "v_proj": (cfg.kv_heads * hd, h), "o_proj": (h, cfg.heads * hd),
                "gate_proj": (cfg.intermediate, h), "up_proj": (cfg.intermediate, h),
                "down_proj": (h, cfg.intermediate)}
        for name, (n, k) in dims.items():
            w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16).to(device)
            self.register_buffer(name, w)
        self.input_layernorm = RMSNorm(h, cfg.eps, device)
        self.post_attention_layernorm = RMSNorm(h, cfg.eps, device)
        self.q_norm = RMSNorm(hd, cfg.eps, device)
        self.k_norm = RMSNorm(hd, cfg.eps, device)

    @staticmethod
    def _linear(x, w):
        """x [..., K] W^T on the MFMA GEMM core (plz_linear_fwd_dense)."""
        return ops.linear_fwd_dense(x.reshape(-1, x.shape[-1]).contiguous(), w).view(
            *x.shape[:-1], w.shape[0])

    @torch.no_grad()
    def forward(self, hs, cos, sin):
        _gpu_bf16(hs, "DenseDecoderLayer input")
        cfg = self.cfg
        B, S, _ = hs.shape
        lin = self._linear
        x = self.input_layernorm(hs)
        q = norm_rope(self.q_norm, lin(x, self.q_proj).view(B, S, cfg.heads, cfg.head_dim), cos, sin)
        k = norm_rope(self.k_norm, lin(x, self.k_proj).view(B, S, cfg.kv_heads, cfg.head_dim),
                      cos, sin)
        v = lin(x, self.v_proj).view(B, S, cfg.kv_heads, cfg.head_dim)
        hs, x = add_rmsnorm(self.post_attention_layernorm, hs,
                            lin(attention(q, k, v, cfg.heads, cfg.kv_heads), self.o_proj))
        if cfg.intermediate % 128 == 0:
            # gate and up in one GEMM with the SwiGLU in its epilogue (never stored)
            if getattr(self, "_gate_up", None) is None:
                self._gate_up = ops.swiglu_weight(self.gate_proj, self.up_proj)
            h = ops.linear_fwd_dense_swiglu(x.reshape(-1, x.shape[-1]), self._gate_up)
            h = h.view(B, S, -1)
        else:
            h = SwiGLUFunction.apply(lin(x, self.gate_proj), lin(x, self.up_proj))
        # the residual add in the down GEMM's epilogue
        return ops.linear_fwd_dense(h.reshape(-1, h.shape[-1]).contiguous(), self.down_proj,
                                    residual=hs.reshape(-1, cfg.hidden)).view(B, S, cfg.hidden)


# ---- loss / schedule / optimizer ----------------------------------------------------------------
def compute_loss(student_out, teacher_out, w_cos=0.5, w_mse=0.5):
    """train_qwen.py:229-249 (loss_type '1-cos+norm_mse', weights normalised) on bf16 GPU
    outputs: plz_distill_loss_fwd / plz_distill_loss_bwd. Returns (loss, l_cos)."""
    _gpu_bf16(student_out, "compute_loss student")
    _gpu_bf16(teacher_out, "compute_loss teacher")
    loss, out = DistillLossFunction.apply(student_out, teacher_out.detach(), w_cos, w_mse)
    return loss, out[1]


def tau_at(step, tau_init=2.0, tau_final=0.5, warmup=500, anneal=6000):
    """train_qwen.py:1176-1192."""
    if step < warmup:
        return tau_init
    if step < warmup + anneal:
        p = (step - warmup) / anneal
        return max(tau_final, tau_init * (1.0 - p) ** 2)
    return tau_final


class LayerTrainer:
    """Owns a student/teacher pair and runs config-5 training steps."""

    def __init__(self, cfg: LayerConfig, device, lrs=None, seed=0, lora_b_std=0.0,
                 fuse_gate_up=True, build_in_update=True, grad_sq_in_backward=True):
        self.cfg = cfg
        self.device = device
        # the optimizer step also builds the next forward's soft weights (plz_adamw_step_build)
        self.build_in_update = build_in_update
        self.student = PalettizedDecoderLayer(cfg, seed=seed, device=device, lora_b_std=lora_b_std,
                                              fuse_gate_up=fuse_gate_up)
        self.teacher = DenseDecoderLayer(cfg, seed=seed + 1, device=device)
        lrs = lrs or {"palettes": 1e-4, "lora": 3e-4, "indices": 1e-2}
        pal, lora, logits = [], [], []
        for lin in self.student.linears():
            pal.append(lin.palette)
            lora += [lin.lora_a, lin.lora_b]
            logits.append(lin.index_logits)
        self.logits = logits
        self.others = pal + lora
        # clip group 0: index logits (max norm 1.0, clamped to +-5 tau); group 1: the rest (0.3).
        # The logits come last: a step that builds the next weights updates them after the
        # palettes those builds read.
        self.opt = FusedAdamW([{"params": pal, "lr": lrs["palettes"], "clip_group": 1},
                               {"params": lora, "lr": lrs["lora"], "clip_group": 1},
                               {"params": logits, "lr": lrs["indices"], "clip_group": 0}])
        self.logits_group = 2
        # the soft backward also writes the logits' squared-gradient sums, which the clip norm
        # of the update reads instead of the gradients: (logits, its GradSq, its rows there)
        self._sq_items = []
        if grad_sq_in_backward:
            K_of = {id(l): l.in_features for l in self.student.linears()}
            for _, u in self.student._units():
                if isinstance(u, SoftLinearGroup):
                    u.grad_sq = GradSq(u.N, u.K, device)
                    r0 = 0
                    for p, n in zip(u.parts, u.rows):
                        self._sq_items.append((p, u.grad_sq, r0, n, u.K))
                        r0 += n
                else:
                    u.grad_sq = GradSq(u.out_features, u.in_features, device)
                    self._sq_items.append((u, u.grad_sq, 0, u.out_features, K_of[id(u)]))
        self._sq_ready = []
        self.step_idx = 0
        self.skipped = 0
        self._rope = {}

    def rope(self, seq):
        if seq not in self._rope:
            self._rope[seq] = rope_tables(seq, self.cfg.head_dim, self.cfg.rope_theta, self.device)
        return self._rope[seq]

    def forward_backward(self, hs):
        """Teacher + student forward, loss, backward; returns (loss, 1 - cos mean)."""
        tau = tau_at(self.step_idx)
        for lin in self.student.linears():
            lin.tau = tau
        cos, sin = self.rope(hs.shape[1])
        t_out = self.teacher(hs, cos, sin)
        s_out = self.student(hs, cos, sin)
        loss, l_cos = compute_loss(s_out, t_out)
        for p in self.logits + self.others:
            p.grad = None
        self._backward(loss)
        return loss.detach(), l_cos.detach()

    def _backward(self, loss):
        """loss.backward(), then note which logits gradients have their squared sums from the
        soft backward (exactly one write since the reset) and the state of those gradients."""
        for _, sq, _, _, _ in self._sq_items:
            sq.writes = 0
        loss.backward()
        self._sq_ready = []
        for lin, sq, r0, n, K in self._sq_items:
            g = lin.index_logits.grad
            if sq.writes == 1 and g is not None:
                self._sq_ready.append((lin.index_logits, sq.rows(r0, n, K), g.data_ptr(),
                                       g._version))

    def _grad_sq(self):
        """{id(logits): sums} for the gradients unchanged since the backward that summed them."""
        out = {}
        for p, sums, ptr, ver in self._sq_ready:
            g = p.grad
            if g is not None and g.data_ptr() == ptr and g._version == ver:
                out[id(p)] = sums
        self._sq_ready = []
        return out

    def update(self):
        """Two-tier clip, AdamW on fp32 masters, logits clamp +-5 tau, advance the step: one
        fused step (plz_adamw_step), which with build_in_update also builds the next forward's
        soft weights from the updated logits (plz_adamw_step_build) at the next step's tau."""
        tau = tau_at(self.step_idx)
        self.opt.set_clamp(self.logits_group, -5.0 * tau, 5.0 * tau)
        nb = self.student.plan_next_build(tau_at(self.step_idx + 1)) if self.build_in_update else None
        self.opt.step(max_norms=(1.0, 0.3), build=nb, grad_sq=self._grad_sq())
        if nb is not None:
            self.student.commit_next_build(nb)
        self.step_idx += 1

    def step(self, hs, skip_nonfinite=False):
        """forward_backward + update. With skip_nonfinite, a non-finite loss skips the
        backward and the update as train_qwen.py:1282-1298 does: gradients are cleared, the
        parameters and optimizer state stay as they are, the step counter still advances and
        `skipped` counts the skip. The check reads the loss on the host (one synchronisation
        between forward and backward), so it is off by default."""
        if not skip_nonfinite:
            loss, l_cos = self.forward_backward(hs)
            self.update()
            return loss, l_cos
        tau = tau_at(self.step_idx)
        for lin in self.student.linears():
            lin.tau = tau
        cos, sin = self.rope(hs.shape[1])
        t_out = self.teacher(hs, cos, sin)
        s_out = self.student(hs, cos, sin)
        loss, l_cos = compute_loss(s_out, t_out)
        for p in self.logits + self.others:
            p.grad = None
        if not bool(torch.isfinite(loss)):
            self.skipped += 1
            self.step_idx += 1
            return loss.detach(), l_cos.detach()
        self._backward(loss)
        self.update()
        return loss.detach(), l_cos.detach()
