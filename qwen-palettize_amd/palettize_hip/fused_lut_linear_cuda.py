"""Drop-in replacement of the reference's ``fused_lut_linear_cuda`` module.

Same names, arguments, layouts and gradient tuples as the reference
(fused_lut_linear_cuda.py:755-994), backed by the MI355X kernels of libpalettize_hip.so:

  fused_lut_linear(x, palette, indices, bias=None, group_size=256) -> y
  CUDAFusedLUTLinear.apply(x, palette, indices, bias, group_size)
      x (M, K) bf16; palette (G, 4) bf16 with G = N / group_size; indices (K, N) int8;
      y = x @ W + bias with W[k, n] = palette[n // group_size, indices[k, n]].
      backward -> (grad_x, grad_palette (G, 4) in palette's dtype, None, grad_bias, None)
  fused_lut_linear_soft(x, palette, logits, bias=None, group_size=256, tau=1.0) -> y
  CUDAFusedLUTLinearSoft.apply(x, palette, logits, bias, group_size, tau)
      logits (4, K, N) fp16 (SoA planes, as the reference stores them). The Gumbel noise is
      the reference's own LCG hash sampler with the same global step-seed counter
      (fused_lut_linear_cuda.py:837-843, fused_lut_kernel.cu:1245-1256), so a run draws the
      same noise integers as the reference. Forward value W_hard = palette[argmax of the
      noisy P] (straight-through); backward -> (grad_x, grad_palette, grad_logits (4, K, N)
      fp16, grad_bias, None, None) with the reference's formulas (no 1/tau factor).
      fused_lut_linear_soft(..., semantics="triton") follows the reference's Triton path
      instead (int32 sampler, argmax of the plain logits; triton_soft_forward.py:51-181).
  fused_compute_P_W_batched(student, tau, step_seed, group_size=None) -> [(P_aos, W_soft)]
      the batched soft build of every soft PalettizedLinear (fused_lut_linear_cuda.py:1016-1077).

The reference layout (one palette per 256 output channels spanning all of K) is mapped onto
the native one (palette per output row and 256-wide K chunk) by expanding the palette; its
gradient is summed back over the expansion. K is zero-padded to a multiple of 256 when needed
(the padded columns multiply zeros and contribute nothing).
"""
from __future__ import annotations

import weakref
from collections import OrderedDict

import torch
import torch.nn.functional as F
from torch import Tensor

from . import ops
from ._lib import PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN, PLZ_W_SOFT

GROUP_SIZE = 256


def _pad_k(K: int) -> int:
    return (K + 255) // 256 * 256


class _PackCache:
    """Packed indices of frozen index tensors, reused while the source tensor lives unchanged.

    An entry holds a weak reference to the tensor it was made from and that tensor's version
    counter. A lookup hits only when the entry's tensor is the very object passed in (a new
    tensor that the allocator placed at a freed tensor's address never matches: the weak
    reference of the old one is dead) and nothing has written to it since."""

    def __init__(self, size: int = 64):
        self.size = size
        self._d: "OrderedDict[tuple, tuple]" = OrderedDict()

    def get(self, t: Tensor, make):
        key = (t.data_ptr(), tuple(t.shape), tuple(t.stride()), str(t.device))
        e = self._d.get(key)
        if e is not None and e[0]() is t and e[1] == t._version:
            self._d.move_to_end(key)
            return e[2]
        packed = make()
        self._d[key] = (weakref.ref(t), t._version, packed)
        self._d.move_to_end(key)
        while len(self._d) > self.size:
            self._d.popitem(last=False)
        return packed

    def clear(self):
        self._d.clear()


_PACK_CACHE = _PackCache()


def packed_from_reference(indices: Tensor) -> Tensor:
    """(K, N) int8/uint8/int64 indices -> native packed int32 [N, Kp/16] of their transpose,
    K zero-padded to a multiple of 256. Frozen index buffers are packed once (see _PackCache)."""

    def make():
        N, K = indices.shape[1], indices.shape[0]
        Kp = _pad_k(K)
        idx = indices.t().to(torch.uint8)
        if Kp != K:
            idx = F.pad(idx, (0, Kp - K))
        return ops.pack_indices(idx.contiguous())

    return _PACK_CACHE.get(indices, make)


def _groups_used(rows: int, group_size: int) -> int:
    return -(-rows // group_size)


def palette_from_reference(palette: Tensor, N: int, K: int, group_size: int) -> Tensor:
    """(G, 4) reference palette -> native fp32 [N, Kp/256, 4] (exact for bf16/fp16 input).

    Row n takes group n // group_size, as the reference's flat gather does
    (qwen_model.py:97-102: palette.reshape(-1)[(n // GS) * 4 + idx]). G may exceed the
    ceil(N / group_size) groups the rows use; the last group may be partial."""
    G = palette.shape[0]
    need = _groups_used(N, group_size)
    if palette.dim() != 2 or palette.shape[1] != 4:
        raise ValueError("palette must be (G, 4)")
    if G < need:
        raise ValueError(f"G mismatch: {N} rows in groups of {group_size} need {need} palettes, "
                         f"palette has {G}")
    kg = _pad_k(K) // 256
    per_row = palette[:need].float().repeat_interleave(group_size, dim=0)[:N]  # [N, 4]
    return per_row[:, None, :].expand(N, kg, 4).contiguous()


def palette_grad_to_reference(grad: Tensor, group_size: int, n_groups: int | None = None) -> Tensor:
    """native [N, KG, 4] -> reference (G, 4): sum over the rows of a group and over KG; groups
    no row uses (G above ceil(N / group_size)) get zero."""
    N = grad.shape[0]
    need = _groups_used(N, group_size)
    G = need if n_groups is None else int(n_groups)
    per_row = grad.sum(dim=1)  # [N, 4]
    if need * group_size != N:
        per_row = F.pad(per_row, (0, 0, 0, need * group_size - N))
    out = per_row.view(need, group_size, 4).sum(dim=1)
    if G > need:
        out = F.pad(out, (0, 0, 0, G - need))
    return out


def _prep_x(x: Tensor, K: int) -> Tensor:
    x = x.contiguous()
    Kp = _pad_k(K)
    return F.pad(x, (0, Kp - K)) if Kp != K else x


class CUDAFusedLUTLinear(torch.autograd.Function):
    """forward(ctx, x, palette, indices, bias, group_size) -> y
    backward(ctx, grad_y) -> (grad_x, grad_palette, None, grad_bias, None)"""

    @staticmethod
    def forward(ctx, x, palette, indices, bias, group_size):
        if x.dtype != torch.bfloat16:
            raise TypeError("x must be bf16 cuda")
        if palette.dim() != 2 or palette.shape[1] != 4:
            raise ValueError("palette must have 4 entries per group")
        K, N = indices.shape
        if x.shape[-1] != K:
            raise ValueError("indices K mismatch")
        if N % 8:
            raise ValueError(f"N ({N}) must be a multiple of 8")
        packed = packed_from_reference(indices)
        pal = palette_from_reference(palette, N, K, group_size)
        xp = _prep_x(x, K)
        b = None if bias is None else bias.to(torch.bfloat16).contiguous()
        y = ops.lut_linear_fwd(xp, packed, pal, b)
        ctx.save_for_backward(xp, packed, pal)
        ctx.group_size, ctx.K, ctx.n_groups = group_size, K, palette.shape[0]
        ctx.pal_dtype = palette.dtype
        ctx.bias_requires_grad = bias is not None and bias.requires_grad
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, grad_y):
        xp, packed, pal = ctx.saved_tensors
        grad_y = grad_y.contiguous()
        grad_x = grad_pal = grad_bias = None
        if ctx.needs_input_grad[0]:
            grad_x = ops.lut_linear_bwd_x(grad_y, packed, pal)[:, : ctx.K].contiguous()
        if ctx.needs_input_grad[1]:
            g = ops.lut_linear_bwd_palette(xp, grad_y, packed)
            grad_pal = palette_grad_to_reference(g, ctx.group_size, ctx.n_groups).to(ctx.pal_dtype)
        if ctx.bias_requires_grad:
            grad_bias = ops.bias_grad(grad_y).to(ctx.bias_dtype)
        return grad_x, grad_pal, None, grad_bias, None


def fused_lut_linear(x: Tensor, palette: Tensor, indices: Tensor, bias: Tensor | None = None,
                     group_size: int = GROUP_SIZE) -> Tensor:
    """Functional interface -- supports autograd."""
    return CUDAFusedLUTLinear.apply(x, palette, indices, bias, group_size)


class PreTransposedLUTLinear(torch.autograd.Function):
    """The hard forward of PalettizedLinear(pre_transposed=True) (qwen_model.py:183-190): indices
    are (out, in) and y = x @ W^T + bias with W^T[o, i] = palette[i // group_size][indices[o, i]],
    so the palette groups run along the input dimension.

    The kernels take the weight in its native orientation as W'[i, o] = W^T[o, i] (N' = in rows,
    K' = out columns, one palette per row i, K' zero-padded to a multiple of 256): y = x W' is
    the grad_x GEMM of W', grad_x = grad_y W'^T its forward GEMM, and dW' = x^T grad_y its
    grad_palette GEMM with x and grad_y in swapped roles. Any group size works this way.
    backward -> (grad_x, grad_palette (G, 4), None, grad_bias, None)."""

    @staticmethod
    def forward(ctx, x, palette, indices, bias, group_size):
        if x.dtype != torch.bfloat16:
            raise TypeError("x must be bf16 cuda")
        if indices.dim() != 2:
            raise ValueError("indices must be (out, in)")
        out_f, in_f = indices.shape
        if x.shape[-1] != in_f:
            raise ValueError(f"x has {x.shape[-1]} columns, indices (out, in) have in={in_f}")
        if in_f % 8:
            raise ValueError(f"in_features ({in_f}) must be a multiple of 8")
        packed = packed_from_reference(indices)                  # [in, Kp'/16]
        pal = palette_from_reference(palette, in_f, out_f, group_size)  # [in, Kp'/256, 4]
        xc = x.contiguous()
        y = ops.lut_linear_bwd_x(xc, packed, pal)
        if y.shape[1] != out_f:
            y = y[:, :out_f].contiguous()
        if bias is not None:
            y = y + bias.to(y.dtype)
        ctx.save_for_backward(xc, packed, pal)
        ctx.group_size, ctx.out_f, ctx.n_groups = group_size, out_f, palette.shape[0]
        ctx.pal_dtype = palette.dtype
        ctx.bias_requires_grad = bias is not None and bias.requires_grad
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, grad_y):
        xc, packed, pal = ctx.saved_tensors
        gy = grad_y.contiguous()
        Kp = _pad_k(ctx.out_f)
        gyp = F.pad(gy, (0, Kp - ctx.out_f)) if Kp != ctx.out_f else gy
        grad_x = grad_pal = grad_bias = None
        if ctx.needs_input_grad[0]:
            grad_x = ops.lut_linear_fwd(gyp, packed, pal)
        if ctx.needs_input_grad[1]:
            g = ops.lut_linear_bwd_palette(gyp, xc, packed)      # [in, Kp'/256, 4]
            grad_pal = palette_grad_to_reference(g, ctx.group_size, ctx.n_groups).to(ctx.pal_dtype)
        if ctx.bias_requires_grad:
            grad_bias = ops.bias_grad(gy).to(ctx.bias_dtype)
        return grad_x, grad_pal, None, grad_bias, None


def fused_lut_linear_pre_transposed(x: Tensor, palette: Tensor, indices: Tensor,
                                    bias: Tensor | None = None,
                                    group_size: int = GROUP_SIZE) -> Tensor:
    """Hard forward of a pre-transposed PalettizedLinear (indices (out, in), palette groups
    along the input dimension) -- supports autograd."""
    return PreTransposedLUTLinear.apply(x, palette, indices, bias, group_size)


# Global step counters for the Gumbel seed (one increment per soft forward), as in the
# reference: the CUDA-C module's (fused_lut_linear_cuda.py:837-843) and the Triton module's own
# (triton_soft_forward.py:308-314), which advance independently.
_SOFT_STEP_SEED = 0
_TRITON_STEP_SEED = 0

# Soft-path semantics of the reference's two implementations:
#   "cuda"   CUDAFusedLUTLinearSoft: uint32 LCG sampler (fused_lut_kernel.cu:1245-1256),
#            W_hard = palette[argmax of the noisy P] (fused_lut_kernel.cu:1998-2003)
#   "triton" TritonSoftLinear, which PalettizedLinear prefers when triton imports
#            (qwen_model.py:111-121,158-163): int32 LCG sampler (triton_soft_forward.py:51-66),
#            W_hard = palette[argmax of the plain logits] (triton_soft_forward.py:160-176)
SEMANTICS = ("cuda", "triton")


def _next_soft_step_seed() -> int:
    global _SOFT_STEP_SEED
    _SOFT_STEP_SEED = (_SOFT_STEP_SEED + 1) & 0xFFFFFFFF
    return _SOFT_STEP_SEED


def _next_triton_step_seed() -> int:
    global _TRITON_STEP_SEED
    _TRITON_STEP_SEED = (_TRITON_STEP_SEED + 1) & 0xFFFFFFFF
    return _TRITON_STEP_SEED


def logits_from_reference(logits: Tensor, K: int) -> Tensor:
    """(4, K, N) SoA planes -> native [N, Kp, 4] (same dtype)."""
    nk4 = logits.permute(2, 1, 0)
    Kp = _pad_k(K)
    if Kp != K:
        nk4 = F.pad(nk4, (0, 0, 0, Kp - K))
    return nk4.contiguous()


def _noise_to_native(noise: Tensor, K: int, N: int, Kp: int) -> Tensor:
    """Supplied Gumbel noise, fp32, in the logits' reference layout (4, K, N) or native
    [N, K, 4] -> native [N, Kp, 4] (padded columns get zero noise; their x is zero)."""
    if noise.dtype != torch.float32:
        raise TypeError("noise must be fp32")
    if tuple(noise.shape) == (4, K, N):
        noise = noise.permute(2, 1, 0)
    elif tuple(noise.shape) != (N, K, 4):
        raise ValueError(f"noise must be (4, K, N) or [N, K, 4], got {tuple(noise.shape)}")
    if Kp != K:
        noise = F.pad(noise, (0, 0, 0, Kp - K))
    return noise.contiguous()


def _soft_forward(ctx, x, palette, logits, bias, group_size, tau, noise, ste, semantics="cuda"):
    """Forward of fused_lut_linear_soft: W from logits + noise + palette (when ste, W_hard of
    the noisy P for "cuda" semantics or of the plain logits for "triton"; else W_soft), then
    y = x W^T + b. Saves what _soft_backward needs."""
    if semantics not in SEMANTICS:
        raise ValueError(f"semantics must be one of {SEMANTICS}, got {semantics!r}")
    if logits.dim() != 3 or logits.shape[0] != 4:
        raise ValueError("logits first dim must be 4")
    if logits.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("logits must be fp16 or bf16")
    _, K, N = logits.shape
    if x.shape[-1] != K:
        raise ValueError(f"x K={x.shape[-1]} != logits K={K}")
    if N % 8:
        raise ValueError(f"N ({N}) must be a multiple of 8")
    xp = _prep_x(x, K)
    Kp = xp.shape[1]
    lg = logits_from_reference(logits, K)
    if noise is None:  # the reference's LCG draw, one seed per forward
        if semantics == "triton":
            noise = ops.gumbel_lcg(N, Kp, _next_triton_step_seed(), device=x.device,
                                   variant="triton")
        else:
            noise = ops.gumbel_lcg(N, Kp, _next_soft_step_seed(), device=x.device)
    else:
        noise = _noise_to_native(noise, K, N, Kp)
    pal = palette_from_reference(palette, N, K, group_size)
    hard = PLZ_W_HARD_PLAIN if semantics == "triton" else PLZ_W_HARD_NOISY
    w, _ = ops.soft_build_w(lg, noise, pal, float(tau), hard if ste else PLZ_W_SOFT)
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    y = ops.linear_fwd_dense(xp, w, b)
    ctx.save_for_backward(xp, pal, lg, noise, w)
    ctx.group_size, ctx.K, ctx.tau = group_size, K, float(tau)
    ctx.n_groups = palette.shape[0]
    ctx.pal_dtype, ctx.logits_dtype = palette.dtype, logits.dtype
    ctx.has_bias = bias is not None
    ctx.bias_dtype = None if bias is None else bias.dtype
    return y


def _soft_backward(ctx, grad_y):
    """(grad_x, grad_palette, grad_logits, grad_bias) in the reference layouts."""
    xp, pal, lg, noise, w = ctx.saved_tensors
    grad_y = grad_y.contiguous()
    grad_x = grad_pal = grad_logits = grad_bias = None
    if ctx.needs_input_grad[0]:
        grad_x = ops.linear_bwd_x_dense(grad_y, w)[:, : ctx.K].contiguous()
    if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
        gl, gp = ops.soft_bwd(xp, grad_y, lg, noise, pal, ctx.tau)
        if ctx.needs_input_grad[2]:
            grad_logits = gl[:, : ctx.K, :].permute(2, 1, 0).contiguous().to(ctx.logits_dtype)
        if ctx.needs_input_grad[1]:
            grad_pal = palette_grad_to_reference(gp, ctx.group_size, ctx.n_groups).to(ctx.pal_dtype)
    if ctx.has_bias and ctx.needs_input_grad[3]:
        grad_bias = ops.bias_grad(grad_y).to(ctx.bias_dtype)
    return grad_x, grad_pal, grad_logits, grad_bias


class CUDAFusedLUTLinearSoft(torch.autograd.Function):
    """forward(ctx, x, palette, logits, bias, group_size, tau) -> y
    backward(ctx, grad_y) -> (grad_x, grad_palette, grad_logits, grad_bias, None, None)"""

    @staticmethod
    def forward(ctx, x, palette, logits, bias, group_size, tau):
        return _soft_forward(ctx, x, palette, logits, bias, group_size, tau, None, True)

    @staticmethod
    def backward(ctx, grad_y):
        return _soft_backward(ctx, grad_y) + (None, None)


class _SoftLUTLinearExt(torch.autograd.Function):
    """fused_lut_linear_soft with supplied noise, the pure-soft forward (ste=False) and / or
    the Triton path's semantics; the backward is the same STE backward (TritonSoftLinear's
    backward, triton_soft_forward.py:367-411, computes the same quantities)."""

    @staticmethod
    def forward(ctx, x, palette, logits, bias, group_size, tau, noise, ste, semantics):
        return _soft_forward(ctx, x, palette, logits, bias, group_size, tau, noise, ste,
                             semantics)

    @staticmethod
    def backward(ctx, grad_y):
        return _soft_backward(ctx, grad_y) + (None, None, None, None, None)


def fused_lut_linear_soft(x: Tensor, palette: Tensor, logits: Tensor, bias: Tensor | None = None,
                          group_size: int = GROUP_SIZE, tau: float = 1.0, *,
                          noise: Tensor | None = None, ste: bool = True,
                          semantics: str = "cuda") -> Tensor:
    """Soft (Gumbel-Softmax) functional interface -- supports autograd.

    Beyond the reference's signature: ``noise`` (fp32, (4, K, N) like the logits or native
    [N, K, 4]) replaces the internal LCG draw; ``ste=False`` makes the forward use W_soft =
    sum_c P_c pal_c instead of the straight-through W_hard (the backward is unchanged);
    ``semantics="triton"`` follows the reference's Triton path (int32 sampler with its own
    step counter, W_hard from the plain logits) instead of its CUDA-C one."""
    if semantics not in SEMANTICS:
        raise ValueError(f"semantics must be one of {SEMANTICS}, got {semantics!r}")
    if noise is None and ste and semantics == "cuda":
        return CUDAFusedLUTLinearSoft.apply(x, palette, logits, bias, group_size, tau)
    return _SoftLUTLinearExt.apply(x, palette, logits, bias, group_size, tau, noise, ste,
                                   semantics)


class _Extension:
    """The raw functions of the reference's compiled module that callers reach through
    _get_module() for the soft build (fused_lut_linear_cuda.py:388-422, :513-607; used by
    test_batched_compute_pw.py and test_profile_kernels.py), in the reference's layouts."""

    @staticmethod
    def fused_compute_P_W_batched(logits_list, palette_list, group_size, tau, step_seed):
        """-> [P_aos_0, W_0, P_aos_1, W_1, ...]: P_aos (K, N, 4) fp16, W (K, N) bf16 = W_soft;
        layer i draws with seed step_seed ^ (i * 0x9E3779B9) (fused_lut_kernel.cu:2129)."""
        return ops.soft_pw_reference_batched(list(logits_list), list(palette_list),
                                             int(group_size), float(tau), int(step_seed))

    @staticmethod
    def fused_lut_linear_soft_fwd_aos(x, palette, logits, group_size, tau, step_seed):
        """-> [P_aos (K, N, 4) fp16, W (K, N) bf16 = W_soft] of one layer, seed step_seed."""
        if not x.is_cuda or x.dtype != torch.bfloat16:
            raise TypeError("x must be bf16 cuda")
        return ops.soft_pw_reference_batched([logits], [palette], int(group_size), float(tau),
                                             int(step_seed))


def _get_module():
    return _Extension


def fused_compute_P_W_batched(student, tau: float, step_seed: int, group_size: int | None = None):
    """P_aos + W_soft for every PalettizedLinear of ``student`` with index_logits and
    ``_use_cuda`` in one launch (fused_lut_linear_cuda.py:1016-1077): a list of (P_aos (K, N, 4)
    fp16, W (K, N) bf16) in named_modules() order; [] when there is none. All layers must share
    one group_size."""
    from .qwen_model import PalettizedLinear

    layers = [mod for _, mod in student.named_modules()
              if isinstance(mod, PalettizedLinear) and mod.index_logits is not None
              and getattr(mod, "_use_cuda", False)]
    if not layers:
        return []
    if group_size is None:
        group_size = layers[0].group_size
    for i, mod in enumerate(layers):
        if mod.group_size != group_size:
            raise ValueError(f"All PalettizedLinears must share group_size for the batched "
                             f"compute_P_W kernel; layer {i} has group_size={mod.group_size} "
                             f"vs expected {group_size}")
    flat = _get_module().fused_compute_P_W_batched(
        [m.index_logits.detach() for m in layers], [m.palette.detach() for m in layers],
        int(group_size), float(tau), int(step_seed))
    return [(flat[i], flat[i + 1]) for i in range(0, len(flat), 2)]
