"""Autograd Functions of the LUT-linear path in the native layout.

  lut_linear(x, packed, palette, bias, lora_a, lora_b, lora_scale)
      hard path: y = x W^T + bias + s (x A^T) B^T with W = dequant(packed, palette).
      Gradients: x, palette (fp32 [N, K/256, 4]), bias, lora_a [r, K], lora_b [N, r].
      Straight-through in the sense of the reference's hard backward
      (fused_lut_linear_cuda.py:787-818): the indices are frozen, the palette receives the
      class-scattered dW.
  soft_lut_linear(x, palette, logits, noise, tau, ...)
      Gumbel-softmax path with straight-through forward (fused_lut_linear_cuda.py:880-970):
      forward uses W_hard (or W_soft for mode=PLZ_W_SOFT), backward differentiates
      W_soft = sum_c P_c pal_c without the 1/tau factor unless scale_by_inv_tau.

Inputs are 2-D ([M, K]); callers flatten leading dimensions.
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import PLZ_W_HARD_NOISY


def _c(t):
    return None if t is None else t.contiguous()


class LUTLinearFunction(torch.autograd.Function):
    """Where the library dequantises W for the forward GEMM (from 4096 rows, see
    ops.lut_linear_staged) and x needs a gradient, the bf16 W is kept for the backward's
    grad_x instead of being dequantised a second time (N*K*2 bytes held from forward to
    backward); without a gradient for x nothing reads it, and it is dropped after the GEMM."""

    @staticmethod
    def forward(ctx, x, packed, palette, bias, lora_a, lora_b, lora_scale):
        x = x.contiguous()
        lora_a, lora_b = _c(lora_a), _c(lora_b)
        t = ops.lora_project(x, lora_a, lora_scale) if lora_a is not None else None
        w = None
        if ops.lut_linear_staged(x.shape[0], packed.shape[0], x.shape[1]):
            w = ops.dequant(packed, palette)
            y = ops.linear_fwd_dense(x, w, bias, t, lora_b)
            if not ctx.needs_input_grad[0]:
                w = None
        else:
            y = ops.lut_linear_fwd(x, packed, palette, bias, t, lora_b)
        ctx.save_for_backward(x, packed, palette, lora_a, lora_b, t, w)
        ctx.lora_scale = float(lora_scale)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, gy):
        x, packed, palette, lora_a, lora_b, t, w = ctx.saved_tensors
        gy = gy.contiguous()
        need_x, _, need_pal, need_b, need_la, need_lb, _ = ctx.needs_input_grad
        # one stream: grad_palette beside grad_x on a second stream measured slower (both are
        # MFMA-bound GEMMs that fill the GPU; they only contend)
        need_lora = lora_a is not None and (need_la or need_lb)
        # the LoRA weight gradients ride on the grad_palette GEMM (from its dW tiles) when both
        # are wanted and the rank is one the fused epilogue takes
        fused = need_lora and need_pal and lora_a.shape[0] in (8, 16, 24, 32)
        gt = None
        if lora_a is not None and (need_x or (need_lora and not fused)):
            gt = ops.lora_grad_t(gy, lora_b, ctx.lora_scale)
        grad_x = None
        if need_x:
            grad_x = (ops.linear_bwd_x_dense(gy, w, gt, lora_a) if w is not None else
                      ops.lut_linear_bwd_x(gy, packed, palette, gt, lora_a))
        grad_bias = ops.bias_grad(gy).to(ctx.bias_dtype) if (ctx.has_bias and need_b) else None
        grad_pal = grad_a = grad_b = None
        if fused:
            grad_pal, grad_a, grad_b = ops.lut_linear_bwd_palette_lora(
                x, gy, packed, lora_a, lora_b, ctx.lora_scale, out_dtype=lora_a.dtype)
        else:
            grad_pal = ops.lut_linear_bwd_palette(x, gy, packed) if need_pal else None
            if need_lora:
                grad_a, grad_b = ops.lora_weight_grads(x, gy, t, gt, 1.0, out_dtype=lora_a.dtype)
        return grad_x, None, grad_pal, grad_bias, grad_a, grad_b, None


def lut_linear(x, packed, palette, bias=None, lora_a=None, lora_b=None, lora_scale=1.0):
    """Hard palettized linear, native layout. x [..., K] -> y [..., N]."""
    lead = x.shape[:-1]
    y = LUTLinearFunction.apply(x.reshape(-1, x.shape[-1]), packed, palette, bias, lora_a, lora_b,
                                lora_scale)
    return y.reshape(*lead, y.shape[-1])


class SoftLUTLinearFunction(torch.autograd.Function):
    """``prebuilt`` (optional): (w, group) with w the forward weight already built from these
    logits, noise, palette and tau by ``group`` (an ops.SoftBuildGroup run); the backward
    checks that no later run of the group has overwritten it. A third element, an object with
    ``buf`` (fp32 [N * K / 128]) and ``writes``, has the backward's fused soft dW also write the
    squared-gradient sums of the logits there (ops.soft_bwd_lora grad_sq) and count the write
    (None: not), and a fourth, the forward's P (fp16 [N, K, 4], the group's ``probs``), has it
    read P instead of drawing the noise again. Without ``prebuilt`` the forward builds w and P
    itself and keeps P for the backward, as the reference's forward keeps its fp16 P_aos
    (fused_lut_linear_cuda.py:903-905, 919); the noise is not kept. ``residual`` (optional,
    bf16 [M, N]) is added to y in the GEMM's epilogue, as a separate bf16 add after it would
    (its gradient is grad_y). ``swiglu`` (optional, a layer.SwiGLULink whose ``pre`` holds the
    [gate | up] pre-activations of the SwiGLU that produced x) has the backward's grad_x GEMM
    run the SwiGLU backward in its epilogue: it leaves [grad_gate | grad_up] in the link and
    returns a placeholder for grad_x, which only that SwiGLU's backward may receive."""

    @staticmethod
    def forward(ctx, x, palette, logits, noise, tau, bias, lora_a, lora_b, lora_scale, mode,
                scale_by_inv_tau, prebuilt=None, residual=None, swiglu=None):
        x = x.contiguous()
        lora_a, lora_b = _c(lora_a), _c(lora_b)
        ctx.guard = None
        ctx.grad_sq = ctx.probs = None
        if prebuilt is None:
            ctx.probs = torch.empty((*logits.shape[:2], 4), dtype=torch.float16,
                                    device=logits.device)
            w, _ = ops.soft_build_w(logits, noise, palette, tau, mode, probs=ctx.probs)
        else:
            w, group = prebuilt[:2]
            ctx.guard = (group, group.generation)
            ctx.grad_sq = prebuilt[2] if len(prebuilt) > 2 else None
            ctx.probs = prebuilt[3] if len(prebuilt) > 3 else None
        t = ops.lora_project(x, lora_a, lora_scale) if lora_a is not None else None
        y = ops.linear_fwd_dense(x, w, bias, t, lora_b,
                                 residual=None if residual is None else residual.contiguous())
        # a Philox noise descriptor is redrawn in the backward's epilogue, not stored; with the
        # forward's P kept, no noise is needed at all
        ctx.philox = noise if isinstance(noise, ops.PhiloxNoise) else None
        keep_noise = ctx.philox is None and ctx.probs is None
        ctx.save_for_backward(x, palette, logits, noise if keep_noise else None, w, lora_a, lora_b,
                              t)
        ctx.swiglu = swiglu
        ctx.tau = float(tau)
        ctx.lora_scale = float(lora_scale)
        ctx.scale_by_inv_tau = bool(scale_by_inv_tau)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, gy):
        x, palette, logits, noise, w, lora_a, lora_b, t = ctx.saved_tensors
        if ctx.guard is not None and ctx.guard[0].generation != ctx.guard[1]:
            raise RuntimeError("the prebuilt soft weight of this forward was rebuilt by a later "
                               "forward before this backward ran")
        if ctx.philox is not None and ctx.probs is None:
            noise = ctx.philox
        gy = gy.contiguous()
        need = ctx.needs_input_grad
        need_x, need_pal, need_log, need_b, need_la, need_lb = (
            need[0], need[1], need[2], need[5], need[6], need[7])
        # one stream: the soft dW GEMM and the grad_x GEMM are both long MFMA-bound launches,
        # and running them side by side measured no faster in the layer step
        need_lora = lora_a is not None and (need_la or need_lb)
        need_soft = need_pal or need_log
        # the LoRA weight gradients ride on the soft dW GEMM (from its dW tiles) when both are
        # wanted and the rank is one the fused epilogue takes
        fused = need_lora and need_soft and lora_a.shape[0] in (8, 16, 24, 32)
        gt = None
        if lora_a is not None and (need_x or (need_lora and not fused)):
            gt = ops.lora_grad_t(gy, lora_b, ctx.lora_scale)
        link = ctx.swiglu
        if need_x and link is not None and link.pre is not None:
            link.grad = ops.linear_bwd_x_dense_swiglu(gy, w, link.pre, gt, lora_a)
            grad_x = torch.empty(1, dtype=gy.dtype, device=gy.device).expand(x.shape)
            link.marker = grad_x.data_ptr()
        else:
            grad_x = ops.linear_bwd_x_dense(gy, w, gt, lora_a) if need_x else None
        grad_logits = grad_pal = grad_a = grad_b = None
        if fused:
            sq = ctx.grad_sq if need_log else None
            grad_logits, grad_pal, grad_a, grad_b = ops.soft_bwd_lora(
                x, gy, logits, noise, palette, ctx.tau, lora_a, lora_b, ctx.lora_scale,
                ctx.scale_by_inv_tau, out_dtype=lora_a.dtype,
                grad_sq=sq.buf if sq is not None else None, probs=ctx.probs)
            if sq is not None:
                sq.writes += 1
        elif need_soft:
            grad_logits, grad_pal = ops.soft_bwd(x, gy, logits, noise, palette, ctx.tau,
                                                 ctx.scale_by_inv_tau, probs=ctx.probs)
        grad_bias = ops.bias_grad(gy).to(ctx.bias_dtype) if (ctx.has_bias and need_b) else None
        if need_lora and not fused:
            grad_a, grad_b = ops.lora_weight_grads(x, gy, t, gt, 1.0, out_dtype=lora_a.dtype)
        return (grad_x, grad_pal if need_pal else None, grad_logits if need_log else None, None,
                None, grad_bias, grad_a, grad_b, None, None, None, None,
                gy if len(need) > 12 and need[12] else None, None)


def soft_lut_linear(x, palette, logits, noise, tau, bias=None, lora_a=None, lora_b=None,
                    lora_scale=1.0, mode=PLZ_W_HARD_NOISY, scale_by_inv_tau=False):
    """Gumbel-softmax palettized linear, native layout. x [..., K] -> y [..., N]."""
    lead = x.shape[:-1]
    y = SoftLUTLinearFunction.apply(x.reshape(-1, x.shape[-1]), palette, logits, noise, tau, bias,
                                    lora_a, lora_b, lora_scale, mode, scale_by_inv_tau)
    return y.reshape(*lead, y.shape[-1])
