"""Tensor-level wrappers of the C ABI (one function per entry point).

PyTorch provides device memory and the current HIP stream; all arithmetic runs in the HIP
kernels of libpalettize_hip.so. Outputs and workspaces are allocated here (the library
never allocates). Inputs must be CUDA (HIP) tensors; nothing falls back to the CPU.

Native layout (the one the kernels use):
  packed  int32 [N, K/16]      2-bit indices, 16 per word along K, LSB first
  palette fp32  [N, K/256, 4]  per output row and per 256 input columns
  logits  bf16/fp16 [N, K, 4], noise fp32 [N, K, 4]
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import call, query

_DT = {torch.bfloat16: _lib.PLZ_DT_BF16, torch.float16: _lib.PLZ_DT_FP16,
       torch.float32: _lib.PLZ_DT_FP32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_gpu(t: torch.Tensor) -> bool:
    return t.is_cuda


def _need(t: torch.Tensor, name: str, dtype=None, ndim=None) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not _on_gpu(t):
        raise RuntimeError(f"{name} must be a GPU tensor (palettize_hip has no CPU path)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _ptr(t):
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def _opt_workspace(nbytes: int, device):
    """An optional workspace: None (NULL) when the query asks for none."""
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device) if nbytes > 0 else None


def _numel(t) -> int:
    return 0 if t is None else t.numel()


def _bias(bias, N: int):
    """bias must be None or bf16 [N]: the C ABI takes no bias length, the epilogue reads N."""
    if bias is None:
        return None
    _need(bias, "bias", torch.bfloat16, 1)
    if bias.numel() != N:
        raise ValueError(f"bias has {bias.numel()} elements, the output has N={N} columns")
    return bias


# ---- formats ------------------------------------------------------------------------
def pack_indices(idx: torch.Tensor) -> torch.Tensor:
    """uint8 [rows, cols] (0..3) -> int32 [rows, cols/16], LSB first."""
    _need(idx, "idx", torch.uint8, 2)
    rows, cols = idx.shape
    out = torch.empty((rows, cols // 16), dtype=torch.int32, device=idx.device)
    call("plz_pack_indices", _ptr(idx), _ptr(out), rows, cols, _stream(idx))
    return out


def unpack_indices(packed: torch.Tensor) -> torch.Tensor:
    _need(packed, "packed", torch.int32, 2)
    rows, words = packed.shape
    out = torch.empty((rows, words * 16), dtype=torch.uint8, device=packed.device)
    call("plz_unpack_indices", _ptr(packed), _ptr(out), rows, words * 16, _stream(packed))
    return out


def _wshape(packed: torch.Tensor, palette: torch.Tensor):
    _need(packed, "packed", torch.int32, 2)
    _need(palette, "palette", torch.float32, 3)
    N, K = packed.shape[0], packed.shape[1] * 16
    if tuple(palette.shape) != (N, K // 256, 4):
        raise ValueError(f"palette shape {tuple(palette.shape)} != {(N, K // 256, 4)}")
    return N, K


def dequant(packed: torch.Tensor, palette: torch.Tensor) -> torch.Tensor:
    N, K = _wshape(packed, palette)
    w = torch.empty((N, K), dtype=torch.bfloat16, device=packed.device)
    call("plz_dequant", _ptr(packed), _ptr(palette), _ptr(w), N, K, _stream(packed))
    return w


# ---- hard linear --------------------------------------------------------------------
def _lora_pair(a, b, first: str, second: str, rows_a: int, rows_b: int):
    if (a is None) != (b is None):
        raise ValueError(f"{first} and {second} must be given together")
    if a is None:
        return 0
    _need(a, first, torch.bfloat16, 2)
    _need(b, second, torch.bfloat16, 2)
    r = a.shape[1]
    if a.shape[0] != rows_a or b.shape[1] != r or b.shape[0] != rows_b:
        raise ValueError(f"{first} {tuple(a.shape)} / {second} {tuple(b.shape)} mismatch")
    return r


def lut_linear_staged(M: int, N: int, K: int) -> bool:
    """True when the library runs the hard forward / grad_x at this size by dequantising W into
    the workspace and running the dense GEMM (its workspace query then asks for the bf16 W)."""
    return (query("plz_lut_linear_fwd_workspace", M, N, K) >
            query("plz_linear_fwd_dense_workspace", M, N, K))


def lut_linear_fwd(x, packed, palette, bias=None, lora_t=None, lora_b=None, staged=True):
    """y = x W^T (+ bias) (+ lora_t lora_b^T).

    staged: give the workspace the query asks for, so that from 4096 rows W is dequantised
    into it and the dense GEMM runs on it; False keeps the one-pass LUT GEMM (workspace for
    its tail partials only)."""
    N, K = _wshape(packed, palette)
    _need(x, "x", torch.bfloat16, 2)
    M = x.shape[0]
    if x.shape[1] != K:
        raise ValueError(f"x has {x.shape[1]} columns, W has K={K}")
    _bias(bias, N)
    rank = _lora_pair(lora_t, lora_b, "lora_t", "lora_b", M, N)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    q = "plz_lut_linear_fwd_workspace" if staged else "plz_linear_fwd_dense_workspace"
    ws = _opt_workspace(query(q, M, N, K), x.device)
    call("plz_lut_linear_fwd", _ptr(x), _ptr(packed), _ptr(palette), _ptr(bias), _ptr(lora_t),
         _ptr(lora_b), rank, _ptr(y), _ptr(ws), _numel(ws), M, N, K, _stream(x))
    return y


def lut_linear_bwd_x(grad_y, packed, palette, lora_gt=None, lora_a=None, staged=True):
    """grad_x = grad_y W (+ lora_gt lora_a).

    staged: give the workspace the query asks for, so that from 4096 rows W is dequantised
    into it and the dense GEMM runs on it; False keeps the one-pass LUT GEMM (workspace for
    its tail partials only)."""
    N, K = _wshape(packed, palette)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    M = grad_y.shape[0]
    if grad_y.shape[1] != N:
        raise ValueError("grad_y columns != N")
    rank = 0
    if lora_gt is not None or lora_a is not None:
        if lora_gt is None or lora_a is None:
            raise ValueError("lora_gt and lora_a must be given together")
        _need(lora_gt, "lora_gt", torch.bfloat16, 2)
        _need(lora_a, "lora_a", torch.bfloat16, 2)
        rank = lora_gt.shape[1]
        if lora_gt.shape[0] != M or tuple(lora_a.shape) != (rank, K):
            raise ValueError("lora_gt / lora_a shape mismatch")
    gx = torch.empty((M, K), dtype=torch.bfloat16, device=grad_y.device)
    q = "plz_lut_linear_bwd_x_workspace" if staged else "plz_linear_bwd_x_dense_workspace"
    ws = _opt_workspace(query(q, M, N, K), grad_y.device)
    call("plz_lut_linear_bwd_x", _ptr(grad_y), _ptr(packed), _ptr(palette), _ptr(lora_gt),
         _ptr(lora_a), rank, _ptr(gx), _ptr(ws), _numel(ws), M, N, K, _stream(grad_y))
    return gx


def lut_linear_bwd_palette(x, grad_y, packed):
    """fp32 [N, K/256, 4]: per-class sums of (grad_y^T x)[n, k] over each 256-k group."""
    _need(packed, "packed", torch.int32, 2)
    _need(x, "x", torch.bfloat16, 2)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    N, K = packed.shape[0], packed.shape[1] * 16
    M = x.shape[0]
    if x.shape[1] != K or tuple(grad_y.shape) != (M, N):
        raise ValueError("x / grad_y shape mismatch")
    out = torch.empty((N, K // 256, 4), dtype=torch.float32, device=x.device)
    nbytes = query("plz_lut_linear_bwd_palette_workspace", M, N, K)
    ws = _workspace(nbytes, x.device)
    call("plz_lut_linear_bwd_palette", _ptr(x), _ptr(grad_y), _ptr(packed), _ptr(out), _ptr(ws),
         ws.numel(), M, N, K, _stream(x))
    return out


def lut_linear_bwd_palette_lora(x, grad_y, packed, lora_a, lora_b, scale: float = 1.0,
                                out_dtype=torch.bfloat16):
    """(grad_palette, grad_a [r, K], grad_b [N, r]) from one dW GEMM: the palette gradient as
    lut_linear_bwd_palette, and the LoRA weight gradients scale * lora_b^T dW and
    scale * dW lora_a^T (dW = grad_y^T x), which lora_weight_grads computes from t and gt."""
    _need(packed, "packed", torch.int32, 2)
    for name, v in (("x", x), ("grad_y", grad_y), ("lora_a", lora_a), ("lora_b", lora_b)):
        _need(v, name, torch.bfloat16, 2)
    N, K = packed.shape[0], packed.shape[1] * 16
    M = x.shape[0]
    r = lora_a.shape[0]
    if x.shape[1] != K or tuple(grad_y.shape) != (M, N):
        raise ValueError("x / grad_y shape mismatch")
    if tuple(lora_a.shape) != (r, K) or tuple(lora_b.shape) != (N, r):
        raise ValueError("lora_a must be [r, K] and lora_b [N, r]")
    out = torch.empty((N, K // 256, 4), dtype=torch.float32, device=x.device)
    ga = torch.empty((r, K), dtype=out_dtype, device=x.device)
    gb = torch.empty((N, r), dtype=out_dtype, device=x.device)
    ws = _workspace(query("plz_lut_linear_bwd_palette_lora_workspace", M, N, K, r), x.device)
    call("plz_lut_linear_bwd_palette_lora", _ptr(x), _ptr(grad_y), _ptr(packed), _ptr(lora_a),
         _ptr(lora_b), r, float(scale), _ptr(out), _ptr(ga), _ptr(gb), _DT[out_dtype], _ptr(ws),
         ws.numel(), M, N, K, _stream(x))
    return out, ga, gb


def lut_linear_bwd_palette_noalloc(x, grad_y, packed, out=None):
    """lut_linear_bwd_palette through the entry point that allocates nothing (its split-M
    partials live in a fixed device array of the library; calls that overlap on one GPU race).
    ``out`` (fp32 [N, K/256, 4]) may be passed in so that the call allocates nothing here
    either."""
    _need(packed, "packed", torch.int32, 2)
    _need(x, "x", torch.bfloat16, 2)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    N, K = packed.shape[0], packed.shape[1] * 16
    M = x.shape[0]
    if x.shape[1] != K or tuple(grad_y.shape) != (M, N):
        raise ValueError("x / grad_y shape mismatch")
    if out is None:
        out = torch.empty((N, K // 256, 4), dtype=torch.float32, device=x.device)
    _need(out, "out", torch.float32, 3)
    if tuple(out.shape) != (N, K // 256, 4):
        raise ValueError(f"out must be [{N}, {K // 256}, 4]")
    call("plz_lut_linear_bwd_palette_noalloc", _ptr(x), _ptr(grad_y), _ptr(packed), _ptr(out),
         M, N, K, _stream(x))
    return out


def bias_grad(grad_y):
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    M, N = grad_y.shape
    out = torch.empty((N,), dtype=torch.float32, device=grad_y.device)
    call("plz_bias_grad", _ptr(grad_y), _ptr(out), M, N, _stream(grad_y))
    return out


# ---- dense linear -----------------------------------------------------------------------
def swiglu_weight(w_gate, w_up):
    """[N, K] gate and up weights -> the [2N, K] interleave of plz_linear_fwd_dense_swiglu
    (128 gate rows, the 128 matching up rows, ...). N must be a multiple of 128."""
    N, K = w_gate.shape
    if w_up.shape != (N, K) or N % 128:
        raise ValueError("gate / up must be the same [N, K] with N a multiple of 128")
    return torch.stack([w_gate.reshape(N // 128, 128, K), w_up.reshape(N // 128, 128, K)],
                       dim=1).reshape(2 * N, K).contiguous()


def linear_fwd_dense_swiglu(x, w_gate_up):
    """h = silu(x Wg^T) * (x Wu^T) in one GEMM (w_gate_up from swiglu_weight)."""
    _need(x, "x", torch.bfloat16, 2)
    _need(w_gate_up, "w_gate_up", torch.bfloat16, 2)
    M, K = x.shape
    N = w_gate_up.shape[0] // 2
    if w_gate_up.shape[1] != K:
        raise ValueError("x / w shape mismatch")
    h = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    call("plz_linear_fwd_dense_swiglu", _ptr(x), _ptr(w_gate_up), _ptr(h), M, N, K, _stream(x))
    return h


def linear_fwd_dense_swiglu_cat(x, w, lora_t=None, lora_b=None, keep_pre=True):
    """(y, h): y = x w^T (+ lora_t lora_b^T) for w = [Wg; Wu] of 2F rows, and h = silu(y[:, :F])
    * y[:, F:] from the same GEMM (plz_linear_fwd_dense_swiglu_cat); y is None unless
    keep_pre. Bit-equal to linear_fwd_dense followed by swiglu_fwd_cat."""
    _need(x, "x", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    M, K = x.shape
    F = w.shape[0] // 2
    if w.shape[1] != K or w.shape[0] != 2 * F:
        raise ValueError("x / w shape mismatch")
    rank = _lora_pair(lora_t, lora_b, "lora_t", "lora_b", M, 2 * F)
    y = torch.empty((M, 2 * F), dtype=torch.bfloat16, device=x.device) if keep_pre else None
    h = torch.empty((M, F), dtype=torch.bfloat16, device=x.device)
    call("plz_linear_fwd_dense_swiglu_cat", _ptr(x), _ptr(w), _ptr(lora_t), _ptr(lora_b), rank,
         _ptr(y), _ptr(h), M, F, K, _stream(x))
    return y, h


def linear_fwd_dense(x, w, bias=None, lora_t=None, lora_b=None, residual=None):
    """y = x w^T (+ bias) (+ lora_t lora_b^T); with residual (bf16 [M, N]) y = residual + that,
    added in the GEMM's epilogue with the rounding of a separate bf16 add
    (plz_linear_fwd_dense_residual)."""
    _need(x, "x", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError("x / w shape mismatch")
    _bias(bias, N)
    rank = _lora_pair(lora_t, lora_b, "lora_t", "lora_b", M, N)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    ws = _opt_workspace(query("plz_linear_fwd_dense_workspace", M, N, K), x.device)
    if residual is not None:
        _need(residual, "residual", torch.bfloat16, 2)
        if tuple(residual.shape) != (M, N):
            raise ValueError(f"residual must be [M, N] = [{M}, {N}]")
        call("plz_linear_fwd_dense_residual", _ptr(x), _ptr(w), _ptr(bias), _ptr(lora_t),
             _ptr(lora_b), rank, _ptr(residual), _ptr(y), _ptr(ws), _numel(ws), M, N, K,
             _stream(x))
        return y
    call("plz_linear_fwd_dense", _ptr(x), _ptr(w), _ptr(bias), _ptr(lora_t), _ptr(lora_b), rank,
         _ptr(y), _ptr(ws), _numel(ws), M, N, K, _stream(x))
    return y


def linear_bwd_x_dense(grad_y, w, lora_gt=None, lora_a=None):
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    M, N = grad_y.shape
    K = w.shape[1]
    if w.shape[0] != N:
        raise ValueError("grad_y / w shape mismatch")
    rank = 0
    if lora_gt is not None or lora_a is not None:
        if lora_gt is None or lora_a is None:
            raise ValueError("lora_gt and lora_a must be given together")
        _need(lora_gt, "lora_gt", torch.bfloat16, 2)
        _need(lora_a, "lora_a", torch.bfloat16, 2)
        rank = lora_gt.shape[1]
        if lora_gt.shape[0] != M or tuple(lora_a.shape) != (rank, K):
            raise ValueError("lora_gt / lora_a shape mismatch")
    gx = torch.empty((M, K), dtype=torch.bfloat16, device=grad_y.device)
    ws = _opt_workspace(query("plz_linear_bwd_x_dense_workspace", M, N, K), grad_y.device)
    call("plz_linear_bwd_x_dense", _ptr(grad_y), _ptr(w), _ptr(lora_gt), _ptr(lora_a), rank,
         _ptr(gx), _ptr(ws), _numel(ws), M, N, K, _stream(grad_y))
    return gx


def linear_bwd_x_dense_swiglu(grad_y, w, gate_up, lora_gt=None, lora_a=None):
    """[grad_gate | grad_up] [M, 2K] of h = silu(gate) * up (gate_up [M, 2K] its pre-activations)
    for grad_h = grad_y w (+ lora_gt lora_a), with the SwiGLU backward in the GEMM's epilogue:
    bit for bit swiglu_bwd_cat(gate_up, linear_bwd_x_dense(...)), grad_h never stored."""
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    _need(w, "w", torch.bfloat16, 2)
    _need(gate_up, "gate_up", torch.bfloat16, 2)
    M, N = grad_y.shape
    K = w.shape[1]
    if w.shape[0] != N or tuple(gate_up.shape) != (M, 2 * K):
        raise ValueError("grad_y [M, N], w [N, K] and gate_up [M, 2K] expected")
    rank = 0
    if lora_gt is not None or lora_a is not None:
        if lora_gt is None or lora_a is None:
            raise ValueError("lora_gt and lora_a must be given together")
        _need(lora_gt, "lora_gt", torch.bfloat16, 2)
        _need(lora_a, "lora_a", torch.bfloat16, 2)
        rank = lora_gt.shape[1]
        if lora_gt.shape[0] != M or tuple(lora_a.shape) != (rank, K):
            raise ValueError("lora_gt / lora_a shape mismatch")
    out = torch.empty((M, 2 * K), dtype=torch.bfloat16, device=grad_y.device)
    ws = _opt_workspace(query("plz_linear_bwd_x_dense_workspace", M, N, K), grad_y.device)
    call("plz_linear_bwd_x_dense_swiglu", _ptr(grad_y), _ptr(w), _ptr(lora_gt), _ptr(lora_a),
         rank, _ptr(gate_up), _ptr(out), _ptr(ws), _numel(ws), M, N, K, _stream(grad_y))
    return out


# ---- soft path ------------------------------------------------------------------------
def gumbel_philox(shape, seed: int, offset: int = 0, device="cuda"):
    n = 1
    for s in shape:
        n *= int(s)
    out = torch.empty(tuple(shape), dtype=torch.float32, device=device)
    call("plz_gumbel_philox", _ptr(out), n, int(seed) & (2**64 - 1), int(offset) & (2**64 - 1),
         _stream(out))
    return out


def gumbel_lcg(N: int, K: int, seed: int, device="cuda", variant: str = "cuda"):
    """The reference's LCG Gumbel noise [N, K, 4], element (n, k, c) drawn at
    idx (k*N + n)*4 + c: the CUDA hash (variant "cuda") or the Triton one ("triton")."""
    if variant not in ("cuda", "triton"):
        raise ValueError(f"unknown LCG variant {variant!r}")
    out = torch.empty((N, K, 4), dtype=torch.float32, device=device)
    call("plz_gumbel_lcg_triton" if variant == "triton" else "plz_gumbel_lcg", _ptr(out),
         int(seed) & 0xFFFFFFFF, N, K, _stream(out))
    return out


def soft_pw_reference_batched(logits_list, palette_list, group_size: int, tau: float,
                              step_seed: int):
    """[P_aos_0, W_0, P_aos_1, W_1, ...] of the reference's fused_compute_P_W_batched
    (fused_lut_linear_cuda.py:513-607) from one launch: logits (4, K, N) fp16 and palettes
    (G, 4) bf16 with G = N / group_size, in and out in the reference's layouts; layer i draws
    its LCG noise with seed step_seed ^ (i * 0x9E3779B9)."""
    n = len(logits_list)
    if n == 0:
        raise ValueError("logits_list must be non-empty")
    if len(palette_list) != n:
        raise ValueError("palette_list size must match logits_list size")
    if n > 64:
        raise ValueError(f"max 64 layers in batched kernel (got {n})")
    group_size = int(group_size)
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    descs = (_lib.PwRefDesc * n)()
    outs, held = [], []  # held: realigned palette copies, alive until the launch is queued
    dev = logits_list[0].device
    for i, (lg, pal) in enumerate(zip(logits_list, palette_list)):
        _need(lg, f"logits[{i}]", torch.float16, 3)
        _need(pal, f"palette[{i}]", torch.bfloat16, 2)
        if lg.shape[0] != 4:
            raise ValueError(f"logits[{i}] must be (4, K, N)")
        if pal.shape[1] != 4:
            raise ValueError(f"palette[{i}] must be (G, 4)")
        if lg.device != dev or pal.device != dev:
            raise ValueError("all tensors must be on one device")
        K, N = lg.shape[1], lg.shape[2]
        if N % group_size:
            raise ValueError(f"layer {i}: N={N} not divisible by group_size={group_size}")
        if N // group_size != pal.shape[0]:
            raise ValueError(f"layer {i}: G mismatch (N/GS={N // group_size} vs "
                             f"palette.size(0)={pal.shape[0]})")
        if pal.data_ptr() % 8:
            pal = pal.clone()
            held.append(pal)
        P = torch.empty((K, N, 4), dtype=torch.float16, device=dev)
        w = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
        outs += [P, w]
        descs[i] = _lib.PwRefDesc(lg.data_ptr(), pal.data_ptr(), P.data_ptr(), w.data_ptr(), K, N,
                                  0, i, 0)
    total = _lib.lib().plz_pw_ref_plan(descs, n, group_size)
    if total < 0:
        raise _lib.PalettizeError("plz_pw_ref_plan failed: " + _lib.lib().plz_last_error().decode())
    raw = bytes(C.string_at(C.addressof(descs), C.sizeof(descs)))
    table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)
    call("plz_soft_pw_ref_batched", table.data_ptr(), n, int(total), group_size, float(tau),
         int(step_seed) & 0xFFFFFFFF, torch.cuda.current_stream(dev).cuda_stream)
    return outs


class PhiloxNoise:
    """Gumbel noise drawn inside the soft kernels instead of a tensor: the values
    gumbel_philox(shape, seed, offset) would hold (Philox counter offset + n*K + k for the 4
    classes of weight (n, k)). Accepted wherever a noise tensor [N, K, 4] is."""

    def __init__(self, seed: int, offset: int):
        self.seed, self.offset = int(seed), int(offset)

    def materialize(self, N: int, K: int, device):
        return gumbel_philox((N, K, 4), seed=self.seed, offset=self.offset, device=device)


def _soft_shapes(logits, noise, palette, probs=None):
    """noise may be None only where the forward's P (probs) replaces it."""
    if logits.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("logits must be bf16 or fp16")
    _need(logits, "logits", None, 3)
    _need(palette, "palette", torch.float32, 3)
    N, K, four = logits.shape
    if noise is None:
        if probs is None:
            raise ValueError("noise is needed unless the forward's P (probs) is given")
    elif not isinstance(noise, PhiloxNoise):
        _need(noise, "noise", torch.float32, 3)
        if tuple(noise.shape) != (N, K, 4):
            raise ValueError("logits [N,K,4], noise [N,K,4], palette [N,K/256,4] expected")
    if four != 4 or tuple(palette.shape) != (N, K // 256, 4):
        raise ValueError("logits [N,K,4], noise [N,K,4], palette [N,K/256,4] expected")
    return N, K


def soft_build_w(logits, noise, palette, tau: float, mode: int = _lib.PLZ_W_HARD_NOISY,
                 want_soft: bool = False, probs=None):
    """(w, w_soft or None). probs (optional fp16 [N, K, 4]) also receives
    P = softmax((logits + noise) / tau), which soft_bwd(probs=...) reads in the backward."""
    N, K = _soft_shapes(logits, noise, palette)
    if probs is not None:
        _need(probs, "probs", torch.float16, 3)
        if tuple(probs.shape) != (N, K, 4):
            raise ValueError(f"probs must be [N, K, 4] = [{N}, {K}, 4]")
    w = torch.empty((N, K), dtype=torch.bfloat16, device=logits.device)
    ws = torch.empty((N, K), dtype=torch.bfloat16, device=logits.device) if want_soft else None
    if isinstance(noise, PhiloxNoise):
        call("plz_soft_build_w_philox", _ptr(logits), _DT[logits.dtype], noise.seed, noise.offset,
             _ptr(palette), float(tau), int(mode), _ptr(w), _ptr(ws), _ptr(probs), N, K,
             _stream(logits))
    else:
        call("plz_soft_build_w", _ptr(logits), _DT[logits.dtype], _ptr(noise), _ptr(palette),
             float(tau), int(mode), _ptr(w), _ptr(ws), _ptr(probs), N, K, _stream(logits))
    return w, ws


class SoftBuildGroup:
    """The forward weights of several soft linears built by one launch
    (plz_soft_build_w_batched_philox). ``items`` is a list of (logits, noise, palette), where
    noise is an fp32 [N, K, 4] tensor or a ``PhiloxNoise`` whose seed is that linear's Philox
    key (its noise is then drawn in the kernel at the counter offset given to ``run``). The
    outputs (w and, with want_soft, w_soft) are allocated once and rewritten by every run;
    ``generation`` counts the runs. With want_probs, every run also writes each linear's
    P = softmax((logits + noise) / tau) as fp16 [N, K, 4] into ``probs[i]``, which
    soft_bwd_lora(probs=...) reads in the backward."""

    def __init__(self, items, mode: int = _lib.PLZ_W_HARD_NOISY, want_soft: bool = False,
                 want_probs: bool = False):
        if not items:
            raise ValueError("empty build group")
        self.mode = int(mode)
        self.device = items[0][0].device
        self.outputs = []
        self.probs = []
        self.generation = 0
        descs = (_lib.BuildWDesc * len(items))()
        for i, (logits, noise, palette) in enumerate(items):
            N, K = _soft_shapes(logits, noise, palette)
            w = torch.empty((N, K), dtype=torch.bfloat16, device=self.device)
            ws = torch.empty((N, K), dtype=torch.bfloat16, device=self.device) if want_soft else None
            pr = (torch.empty((N, K, 4), dtype=torch.float16, device=self.device) if want_probs
                  else None)
            self.outputs.append((w, ws))
            self.probs.append(pr)
            philox = isinstance(noise, PhiloxNoise)
            descs[i] = _lib.BuildWDesc(logits.data_ptr(), None if philox else noise.data_ptr(),
                                       palette.data_ptr(), w.data_ptr(),
                                       ws.data_ptr() if ws is not None else None,
                                       N, K, _DT[logits.dtype], 0, 0,
                                       (noise.seed & (2**64 - 1)) if philox else 0, 0,
                                       pr.data_ptr() if pr is not None else None)
        self._keep = items
        total = _lib.lib().plz_build_w_plan(descs, len(items))
        if total < 0:
            raise _lib.PalettizeError(
                "plz_build_w_plan failed: " + _lib.lib().plz_last_error().decode())
        self.total_blocks = int(total)
        raw = bytes(C.string_at(C.addressof(descs), C.sizeof(descs)))
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        self.n = len(items)

    def run(self, tau: float, noise_offset: int = 0):
        call("plz_soft_build_w_batched_philox", self.table.data_ptr(), self.n, self.total_blocks,
             int(noise_offset) & (2**64 - 1), float(tau), self.mode,
             torch.cuda.current_stream(self.device).cuda_stream)
        self.generation += 1
        return self.outputs


def soft_bwd(x, grad_y, logits, noise, palette, tau: float, scale_by_inv_tau: bool = False,
             probs=None):
    """(grad_logits, grad_palette). probs (optional fp16 [N, K, 4], the forward's P from
    soft_build_w(probs=...)) is read instead of logits and noise (plz_soft_bwd_probs), as the
    reference's backward reads its saved P_aos; logits and noise then give only the shapes and
    the gradient's dtype (noise may then be None)."""
    N, K = _soft_shapes(logits, noise, palette, probs)
    _need(x, "x", torch.bfloat16, 2)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    M = x.shape[0]
    if x.shape[1] != K or tuple(grad_y.shape) != (M, N):
        raise ValueError("x / grad_y shape mismatch")
    gl = torch.empty_like(logits)
    gp = torch.empty((N, K // 256, 4), dtype=torch.float32, device=x.device)
    ws = _workspace(query("plz_soft_bwd_workspace", M, N, K), x.device)
    if probs is not None:
        _need(probs, "probs", torch.float16, 3)
        if tuple(probs.shape) != (N, K, 4):
            raise ValueError(f"probs must be [N, K, 4] = [{N}, {K}, 4]")
        call("plz_soft_bwd_probs", _ptr(x), _ptr(grad_y), _ptr(probs), _ptr(palette), float(tau),
             int(bool(scale_by_inv_tau)), _ptr(gl), _DT[logits.dtype], _ptr(gp), _ptr(ws),
             ws.numel(), M, N, K, _stream(x))
    elif isinstance(noise, PhiloxNoise):
        call("plz_soft_bwd_philox", _ptr(x), _ptr(grad_y), _ptr(logits), _DT[logits.dtype],
             noise.seed, noise.offset, _ptr(palette), float(tau), int(bool(scale_by_inv_tau)),
             _ptr(gl), _ptr(gp), _ptr(ws), ws.numel(), M, N, K, _stream(x))
    else:
        call("plz_soft_bwd", _ptr(x), _ptr(grad_y), _ptr(logits), _DT[logits.dtype], _ptr(noise),
             _ptr(palette), float(tau), int(bool(scale_by_inv_tau)), _ptr(gl), _ptr(gp), _ptr(ws),
             ws.numel(), M, N, K, _stream(x))
    return gl, gp


def soft_bwd_lora(x, grad_y, logits, noise, palette, tau: float, lora_a, lora_b,
                  scale: float = 1.0, scale_by_inv_tau: bool = False, out_dtype=torch.bfloat16,
                  grad_sq=None, probs=None):
    """(grad_logits, grad_palette, grad_a [r, K], grad_b [N, r]) from one dW GEMM: the soft
    backward as soft_bwd (bit for bit), and the LoRA weight gradients scale * lora_b^T dW and
    scale * dW lora_a^T (dW = grad_y^T x), which lora_weight_grads computes from t and gt.
    grad_sq (optional fp32 [N * K / 128]) receives the sum of squares of each 512 consecutive
    grad_logits values, for FusedAdamW.step(grad_sq=...). probs (optional fp16 [N, K, 4]): the
    forward's P (SoftBuildGroup(want_probs=True)), read instead of redrawing the noise (noise
    may then be None)."""
    N, K = _soft_shapes(logits, noise, palette, probs)
    if probs is not None:
        _need(probs, "probs", torch.float16, 3)
        if tuple(probs.shape) != (N, K, 4):
            raise ValueError(f"probs must be [N, K, 4] = [{N}, {K}, 4]")
    if grad_sq is not None:
        _need(grad_sq, "grad_sq", torch.float32, 1)
        if grad_sq.numel() != N * K // 128:
            raise ValueError(f"grad_sq must hold N*K/128 = {N * K // 128} floats")
    for name, v in (("x", x), ("grad_y", grad_y), ("lora_a", lora_a), ("lora_b", lora_b)):
        _need(v, name, torch.bfloat16, 2)
    M = x.shape[0]
    r = lora_a.shape[0]
    if x.shape[1] != K or tuple(grad_y.shape) != (M, N):
        raise ValueError("x / grad_y shape mismatch")
    if tuple(lora_a.shape) != (r, K) or tuple(lora_b.shape) != (N, r):
        raise ValueError("lora_a must be [r, K] and lora_b [N, r]")
    gl = torch.empty_like(logits)
    gp = torch.empty((N, K // 256, 4), dtype=torch.float32, device=x.device)
    ga = torch.empty((r, K), dtype=out_dtype, device=x.device)
    gb = torch.empty((N, r), dtype=out_dtype, device=x.device)
    ws = _workspace(query("plz_soft_bwd_lora_workspace", M, N, K, r), x.device)
    philox = isinstance(noise, PhiloxNoise)
    call("plz_soft_bwd_lora", _ptr(x), _ptr(grad_y), _ptr(logits), _DT[logits.dtype],
         None if philox else _ptr(noise), noise.seed if philox else 0,
         noise.offset if philox else 0, _ptr(probs), _ptr(palette), float(tau),
         int(bool(scale_by_inv_tau)), _ptr(lora_a), _ptr(lora_b), r, float(scale), _ptr(gl),
         _ptr(gp), _ptr(ga), _ptr(gb), _DT[out_dtype], _ptr(grad_sq), _ptr(ws), ws.numel(), M, N,
         K, _stream(x))
    return gl, gp, ga, gb


# ---- LoRA -----------------------------------------------------------------------------
def lora_project(x, lora_a, scale: float):
    """t = scale * x lora_a^T, lora_a [r, K]."""
    _need(x, "x", torch.bfloat16, 2)
    _need(lora_a, "lora_a", torch.bfloat16, 2)
    M, K = x.shape
    r = lora_a.shape[0]
    if lora_a.shape[1] != K:
        raise ValueError("lora_a must be [r, K]")
    t = torch.empty((M, r), dtype=torch.bfloat16, device=x.device)
    call("plz_lora_project", _ptr(x), _ptr(lora_a), float(scale), _ptr(t), M, K, r, _stream(x))
    return t


def lora_grad_t(grad_y, lora_b, scale: float):
    """gt = scale * grad_y lora_b, lora_b [N, r]."""
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    _need(lora_b, "lora_b", torch.bfloat16, 2)
    M, N = grad_y.shape
    r = lora_b.shape[1]
    if lora_b.shape[0] != N:
        raise ValueError("lora_b must be [N, r]")
    gt = torch.empty((M, r), dtype=torch.bfloat16, device=grad_y.device)
    call("plz_lora_grad_t", _ptr(grad_y), _ptr(lora_b), float(scale), _ptr(gt), M, N, r,
         _stream(grad_y))
    return gt


def lora_weight_grads(x, grad_y, t, gt, scale: float = 1.0, out_dtype=torch.float32):
    """grad_a [r, K] = gt^T x ; grad_b [N, r] = scale * grad_y^T t."""
    for name, v in (("x", x), ("grad_y", grad_y), ("t", t), ("gt", gt)):
        _need(v, name, torch.bfloat16, 2)
    M, K = x.shape
    N = grad_y.shape[1]
    r = t.shape[1]
    ga = torch.empty((r, K), dtype=out_dtype, device=x.device)
    gb = torch.empty((N, r), dtype=out_dtype, device=x.device)
    ws = _workspace(query("plz_lora_weight_grads_workspace", M, N, K, r), x.device)
    call("plz_lora_weight_grads", _ptr(x), _ptr(grad_y), _ptr(t), _ptr(gt), float(scale),
         _ptr(ga), _ptr(gb), _DT[out_dtype], _ptr(ws), ws.numel(), M, N, K, r, _stream(x))
    return ga, gb


# ---- decode GEMV ------------------------------------------------------------------------
def lut_gemv(x, packed, palette):
    N, K = _wshape(packed, palette)
    _need(x, "x", torch.bfloat16, 2)
    M = x.shape[0]
    if x.shape[1] != K:
        raise ValueError("x / W shape mismatch")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    call("plz_lut_gemv", _ptr(x), _ptr(packed), _ptr(palette), _ptr(y), M, N, K, _stream(x))
    return y


def gemv_pack_palettes(palette):
    """One-time decode layout of a palette [N, K/256, 4] (plz_gemv_pack_palettes): per 128-row
    item, group and row the two 32-bit lookup words of the bf16-rounded entries (low bytes, then
    high bytes), [ceil(N/128), K/256, 128, 2]. Returned as a flat int32 tensor."""
    _need(palette, "palette", torch.float32, 3)
    N, G = palette.shape[0], palette.shape[1]
    nbytes = query("plz_gemv_palette_items_bytes", N, G * 256)
    out = torch.empty(max(nbytes // 4, 4), dtype=torch.int32, device=palette.device)
    call("plz_gemv_pack_palettes", _ptr(palette), _ptr(out), N, G * 256, _stream(palette))
    return out


def gemv_pack_indices(packed):
    """One-time decode layout of packed indices [N, K/16] (plz_gemv_pack_indices): one
    contiguous 8 KB block per 128-row item and 256-k stage, fields permuted for natural-order
    dequantisation. Returned as a flat int32 tensor."""
    _need(packed, "packed", torch.int32, 2)
    N, K = packed.shape[0], packed.shape[1] * 16
    nbytes = query("plz_gemv_packed_items_bytes", N, K)
    out = torch.empty(max(nbytes // 4, 4), dtype=torch.int32, device=packed.device)
    call("plz_gemv_pack_indices", _ptr(packed), _ptr(out), N, K, _stream(packed))
    return out


def gemv_pack_planes(packed):
    """One-time planes layout of packed indices [N, K/16] (plz_gemv_pack_planes) for the
    bit-plane GEMV: the decode layout's 8 KB blocks per 128-row item and 256-k stage, each
    lane's words those of k = 128h + 32j .. +31 (h = 0, 1), a word's nibble i holding the
    indices of k0 + i and k0 + 8 + i. Returned as a flat int32 tensor."""
    _need(packed, "packed", torch.int32, 2)
    N, K = packed.shape[0], packed.shape[1] * 16
    nbytes = query("plz_gemv_packed_items_bytes", N, K)
    out = torch.empty(max(nbytes // 4, 4), dtype=torch.int32, device=packed.device)
    call("plz_gemv_pack_planes", _ptr(packed), _ptr(out), N, K, _stream(packed))
    return out


def lut_gemv_planes(x, planes_items, palette_items, N):
    """lut_gemv on weights in the planes layout (gemv_pack_planes, gemv_pack_palettes): the
    bit-plane FP8 x FP4 MFMA GEMV, with its x pieces in a workspace allocated here."""
    _need(x, "x", torch.bfloat16, 2)
    M, K = x.shape
    if planes_items.numel() * 4 < query("plz_gemv_packed_items_bytes", N, K) or \
            palette_items.numel() * 4 < query("plz_gemv_palette_items_bytes", N, K):
        raise ValueError("planes-layout weights smaller than N x K needs")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    ws = _opt_workspace(query("plz_gemv_planes_workspace", 1, K, M), x.device)
    call("plz_lut_gemv_planes", _ptr(x), _ptr(planes_items), _ptr(palette_items), _ptr(y), M, N,
         K, _ptr(ws), _numel(ws), _stream(x))
    return y


def lut_gemv_decode(x, packed_items, palette_items, N):
    """lut_gemv on weights in the decode layouts (gemv_pack_indices, gemv_pack_palettes)."""
    _need(x, "x", torch.bfloat16, 2)
    M, K = x.shape
    if packed_items.numel() * 4 < query("plz_gemv_packed_items_bytes", N, K) or \
            palette_items.numel() * 4 < query("plz_gemv_palette_items_bytes", N, K):
        raise ValueError("decode-layout weights smaller than N x K needs")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    call("plz_lut_gemv_decode", _ptr(x), _ptr(packed_items), _ptr(palette_items), _ptr(y), M, N,
         K, _stream(x))
    return y


class GemvGroup:
    """A fixed set of independent GEMVs (same M) run by one grouped launch.

    ``items`` is a list of (x [M,K] bf16, packed, palette); outputs are allocated once and
    reused by every ``run()``. The descriptor table lives in device memory. ``layout``:
    "auto" (default: "planes" up to 8 tokens, where one FP8 operand holds every token's two x
    pieces, "decode" above), "decode" (indices and palettes repacked once into the decode
    layouts, plz_gemv_pack_indices / plz_gemv_pack_palettes, streamed contiguously and
    dequantised to bf16), "planes" (the bit-plane MFMA GEMV on plz_gemv_pack_planes indices, with
    a workspace for the x pieces) or "native" (the packed indices and fp32 palettes as given).
    ``prepack=False`` is "native".
    """

    LAYOUTS = {"native": _lib.PLZ_GEMV_NATIVE, "decode": _lib.PLZ_GEMV_DECODE,
               "planes": _lib.PLZ_GEMV_PLANES}

    def __init__(self, items, prepack=True, layout=None):
        if not items:
            raise ValueError("empty GEMV group")
        self.M = items[0][0].shape[0]
        if layout is None:
            layout = "auto" if prepack else "native"
        if layout == "auto":
            layout = "planes" if self.M <= 8 else "decode"
        if layout not in self.LAYOUTS:
            raise ValueError(f"layout must be one of {sorted(self.LAYOUTS)}")
        prepack = layout != "native"
        self.M = items[0][0].shape[0]
        self.device = items[0][0].device
        self.outputs = []
        self._packed_palettes = []
        self._packed_indices = []
        descs = (_lib.GemvDesc * len(items))()
        for i, (x, packed, palette) in enumerate(items):
            N, K = _wshape(packed, palette)
            _need(x, "x", torch.bfloat16, 2)
            if x.shape != (self.M, K):
                raise ValueError(f"item {i}: x must be [{self.M}, {K}]")
            y = torch.empty((self.M, N), dtype=torch.bfloat16, device=self.device)
            self.outputs.append(y)
            pre = gemv_pack_palettes(palette) if prepack and N > 0 and K > 0 else None
            pack_i = gemv_pack_planes if layout == "planes" else gemv_pack_indices
            pri = pack_i(packed) if prepack and N > 0 and K > 0 else None
            self._packed_palettes.append(pre)
            self._packed_indices.append(pri)
            descs[i] = _lib.GemvDesc(x.data_ptr(), packed.data_ptr(), palette.data_ptr(),
                                     y.data_ptr(), N, K, 0, 0,
                                     pre.data_ptr() if pre is not None else None,
                                     pri.data_ptr() if pri is not None else None)
        self._keep = items
        self.layout = self.LAYOUTS[layout]
        self.max_K = max(int(it[1].shape[1]) * 16 for it in items)
        self.workspace = None
        if layout == "planes":
            self.workspace = _opt_workspace(
                query("plz_gemv_planes_workspace", len(items), self.max_K, self.M), self.device)
        total = _lib.lib().plz_gemv_plan(descs, len(items), self.M, self.layout)
        if total < 0:
            raise _lib.PalettizeError(
                "plz_gemv_plan failed: " + _lib.lib().plz_last_error().decode())
        self.total_blocks = int(total)
        raw = bytes(C.string_at(C.addressof(descs), C.sizeof(descs)))
        host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
        self.table = host.to(self.device)
        self.n = len(items)

    def run(self):
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if self.layout == _lib.PLZ_GEMV_PLANES:
            call("plz_lut_gemv_grouped_planes", self.table.data_ptr(), self.n, self.total_blocks,
                 self.M, self.max_K, _ptr(self.workspace), _numel(self.workspace), stream)
        else:
            call("plz_lut_gemv_grouped", self.table.data_ptr(), self.n, self.total_blocks,
                 self.M, self.layout, stream)
        return self.outputs


# ---- RMSNorm / SwiGLU -----------------------------------------------------------------------
def _norm_weight(weight, cols: int):
    _need(weight, "weight", torch.bfloat16, 1)
    if weight.numel() != cols:
        raise ValueError(f"weight has {weight.numel()} elements, rows have {cols} columns")


def rmsnorm_fwd(x, weight, eps: float):
    _need(x, "x", torch.bfloat16, 2)
    rows, cols = x.shape
    _norm_weight(weight, cols)
    y = torch.empty_like(x)
    rstd = torch.empty((rows,), dtype=torch.float32, device=x.device)
    call("plz_rmsnorm_fwd", _ptr(x), _ptr(weight), _ptr(y), _ptr(rstd), rows, cols, float(eps),
         _stream(x))
    return y, rstd


def add_rmsnorm_fwd(x, residual, weight, eps: float):
    """(sum = x + residual, rmsnorm(sum), rstd) in one pass; bf16 [rows, cols] inputs."""
    _need(x, "x", torch.bfloat16, 2)
    _need(residual, "residual", torch.bfloat16, 2)
    if residual.shape != x.shape:
        raise ValueError("x / residual shape mismatch")
    rows, cols = x.shape
    _norm_weight(weight, cols)
    s, y = torch.empty_like(x), torch.empty_like(x)
    rstd = torch.empty((rows,), dtype=torch.float32, device=x.device)
    call("plz_add_rmsnorm_fwd", _ptr(x), _ptr(residual), _ptr(weight), _ptr(s), _ptr(y),
         _ptr(rstd), rows, cols, float(eps), _stream(x))
    return s, y, rstd


def rmsnorm_bwd_add(x, weight, rstd, grad_y, grad_add):
    """rmsnorm_bwd's grad_x (bf16) + grad_add, without the weight gradient."""
    _need(x, "x", torch.bfloat16, 2)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    _need(grad_add, "grad_add", torch.bfloat16, 2)
    rows, cols = x.shape
    _norm_weight(weight, cols)
    if grad_y.shape != x.shape or grad_add.shape != x.shape or rstd.numel() != rows:
        raise ValueError("grad_y / grad_add / rstd do not match x")
    gx = torch.empty_like(x)
    call("plz_rmsnorm_bwd_add", _ptr(x), _ptr(weight), _ptr(rstd), _ptr(grad_y), _ptr(grad_add),
         _ptr(gx), rows, cols, _stream(x))
    return gx


def rmsnorm_bwd(x, weight, rstd, grad_y):
    _need(x, "x", torch.bfloat16, 2)
    _need(grad_y, "grad_y", torch.bfloat16, 2)
    rows, cols = x.shape
    _norm_weight(weight, cols)
    _need(rstd, "rstd", torch.float32, 1)
    if rstd.numel() != rows or grad_y.shape != x.shape:
        raise ValueError("rstd must be [rows] and grad_y the shape of x")
    gx = torch.empty_like(x)
    gw = torch.empty((cols,), dtype=torch.float32, device=x.device)
    ws = _workspace(query("plz_rmsnorm_bwd_workspace", rows, cols), x.device)
    call("plz_rmsnorm_bwd", _ptr(x), _ptr(weight), _ptr(rstd), _ptr(grad_y), _ptr(gx), _ptr(gw),
         _ptr(ws), ws.numel(), rows, cols, _stream(x))
    return gx, gw


def swiglu_fwd(gate, up):
    _need(gate, "gate", torch.bfloat16)
    _need(up, "up", torch.bfloat16)
    h = torch.empty_like(gate)
    call("plz_swiglu_fwd", _ptr(gate), _ptr(up), _ptr(h), gate.numel(), _stream(gate))
    return h


def swiglu_bwd(gate, up, grad_h):
    _need(gate, "gate", torch.bfloat16)
    _need(up, "up", torch.bfloat16)
    _need(grad_h, "grad_h", torch.bfloat16)
    gg = torch.empty_like(gate)
    gu = torch.empty_like(up)
    call("plz_swiglu_bwd", _ptr(gate), _ptr(up), _ptr(grad_h), _ptr(gg), _ptr(gu), gate.numel(),
         _stream(gate))
    return gg, gu


def swiglu_fwd_cat(gate_up):
    """h [..., F] = silu(gate) * up from a fused projection's output [..., 2F] = [gate | up]."""
    _need(gate_up, "gate_up", torch.bfloat16)
    F2 = gate_up.shape[-1]
    if F2 % 16:
        raise ValueError("gate_up: the last dimension must be 2F with F a multiple of 8")
    F = F2 // 2
    g = gate_up.reshape(-1, F2)
    h = torch.empty(gate_up.shape[:-1] + (F,), dtype=torch.bfloat16, device=gate_up.device)
    call("plz_swiglu_fwd_rows", _ptr(g), _ptr(g) + 2 * F, F2, _ptr(h), F, g.shape[0], F,
         _stream(gate_up))
    return h


def swiglu_bwd_cat(gate_up, grad_h):
    """[grad_gate | grad_up] [..., 2F] of swiglu_fwd_cat for the gradient grad_h [..., F]."""
    _need(gate_up, "gate_up", torch.bfloat16)
    _need(grad_h, "grad_h", torch.bfloat16)
    F2 = gate_up.shape[-1]
    F = F2 // 2
    if F2 % 16 or tuple(grad_h.shape) != tuple(gate_up.shape[:-1]) + (F,):
        raise ValueError("gate_up [..., 2F] and grad_h [..., F] expected, F a multiple of 8")
    g = gate_up.reshape(-1, F2)
    out = torch.empty_like(g)
    call("plz_swiglu_bwd_rows", _ptr(g), _ptr(g) + 2 * F, F2, _ptr(grad_h), F, _ptr(out),
         _ptr(out) + 2 * F, F2, g.shape[0], F, _stream(gate_up))
    return out.reshape(gate_up.shape)


# ---- layer step: RoPE and the distillation loss ----------------------------------------------
def _rope(name, x, cos, sin):
    _need(x, "x", torch.bfloat16)
    if x.dim() < 3 or not x.is_contiguous():
        raise ValueError("x must be contiguous [..., seq, heads, head_dim]")
    seq, heads, hd = x.shape[-3], x.shape[-2], x.shape[-1]
    for t, nm in ((cos, "cos"), (sin, "sin")):
        _need(t, nm, torch.float32, 2)
        if tuple(t.shape) != (seq, hd):
            raise ValueError(f"{nm} must be [seq={seq}, head_dim={hd}]")
    y = torch.empty_like(x)
    rows = x.numel() // (heads * hd)
    call(name, _ptr(x), _ptr(cos), _ptr(sin), _ptr(y), rows, seq, heads, hd, _stream(x))
    return y


def rope_fwd(x, cos, sin):
    """x bf16 [..., seq, heads, head_dim] -> x cos + rotate_half(x) sin (fp32 math, bf16 out)."""
    return _rope("plz_rope_fwd", x, cos, sin)


def rope_bwd(grad_y, cos, sin):
    return _rope("plz_rope_bwd", grad_y, cos, sin)


def _head_rows(x, cos, sin, what):
    _need(x, what, torch.bfloat16)
    if x.dim() < 3 or not x.is_contiguous():
        raise ValueError(f"{what} must be contiguous [..., seq, heads, head_dim]")
    seq, heads, hd = x.shape[-3], x.shape[-2], x.shape[-1]
    for t, nm in ((cos, "cos"), (sin, "sin")):
        _need(t, nm, torch.float32, 2)
        if tuple(t.shape) != (seq, hd):
            raise ValueError(f"{nm} must be [seq={seq}, head_dim={hd}]")
    return x.numel() // (heads * hd), seq, heads, hd


def head_norm_rope_fwd(x, weight, cos, sin, eps: float):
    """rope_fwd(rmsnorm over each head's head_dim values) in one pass, bit-identical to the two:
    x bf16 [..., seq, heads, 128] -> (y like x, rstd fp32 [x.numel() / 128])."""
    rows, seq, heads, hd = _head_rows(x, cos, sin, "x")
    _norm_weight(weight, hd)
    y = torch.empty_like(x)
    rstd = torch.empty((rows * heads,), dtype=torch.float32, device=x.device)
    call("plz_head_norm_rope_fwd", _ptr(x), _ptr(weight), _ptr(cos), _ptr(sin), _ptr(y),
         _ptr(rstd), rows, seq, heads, hd, float(eps), _stream(x))
    return y, rstd


def head_norm_rope_bwd(x, weight, rstd, cos, sin, grad_y):
    """grad_x of head_norm_rope_fwd (rope_bwd then rmsnorm_bwd, bit for bit; no weight gradient)."""
    rows, seq, heads, hd = _head_rows(x, cos, sin, "x")
    _norm_weight(weight, hd)
    _need(rstd, "rstd", torch.float32, 1)
    if grad_y.shape != x.shape or not grad_y.is_contiguous() or rstd.numel() != rows * heads:
        raise ValueError("grad_y / rstd do not match x")
    gx = torch.empty_like(x)
    call("plz_head_norm_rope_bwd", _ptr(x), _ptr(weight), _ptr(rstd), _ptr(cos), _ptr(sin),
         _ptr(grad_y), _ptr(gx), rows, seq, heads, hd, _stream(x))
    return gx


def distill_loss_fwd(student, teacher, w_cos=0.5, w_mse=0.5, eps=1e-4):
    """Returns (out4 fp32 [4] = loss, l_cos, t_var, l_mse; workspace for the backward)."""
    _need(student, "student", torch.bfloat16)
    _need(teacher, "teacher", torch.bfloat16)
    if student.shape != teacher.shape:
        raise ValueError("student / teacher shape mismatch")
    dim = student.shape[-1]
    rows = student.numel() // dim
    out = torch.empty(4, dtype=torch.float32, device=student.device)
    ws = _workspace(query("plz_distill_loss_workspace", rows), student.device)
    call("plz_distill_loss_fwd", _ptr(student), _ptr(teacher), float(w_cos), float(w_mse),
         float(eps), _ptr(out), _ptr(ws), ws.numel(), rows, dim, _stream(student))
    return out, ws


def distill_loss_bwd(student, teacher, out4, ws, grad_loss, w_cos=0.5, w_mse=0.5, eps=1e-4):
    dim = student.shape[-1]
    rows = student.numel() // dim
    gl = grad_loss.reshape(1).to(torch.float32).contiguous()
    gs = torch.empty_like(student)
    call("plz_distill_loss_bwd", _ptr(student), _ptr(teacher), _ptr(out4), _ptr(gl),
         float(w_cos), float(w_mse), float(eps), _ptr(gs), _ptr(ws), ws.numel(), rows, dim,
         _stream(student))
    return gs


# ---- attention ---------------------------------------------------------------------------------
def attn_fwd(q, k, v, scale=None):
    """Causal grouped-query attention. q [B, S, Hq, 128], k/v [B, S, Hkv, 128] bf16 ->
    (o [B, S, Hq, 128] bf16, lse [B, Hq, S] fp32)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, nm, torch.bfloat16, 4)
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    if tuple(k.shape) != (B, S, Hkv, D) or tuple(v.shape) != (B, S, Hkv, D):
        raise ValueError("q / k / v shape mismatch")
    scale = D ** -0.5 if scale is None else float(scale)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    call("plz_attn_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, S, Hq, Hkv, D, scale,
         _stream(q))
    return o, lse


def attn_bwd(q, k, v, o, lse, grad_o, scale=None):
    """Backward of attn_fwd: (grad_q, grad_k, grad_v), bf16 in the shapes of q, k, v."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (o, "o"), (grad_o, "grad_o")):
        _need(t, nm, torch.bfloat16, 4)
    _need(lse, "lse", torch.float32, 3)
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    if (tuple(k.shape) != (B, S, Hkv, D) or tuple(v.shape) != (B, S, Hkv, D)
            or o.shape != q.shape or grad_o.shape != q.shape or tuple(lse.shape) != (B, Hq, S)):
        raise ValueError("attention backward shape mismatch")
    scale = D ** -0.5 if scale is None else float(scale)
    gq, gk, gv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = _opt_workspace(query("plz_attn_bwd_workspace", B, S, Hq), q.device)
    call("plz_attn_bwd", _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(grad_o), _ptr(lse), _ptr(gq),
         _ptr(gk), _ptr(gv), _ptr(ws), _numel(ws), B, S, Hq, Hkv, D, scale, _stream(q))
    return gq, gk, gv
