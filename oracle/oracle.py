"""CPU oracle, numpy part -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker; no product code path calls it. Each function restates the
reference's algorithm (file:line cited) in plain numpy, in the native layout:
  W[n, k] = bf16(palette[n, k // 256, idx[n, k]]), palette fp32 [N, K/256, 4],
  logits / noise [N, K, 4].
The C part (plz_oracle.c, loaded by ``clib()``) restates the bit-level pieces a second time.

Pinning (what fixes each function independently of its own formula) is listed in
tests/test_oracle.py; every function below has at least one such check.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# --------------------------------------------------------------------------------------
# bf16 / fp16 rounding
# --------------------------------------------------------------------------------------


def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN -> quiet NaN."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


# --------------------------------------------------------------------------------------
# index packing (palettize_core.py:31-47, :159-172)
# --------------------------------------------------------------------------------------


def pack_idx2(flat) -> bytes:
    """Reference .idx2 packing: 4 indices per byte, byte = a | b<<2 | c<<4 | d<<6
    (palettize_core.py:31-42), with a zero-padded last byte."""
    flat = np.asarray(flat, dtype=np.uint8).ravel() & 3
    pad = (-flat.size) % 4
    if pad:
        flat = np.concatenate([flat, np.zeros(pad, np.uint8)])
    q = flat.reshape(-1, 4)
    return (q[:, 0] | (q[:, 1] << 2) | (q[:, 2] << 4) | (q[:, 3] << 6)).astype(np.uint8).tobytes()


def unpack_idx2(data: bytes, n: int) -> np.ndarray:
    """palettize_core.py:159-164."""
    arr = np.frombuffer(data, dtype=np.uint8)
    i = np.arange(n)
    return ((arr[i // 4] >> ((i % 4) * 2)) & 3).astype(np.uint8)


def pack_native(idx) -> np.ndarray:
    """uint8 [rows, cols] -> int32 [rows, cols/16]: each row's .idx2 bytes read as
    little-endian int32 words (16 indices per word, LSB first)."""
    idx = np.asarray(idx, dtype=np.uint8)
    rows, cols = idx.shape
    assert cols % 16 == 0
    out = np.empty((rows, cols // 16), dtype=np.int32)
    for r in range(rows):
        out[r] = np.frombuffer(pack_idx2(idx[r]), dtype="<i4")
    return out


def unpack_native(packed) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.int32)
    rows, words = packed.shape
    u = packed.view(np.uint32)[:, :, None]
    shifts = (2 * np.arange(16, dtype=np.uint32))[None, None, :]
    return ((u >> shifts) & 3).astype(np.uint8).reshape(rows, words * 16)


def idx2_to_native(data: bytes, N: int, K: int) -> np.ndarray:
    """.idx2 bytes of the (K, N) index matrix (palettize_core.py:167-172 load_indices) ->
    native packed int32 [N, K/16]."""
    kn = unpack_idx2(data, N * K).reshape(K, N)
    return pack_native(np.ascontiguousarray(kn.T))


def native_to_idx2(packed) -> bytes:
    """Native packed [N, K/16] -> .idx2 bytes of its (K, N) transpose (palettize_core.py:45-47
    pack_indices_transposed_2bit)."""
    return pack_idx2(np.ascontiguousarray(unpack_native(packed).T))


def logits_argmax(logits) -> np.ndarray:
    """(4, K, N) index logits -> (K, N) argmax over the planes, first maximum winning
    (torch.argmax; train_qwen.py:826-829)."""
    return np.argmax(np.asarray(logits, dtype=np.float32), axis=0).astype(np.uint8)


# --------------------------------------------------------------------------------------
# dequantisation (qwen_model.py:97-102, :185-186) and layout maps
# --------------------------------------------------------------------------------------


def dequant_bits(idx, palette) -> np.ndarray:
    """idx uint8 [N, K], palette fp32 [N, K/256, 4] -> bf16 bits [N, K] via the flat gather
    flat_palette[group_id * 4 + idx] with group_id = n * (K/256) + k // 256."""
    idx = np.asarray(idx).astype(np.int64)
    N, K = idx.shape
    G = K // 256
    group_id = np.arange(N)[:, None] * G + (np.arange(K) // 256)[None, :]
    flat = np.asarray(palette, dtype=np.float32).reshape(-1)
    return bf16_bits(flat[group_id * 4 + idx])


def dequant(idx, palette) -> np.ndarray:
    return bf16_to_f32(dequant_bits(idx, palette))


def expand_reference_palette(pal_ref, N: int, K: int, group_size: int = 256) -> np.ndarray:
    """Reference palette (G, 4) over output groups of `group_size` rows spanning all of K
    (qwen_model.py:97-102) -> native [N, K/256, 4]."""
    pal_ref = np.asarray(pal_ref, dtype=np.float32)
    per_row = np.repeat(pal_ref, group_size, axis=0)[:N]
    return np.ascontiguousarray(np.broadcast_to(per_row[:, None, :], (N, K // 256, 4)))


def reference_weight(indices_kn, pal_ref, group_size: int = 256) -> np.ndarray:
    """The reference's own gather, (K, N) layout: W[k, n] = palette[n // GS, idx[k, n]]
    (qwen_model.py:97-102, 185-186), values rounded to bf16 as the bf16 palette is."""
    indices_kn = np.asarray(indices_kn).astype(np.int64)
    K, N = indices_kn.shape
    flat_idx = (np.arange(N) // group_size)[None, :] * 4 + indices_kn
    return bf16_round(np.asarray(pal_ref, np.float32).reshape(-1)[flat_idx])


# --------------------------------------------------------------------------------------
# decode-GEMV index layout (this library's own; the reference has no decode path)
# --------------------------------------------------------------------------------------


def gemv_decode_k(B: int, j: int) -> int:
    """k offset (within a word's 16) stored in field 8B + 2j of a decode-layout word."""
    return (0 if B < 2 else 8) + 2 * j + (B & 1)


def gemv_decode_layout(idx) -> np.ndarray:
    """idx [N, K] (0..3) -> uint32 words [ceil(N/128), K/256, 4 waves, 2 blocks, 64 lanes, 4]:
    lane l = 16q + r of block b of wave w holds the words of item row 32w + 16b + r for
    k = 64q + 16t + (0..15) of the stage (t = word 0..3); field 8B + 2j of a word holds
    k offset gemv_decode_k(B, j). Rows past N are zero."""
    idx = np.asarray(idx, np.uint32)
    N, K = idx.shape
    items = (N + 127) // 128
    full = np.zeros((items * 128, K), np.uint32)
    full[:N] = idx
    v = full.reshape(items, 4, 2, 16, K // 256, 4, 4, 16)  # item, w, b, r, stage, q, t, k16
    out = np.zeros(v.shape[:-1], np.uint32)
    for B in range(4):
        for j in range(4):
            out |= v[..., gemv_decode_k(B, j)] << np.uint32(8 * B + 2 * j)
    return np.ascontiguousarray(out.transpose(0, 4, 1, 2, 5, 3, 6)).reshape(-1)


def gemv_planes_layout(idx) -> np.ndarray:
    """idx [N, K] (0..3) -> uint32 words [ceil(N/128), K/256, 4 waves, 2 blocks, 64 lanes, 4] of
    the bit-plane GEMV: lane l = 16g + r of block b of wave w holds item row 32w + 16b + r in
    four words; nibble i of word j holds the index of stage k = 32g + 8j + i in bits 4i, 4i+1
    and that of k = 128 + 32g + 8j + i in bits 4i+2, 4i+3. Rows past N are zero."""
    idx = np.asarray(idx, np.uint32)
    N, K = idx.shape
    items = (N + 127) // 128
    full = np.zeros((items * 128, K), np.uint32)
    full[:N] = idx
    # item, w, b, r, stage, half (k < 128 or not), g, j, i
    v = full.reshape(items, 4, 2, 16, K // 256, 2, 4, 4, 8)
    out = np.zeros(v.shape[:5] + (4, 4), np.uint32)  # ..., g, j
    for i in range(8):
        out |= (v[..., 0, :, :, i] << np.uint32(4 * i)) | (v[..., 1, :, :, i] << np.uint32(4 * i + 2))
    # item, w, b, r, stage, g, j -> item, stage, w, b, g, r, j
    out = out.transpose(0, 4, 1, 2, 5, 3, 6)
    return np.ascontiguousarray(out).reshape(-1)


def gemv_palette_luts(palette) -> np.ndarray:
    """palette fp32 [N, G, 4] -> uint32 [ceil(N/128), G, 128, 2]: per row and group the bf16
    (RNE) entries' low bytes (entry c in byte c), then their high bytes; rows past N zero."""
    pal = np.asarray(palette, np.float32)
    N, G = pal.shape[:2]
    items = (N + 127) // 128
    bits = np.zeros((items * 128, G, 4), np.uint32)
    bits[:N] = bf16_bits(pal).astype(np.uint32)
    sh = np.arange(4, dtype=np.uint32) * 8
    lo = ((bits & 0xFF) << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    hi = ((bits >> 8) << sh).sum(-1, dtype=np.uint64).astype(np.uint32)
    out = np.stack([lo, hi], -1).reshape(items, 128, G, 2).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(out).reshape(-1)


# --------------------------------------------------------------------------------------
# hard linear: forward / backward (fused_lut_linear_cuda.py:755-818,
# fused_lut_kernel.cu:309-518, 551-720, 902-1123, 1129-1147)
# --------------------------------------------------------------------------------------


def lut_linear_fwd(x, W, bias=None, t=None, lora_b=None) -> np.ndarray:
    """fp64 y = x W^T (+ bias) (+ t lora_b^T)."""
    y = np.asarray(x, np.float64) @ np.asarray(W, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    if t is not None:
        y = y + np.asarray(t, np.float64) @ np.asarray(lora_b, np.float64).T
    return y


def grad_x(gy, W) -> np.ndarray:
    return np.asarray(gy, np.float64) @ np.asarray(W, np.float64)


def grad_palette(x, gy, idx) -> np.ndarray:
    """grad_pal[n, g, c] = sum_{k in group g, idx[n,k] = c} (gy^T x)[n, k]
    (the class scatter of fused_lut_kernel.cu:1100-1120, in the native layout)."""
    dW = np.asarray(gy, np.float64).T @ np.asarray(x, np.float64)  # [N, K]
    idx = np.asarray(idx).astype(np.int64)
    N, K = idx.shape
    G = K // 256
    gid = (np.arange(N)[:, None] * G + (np.arange(K) // 256)[None, :]) * 4 + idx
    out = np.bincount(gid.ravel(), weights=dW.ravel(), minlength=N * G * 4)
    return out.reshape(N, G, 4)


def grad_bias(gy) -> np.ndarray:
    return np.asarray(gy, np.float64).sum(axis=0)


# --------------------------------------------------------------------------------------
# Gumbel noise
# --------------------------------------------------------------------------------------


def lcg_bits(seed: int, idx) -> np.ndarray:
    """Integer part of gumbel_sample (fused_lut_kernel.cu:1245-1253): 24-bit uniforms."""
    x = np.uint32(seed) ^ (np.asarray(idx, np.uint32) * np.uint32(0x9E3779B9))
    x = x ^ (x >> np.uint32(13))
    x = x * np.uint32(1103515245) + np.uint32(12345)
    x = x ^ (x >> np.uint32(17))
    x = x * np.uint32(1103515245) + np.uint32(12345)
    return x & np.uint32(0xFFFFFF)


def lcg_bits_i32(seed: int, idx) -> np.ndarray:
    """Integer part of the Triton sampler _gumbel_sample (triton_soft_forward.py:51-66): the
    same statements in int32, where ``>>`` is an arithmetic shift and 0x9E3779B9 is written
    as -1640531527. Wherever neither shifted intermediate has bit 31 set it equals lcg_bits
    (see lcg_variants_agree); elsewhere the two samplers draw different numbers."""
    s = np.uint32(seed & 0xFFFFFFFF).view(np.int32)
    with np.errstate(over="ignore"):
        x = s ^ (np.asarray(idx, np.uint32).view(np.int32) * np.int32(-1640531527))
        x = x ^ (x >> np.int32(13))
        x = x * np.int32(1103515245) + np.int32(12345)
        x = x ^ (x >> np.int32(17))
        x = x * np.int32(1103515245) + np.int32(12345)
    return (x & np.int32(0xFFFFFF)).astype(np.uint32)


def lcg_variants_agree(seed: int, idx) -> np.ndarray:
    """True where the CUDA (uint32) and Triton (int32) hashes give the same bits: the value
    shifted right by 13 and the value shifted right by 17 both have bit 31 clear, so the
    logical and arithmetic shifts coincide. Both are taken from the uint32 hash; up to the
    first shift the two hashes are identical, and up to the second one wherever the first
    shift agreed."""
    x = np.uint32(seed & 0xFFFFFFFF) ^ (np.asarray(idx, np.uint32) * np.uint32(0x9E3779B9))
    ok = (x >> np.uint32(31)) == 0
    x = x ^ (x >> np.uint32(13))
    x = x * np.uint32(1103515245) + np.uint32(12345)
    return ok & ((x >> np.uint32(31)) == 0)


def lcg_index(N: int, K: int) -> np.ndarray:
    """idx [N, K, 4] of element (n, k, c): (k*N + n)*4 + c in uint32, the flat (K, N) index of
    the reference's (4, K, N) logits times 4 plus the class (fused_lut_kernel.cu:1960-1977,
    triton_soft_forward.py:124-138)."""
    n = np.arange(N, dtype=np.uint32)[:, None, None]
    k = np.arange(K, dtype=np.uint32)[None, :, None]
    c = np.arange(4, dtype=np.uint32)[None, None, :]
    with np.errstate(over="ignore"):
        return (k * np.uint32(N) + n) * np.uint32(4) + c


def gumbel_from_bits24(bits) -> np.ndarray:
    """-log(-log(max(u, 1e-7))), u = bits / 2^24, in fp32 (fused_lut_kernel.cu:1253-1255,
    triton_soft_forward.py:63-66)."""
    u = np.asarray(bits, np.uint32).astype(np.float32) * np.float32(1.0 / 16777216.0)
    u = np.maximum(u, np.float32(1e-7))
    return (-np.log(-np.log(u))).astype(np.float32)


def lcg_gumbel(seed: int, N: int, K: int, variant: str = "cuda") -> np.ndarray:
    """noise[n, k, c] of the reference's LCG sampler, idx = (k*N + n)*4 + c, fp32 arithmetic:
    the CUDA hash (fused_lut_kernel.cu:1245-1256, variant "cuda") or the Triton one
    (triton_soft_forward.py:51-66, variant "triton")."""
    idx = lcg_index(N, K)
    if variant == "cuda":
        return gumbel_from_bits24(lcg_bits(seed, idx))
    if variant == "triton":
        return gumbel_from_bits24(lcg_bits_i32(seed, idx))
    raise ValueError(f"unknown LCG variant {variant!r}")


_PHILOX_M = (np.uint64(0xD2511F53), np.uint64(0xCD9E8D57))
_PHILOX_W = (np.uint32(0x9E3779B9), np.uint32(0xBB67AE85))


def philox4x32_10(ctr, key) -> np.ndarray:
    """Philox4x32-10 (Salmon et al., SC'11). ctr uint32 [n, 4], key uint32 [2]."""
    c = np.asarray(ctr, dtype=np.uint32).reshape(-1, 4).copy()
    k0, k1 = np.uint32(key[0]), np.uint32(key[1])
    mask = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = c[:, 0].astype(np.uint64) * _PHILOX_M[0]
        p1 = c[:, 2].astype(np.uint64) * _PHILOX_M[1]
        hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), (p0 & mask).astype(np.uint32)
        hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), (p1 & mask).astype(np.uint32)
        c = np.stack([hi1 ^ c[:, 1] ^ k0, lo1, hi0 ^ c[:, 3] ^ k1, lo0], axis=1)
        with np.errstate(over="ignore"):
            k0 = np.uint32(k0 + _PHILOX_W[0])
            k1 = np.uint32(k1 + _PHILOX_W[1])
    return c


def gumbel_philox(n: int, seed: int, offset: int = 0) -> np.ndarray:
    """Noise of plz_gumbel_philox: counter = offset + i/4, key = seed, u = (b>>9 + .5)/2^23."""
    t = np.arange(n // 4, dtype=np.uint64) + np.uint64(offset)
    ctr = np.zeros((n // 4, 4), np.uint32)
    ctr[:, 0] = (t & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    ctr[:, 1] = (t >> np.uint64(32)).astype(np.uint32)
    bits = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)).reshape(-1)
    return gumbel_from_bits(bits)


def gumbel_from_bits(bits) -> np.ndarray:
    """u = (bits >> 9 + 0.5) / 2^23 in [2^-24, 1 - 2^-24] (exact in fp32); -log(-log u)."""
    bits = np.asarray(bits, dtype=np.uint32)
    u = ((bits >> np.uint32(9)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
    return (-np.log(-np.log(u))).astype(np.float32)


# --------------------------------------------------------------------------------------
# soft path (fused_lut_kernel.cu:1946-2004 forward, :1877-1924 backward;
# triton_soft_forward.py:83-181; fused_lut_linear_cuda.py:880-970)
# --------------------------------------------------------------------------------------

W_SOFT, W_HARD_NOISY, W_HARD_PLAIN = 0, 1, 2


def soft_probs(logits, noise, tau: float) -> np.ndarray:
    """P = softmax_c((logit + noise) / tau) with max subtraction (fp64)."""
    a = (np.asarray(logits, np.float64) + np.asarray(noise, np.float64)) / tau
    a = a - a.max(axis=-1, keepdims=True)
    e = np.exp(a)
    return e / e.sum(axis=-1, keepdims=True)


def _pal_per_weight(palette, K: int) -> np.ndarray:
    return np.repeat(np.asarray(palette, np.float64), 256, axis=1)[:, :K, :]  # [N, K, 4]


def soft_weights(logits, noise, palette, tau: float, mode: int = W_HARD_NOISY):
    """Returns (P [N,K,4], W_soft [N,K], W_fwd [N,K]) in fp64 (W_fwd before bf16 rounding).
    W_hard uses the first maximum: of P for W_HARD_NOISY (fused_lut_kernel.cu:1998-2003), of
    the plain logits for W_HARD_PLAIN (triton_soft_forward.py:160-176)."""
    logits = np.asarray(logits, np.float64)
    N, K, _ = logits.shape
    P = soft_probs(logits, noise, tau)
    pw = _pal_per_weight(palette, K)
    w_soft = (P * pw).sum(-1)
    if mode == W_SOFT:
        return P, w_soft, w_soft
    src = P if mode == W_HARD_NOISY else logits
    am = np.argmax(src, axis=-1)  # numpy argmax returns the first maximum
    w_hard = np.take_along_axis(pw, am[..., None], axis=-1)[..., 0]
    return P, w_soft, w_hard


def soft_backward(x, gy, logits, noise, palette, tau: float, scale_by_inv_tau: bool = False):
    """grad_logits[n,k,c] = s * dW P_c (pal_c - W_soft); grad_pal[n,g,c] = sum_{k in g} dW P_c
    with dW = gy^T x and s = 1 (reference: soft_bwd_elementwise_aos_kernel,
    fused_lut_kernel.cu:1914-1922) or 1/tau."""
    dW = np.asarray(gy, np.float64).T @ np.asarray(x, np.float64)
    P = soft_probs(logits, noise, tau)
    N, K, _ = P.shape
    pw = _pal_per_weight(palette, K)
    w_soft = (P * pw).sum(-1, keepdims=True)
    s = 1.0 / tau if scale_by_inv_tau else 1.0
    g_logits = s * dW[..., None] * P * (pw - w_soft)
    gp = (dW[..., None] * P).reshape(N, K // 256, 256, 4).sum(axis=2)
    return g_logits, gp


# --------------------------------------------------------------------------------------
# LoRA (qwen_model.py:291-304), RMSNorm / SwiGLU (HF Qwen3, modeling_qwen3.py:50-83)
# --------------------------------------------------------------------------------------


def adamw_step(masters, grads, ms, vs, lrs, clip_groups, max_norms, clamps, step: int,
               betas=(0.9, 0.95), eps: float = 1e-8, weight_decay: float = 0.0):
    """One step of the layer optimizer in fp64, updating the lists in place: per clip group
    G, grads scaled by min(1, max_norm_G / (||grad_G|| + 1e-6)) (torch clip_grad_norm_,
    train_qwen.py:1303-1319); torch.optim.AdamW's update on the fp32 masters
    (train_qwen.py:154-221, 600); clamp to (lo, hi) (train_qwen.py:1343-1348).
    Returns the two groups' unclipped gradient norms."""
    b1, b2 = betas
    sq = [0.0, 0.0]
    for g, G in zip(grads, clip_groups):
        sq[G] += float(np.sum(np.asarray(g, np.float64) ** 2))
    norms = [np.sqrt(x) for x in sq]
    coef = [min(1.0, mx / (nrm + 1e-6)) if mx > 0 else 1.0 for mx, nrm in zip(max_norms, norms)]
    bc1, bc2 = 1.0 - b1 ** step, 1.0 - b2 ** step
    for i in range(len(masters)):
        g = np.asarray(grads[i], np.float64) * coef[clip_groups[i]]
        p = masters[i] * (1.0 - lrs[i] * weight_decay)
        ms[i] = ms[i] + (1.0 - b1) * (g - ms[i])
        vs[i] = b2 * vs[i] + (1.0 - b2) * g * g
        p = p - (lrs[i] / bc1) * ms[i] / (np.sqrt(vs[i]) / np.sqrt(bc2) + eps)
        lo, hi = clamps[i]
        masters[i] = np.clip(p, lo, hi)
    return norms


def lora_forward(x, lora_a, lora_b, scale: float) -> np.ndarray:
    """scale * (x A^T) B^T with A [r, K], B [N, r] (fp64)."""
    return scale * (np.asarray(x, np.float64) @ np.asarray(lora_a, np.float64).T) @ np.asarray(
        lora_b, np.float64).T


def lora_weight_grads(x, gy, lora_a, lora_b, scale: float):
    """Gradients of y = scale (x A^T) B^T (QwenLoRA.forward, qwen_model.py:291-304, in the
    native layout A [r, K], B [N, r]) for the output gradient gy: (grad_A [r, K], grad_B [N, r])
    = (scale (gy B)^T x, scale gy^T (x A^T)) in fp64."""
    x = np.asarray(x, np.float64)
    gy = np.asarray(gy, np.float64)
    a = np.asarray(lora_a, np.float64)
    b = np.asarray(lora_b, np.float64)
    return scale * (gy @ b).T @ x, scale * gy.T @ (x @ a.T)


def rmsnorm_fwd(x, weight, eps: float):
    """y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), statistics in fp32."""
    xf = np.asarray(x, np.float32)
    ms = (xf.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    r = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    h = bf16_round(xf * r)
    return bf16_round(np.asarray(weight, np.float32) * h), r[..., 0]


def rmsnorm_bwd(x, weight, gy, eps: float):
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    gy = np.asarray(gy, np.float64)
    r = 1.0 / np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + eps)
    h = x * r
    g = gy * w
    gx = r * (g - h * (g * h).mean(axis=-1, keepdims=True))
    gw = (gy * bf16_round(h.astype(np.float32))).sum(axis=0)
    return gx, gw


def silu(g):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g))


def swiglu_fwd(gate, up) -> np.ndarray:
    """bf16(bf16(silu(gate)) * up)."""
    return bf16_round(bf16_round(silu(gate).astype(np.float32)) * np.asarray(up, np.float32))


def swiglu_bwd(gate, up, gh):
    g = np.asarray(gate, np.float64)
    u = np.asarray(up, np.float64)
    d = np.asarray(gh, np.float64)
    sg = 1.0 / (1.0 + np.exp(-g))
    return d * u * sg * (1.0 + g * (1.0 - sg)), d * g * sg


# --------------------------------------------------------------------------------------
# C part
# --------------------------------------------------------------------------------------
_clib = None


def clib():
    """ctypes handle of liboracle.so (built by oracle/Makefile)."""
    global _clib
    if _clib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        P = C.c_void_p
        L.orc_f2bf.restype = C.c_uint16
        L.orc_f2bf.argtypes = [C.c_float]
        L.orc_pack.argtypes = [P, P, C.c_int64]
        L.orc_unpack.argtypes = [P, P, C.c_int64]
        L.orc_dequant.argtypes = [P, P, P, C.c_int64, C.c_int64]
        L.orc_lcg_bits.argtypes = [P, C.c_uint32, P, C.c_int64]
        L.orc_lcg_bits_i32.argtypes = [P, C.c_uint32, P, C.c_int64]
        L.orc_gumbel_lcg.argtypes = [P, C.c_uint32, C.c_int64, C.c_int64, C.c_int]
        L.orc_philox.argtypes = [P, P, P]
        L.orc_gumbel_philox.argtypes = [P, C.c_int64, C.c_uint64, C.c_uint64]
        _clib = L
    return _clib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def c_pack(idx) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.uint8)
    out = np.empty((idx.shape[0], idx.shape[1] // 16), np.int32)
    clib().orc_pack(_p(idx), _p(out), out.size)
    return out


def c_unpack(packed) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    out = np.empty((packed.shape[0], packed.shape[1] * 16), np.uint8)
    clib().orc_unpack(_p(packed), _p(out), packed.size)
    return out


def c_dequant_bits(packed, palette) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    palette = np.ascontiguousarray(palette, dtype=np.float32)
    N, K = packed.shape[0], packed.shape[1] * 16
    out = np.empty((N, K), np.uint16)
    clib().orc_dequant(_p(packed), _p(palette), _p(out), N, K)
    return out


def c_lcg_bits(seed: int, idx) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    out = np.empty_like(idx)
    clib().orc_lcg_bits(_p(out), seed & 0xFFFFFFFF, _p(idx), idx.size)
    return out


def c_lcg_bits_i32(seed: int, idx) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    out = np.empty_like(idx)
    clib().orc_lcg_bits_i32(_p(out), seed & 0xFFFFFFFF, _p(idx), idx.size)
    return out


def c_gumbel_lcg(seed: int, N: int, K: int, variant: str = "cuda") -> np.ndarray:
    if variant not in ("cuda", "triton"):
        raise ValueError(f"unknown LCG variant {variant!r}")
    out = np.empty((N, K, 4), np.float32)
    clib().orc_gumbel_lcg(_p(out), seed & 0xFFFFFFFF, N, K, int(variant == "triton"))
    return out


def c_philox(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, np.uint32)
    clib().orc_philox(_p(c), _p(k), _p(out))
    return out


def c_gumbel_philox(n: int, seed: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    clib().orc_gumbel_philox(_p(out), n, seed, offset)
    return out
