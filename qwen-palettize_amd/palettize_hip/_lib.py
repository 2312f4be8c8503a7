"""ctypes binding of libpalettize_hip.so (the C ABI declared in include/palettize_hip.h).

The library is loaded from this package directory only; there is no fallback: every op
raises if the library or a GPU is missing.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpalettize_hip.so")

PLZ_OK, PLZ_EINVAL, PLZ_EHIP, PLZ_EUNSUPPORTED, PLZ_EWORKSPACE = 0, 1, 2, 3, 4
PLZ_DT_BF16, PLZ_DT_FP16, PLZ_DT_FP32 = 0, 1, 2
PLZ_W_SOFT, PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN = 0, 1, 2
PLZ_GEMV_NATIVE, PLZ_GEMV_DECODE, PLZ_GEMV_PLANES = 0, 1, 2

p = C.c_void_p
i32, i64, u32, u64, f32, sz = C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_float, C.c_size_t


class BuildWDesc(C.Structure):
    _fields_ = [("logits", p), ("noise", p), ("palette", p), ("w", p), ("w_soft", p),
                ("N", i64), ("K", i64), ("logits_dtype", i32), ("reserved", i32),
                ("block_begin", i64), ("noise_seed", u64), ("noise_counter", u64),
                ("p_out", p)]


class PwRefDesc(C.Structure):
    _fields_ = [("logits", p), ("palette", p), ("p_aos", p), ("w", p), ("K", i64), ("N", i64),
                ("block_begin", i64), ("seed_offset", u32), ("vec", i32)]


class AdamWDesc(C.Structure):
    _fields_ = [("param", p), ("grad", p), ("master", p), ("exp_avg", p), ("exp_avg_sq", p),
                ("n", i64), ("dtype", i32), ("clip_group", i32), ("lr", f32), ("clamp_lo", f32),
                ("clamp_hi", f32), ("reserved", f32), ("block_begin", i64), ("grad_sq", p)]


class GemvDesc(C.Structure):
    _fields_ = [("x", p), ("packed", p), ("palette", p), ("y", p), ("N", i64), ("K", i64),
                ("block_begin", i64), ("cost_begin", i64), ("palette_items", p),
                ("packed_items", p)]


# name -> (restype, argtypes); kept in the order of include/palettize_hip.h
SIGNATURES: dict[str, tuple] = {
    "plz_last_error": (C.c_char_p, []),
    "plz_abi_version": (i32, []),
    "plz_pack_indices": (i32, [p, p, i64, i64, p]),
    "plz_unpack_indices": (i32, [p, p, i64, i64, p]),
    "plz_dequant": (i32, [p, p, p, i64, i64, p]),
    "plz_attn_fwd": (i32, [p, p, p, p, p, i32, i32, i32, i32, i32, f32, p]),
    "plz_attn_bwd_workspace": (sz, [i32, i32, i32]),
    "plz_attn_bwd": (i32, [p, p, p, p, p, p, p, p, p, p, sz, i32, i32, i32, i32, i32, f32, p]),
    "plz_rope_fwd": (i32, [p, p, p, p, i64, i64, i32, i32, p]),
    "plz_rope_bwd": (i32, [p, p, p, p, i64, i64, i32, i32, p]),
    "plz_head_norm_rope_fwd": (i32, [p, p, p, p, p, p, i64, i64, i32, i32, f32, p]),
    "plz_head_norm_rope_bwd": (i32, [p, p, p, p, p, p, p, i64, i64, i32, i32, p]),
    "plz_distill_loss_workspace": (sz, [i64]),
    "plz_distill_loss_fwd": (i32, [p, p, f32, f32, f32, p, p, sz, i64, i64, p]),
    "plz_distill_loss_bwd": (i32, [p, p, p, p, f32, f32, f32, p, p, sz, i64, i64, p]),
    "plz_lut_linear_fwd": (i32, [p, p, p, p, p, p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_lut_linear_fwd_workspace": (sz, [i64, i64, i64]),
    "plz_lut_linear_bwd_x": (i32, [p, p, p, p, p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_lut_linear_bwd_x_workspace": (sz, [i64, i64, i64]),
    "plz_lut_linear_bwd_palette_workspace": (sz, [i64, i64, i64]),
    "plz_lut_linear_bwd_palette": (i32, [p, p, p, p, p, sz, i64, i64, i64, p]),
    "plz_lut_linear_bwd_palette_noalloc": (i32, [p, p, p, p, i64, i64, i64, p]),
    "plz_lut_linear_bwd_palette_lora_workspace": (sz, [i64, i64, i64, i32]),
    "plz_lut_linear_bwd_palette_lora": (i32, [p, p, p, p, p, i32, f32, p, p, p, i32, p, sz,
                                              i64, i64, i64, p]),
    "plz_bias_grad": (i32, [p, p, i64, i64, p]),
    "plz_linear_fwd_dense": (i32, [p, p, p, p, p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_linear_fwd_dense_residual": (i32, [p, p, p, p, p, i32, p, p, p, sz, i64, i64, i64, p]),
    "plz_linear_bwd_x_dense_swiglu": (i32, [p, p, p, p, i32, p, p, p, sz, i64, i64, i64, p]),
    "plz_linear_fwd_dense_workspace": (sz, [i64, i64, i64]),
    "plz_linear_fwd_dense_swiglu": (i32, [p, p, p, i64, i64, i64, p]),
    "plz_linear_fwd_dense_swiglu_cat": (i32, [p, p, p, p, i32, p, p, i64, i64, i64, p]),
    "plz_linear_bwd_x_dense": (i32, [p, p, p, p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_linear_bwd_x_dense_workspace": (sz, [i64, i64, i64]),
    "plz_gumbel_philox": (i32, [p, i64, u64, u64, p]),
    "plz_gumbel_lcg": (i32, [p, u32, i64, i64, p]),
    "plz_gumbel_lcg_triton": (i32, [p, u32, i64, i64, p]),
    "plz_pw_ref_plan": (i64, [C.POINTER(PwRefDesc), i32, i64]),
    "plz_soft_pw_ref_batched": (i32, [p, i32, i64, i64, f32, u32, p]),
    "plz_soft_build_w": (i32, [p, i32, p, p, f32, i32, p, p, p, i64, i64, p]),
    "plz_soft_build_w_philox": (i32, [p, i32, u64, u64, p, f32, i32, p, p, p, i64, i64, p]),
    "plz_build_w_plan": (i64, [C.POINTER(BuildWDesc), i32]),
    "plz_soft_build_w_batched": (i32, [p, i32, i64, f32, i32, p]),
    "plz_soft_build_w_batched_philox": (i32, [p, i32, i64, u64, f32, i32, p]),
    "plz_soft_bwd_workspace": (sz, [i64, i64, i64]),
    "plz_soft_bwd": (i32, [p, p, p, i32, p, p, f32, i32, p, p, p, sz, i64, i64, i64, p]),
    "plz_soft_bwd_philox": (i32, [p, p, p, i32, u64, u64, p, f32, i32, p, p, p, sz, i64, i64, i64, p]),
    "plz_soft_bwd_probs": (i32, [p, p, p, p, f32, i32, p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_soft_bwd_lora_workspace": (sz, [i64, i64, i64, i32]),
    "plz_soft_bwd_lora": (i32, [p, p, p, i32, p, u64, u64, p, p, f32, i32, p, p, i32, f32, p, p, p,
                                p, i32, p, p, sz, i64, i64, i64, p]),
    "plz_lora_project": (i32, [p, p, f32, p, i64, i64, i32, p]),
    "plz_lora_grad_t": (i32, [p, p, f32, p, i64, i64, i32, p]),
    "plz_lora_weight_grads_workspace": (sz, [i64, i64, i64, i32]),
    "plz_lora_weight_grads": (i32, [p, p, p, p, f32, p, p, i32, p, sz, i64, i64, i64, i32, p]),
    "plz_lut_gemv": (i32, [p, p, p, p, i64, i64, i64, p]),
    "plz_gemv_palette_items_bytes": (sz, [i64, i64]),
    "plz_gemv_pack_palettes": (i32, [p, p, i64, i64, p]),
    "plz_gemv_packed_items_bytes": (sz, [i64, i64]),
    "plz_gemv_pack_indices": (i32, [p, p, i64, i64, p]),
    "plz_lut_gemv_decode": (i32, [p, p, p, p, i64, i64, i64, p]),
    "plz_gemv_plan": (i64, [C.POINTER(GemvDesc), i32, i32, i32]),
    "plz_lut_gemv_grouped": (i32, [p, i32, i64, i32, i32, p]),
    "plz_gemv_pack_planes": (i32, [p, p, i64, i64, p]),
    "plz_gemv_planes_workspace": (sz, [i32, i64, i32]),
    "plz_lut_gemv_planes": (i32, [p, p, p, p, i64, i64, i64, p, sz, p]),
    "plz_lut_gemv_grouped_planes": (i32, [p, i32, i64, i32, i64, p, sz, p]),
    "plz_idx2_to_packed": (i32, [p, p, i64, i64, p]),
    "plz_packed_to_idx2": (i32, [p, p, i64, i64, p]),
    "plz_logits_argmax_idx2": (i32, [p, i32, p, i64, i64, p]),
    "plz_lut_to_palette": (i32, [p, p, i64, i64, i32, p]),
    "plz_adamw_plan": (i64, [C.POINTER(AdamWDesc), i32]),
    "plz_adamw_workspace": (sz, [i64]),
    "plz_adamw_step": (i32, [p, i32, i64, f32, f32, C.c_double, C.c_double, f32, f32, i64, p, p,
                             sz, p]),
    "plz_adamw_plan_build": (i64, [C.POINTER(AdamWDesc), C.POINTER(BuildWDesc), i32,
                                   C.POINTER(C.c_int64)]),
    "plz_adamw_step_build": (i32, [p, p, i32, i64, i64, u64, f32, i32, f32, f32, C.c_double,
                                   C.c_double, f32, f32, i64, p, p, sz, p]),
    "plz_rmsnorm_fwd": (i32, [p, p, p, p, i64, i64, f32, p]),
    "plz_add_rmsnorm_fwd": (i32, [p, p, p, p, p, p, i64, i64, f32, p]),
    "plz_rmsnorm_bwd_add": (i32, [p, p, p, p, p, p, i64, i64, p]),
    "plz_rmsnorm_bwd_workspace": (sz, [i64, i64]),
    "plz_rmsnorm_bwd": (i32, [p, p, p, p, p, p, p, sz, i64, i64, p]),
    "plz_swiglu_fwd": (i32, [p, p, p, i64, p]),
    "plz_swiglu_bwd": (i32, [p, p, p, p, p, i64, p]),
    "plz_swiglu_fwd_rows": (i32, [p, p, i64, p, i64, i64, i64, p]),
    "plz_swiglu_bwd_rows": (i32, [p, p, i64, p, i64, p, p, i64, i64, i64, p]),
}

_lib = None
_lock = threading.Lock()


class PalettizeError(RuntimeError):
    """Raised when a library call returns a non-zero status."""


def lib():
    """Loads and returns the library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise PalettizeError(
                        f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                        "(there is no CPU fallback)")
                handle = C.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def call(name: str, *args) -> int:
    """Calls an int-returning entry point and raises PalettizeError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != PLZ_OK:
        msg = lib().plz_last_error().decode(errors="replace")
        raise PalettizeError(f"{name} failed (status {rc}): {msg}")
    return rc


def query(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))
