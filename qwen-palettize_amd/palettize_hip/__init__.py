"""palettize_hip: MI355X (gfx950) kernels for qwen-palettize's fused 2-bit LUT-linear path.

Host-side mirror of the reference's Python interface over the C ABI of libpalettize_hip.so:
  ops                     one wrapper per C entry point (native layout)
  functional              autograd Functions in the native layout (lut_linear, soft_lut_linear)
  fused_lut_linear_cuda   drop-in for the reference module of the same name
  qwen_model              PalettizedLinear / QwenLoRA with the reference's constructor API
  layer                   one palettized Qwen-4B-shaped decoder layer training step
"""
from . import _lib, ops  # noqa: F401
from ._lib import (PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN, PLZ_W_SOFT,  # noqa: F401
                   PalettizeError, LIB_PATH)
from .functional import lut_linear, soft_lut_linear  # noqa: F401

__all__ = ["ops", "lut_linear", "soft_lut_linear", "PalettizeError", "LIB_PATH",
           "PLZ_W_SOFT", "PLZ_W_HARD_NOISY", "PLZ_W_HARD_PLAIN"]
