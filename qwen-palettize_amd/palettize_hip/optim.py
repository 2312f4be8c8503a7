"""Fused optimizer step (plz_adamw_step): the reference's FP32MasterOptimizer
(train_qwen.py:154-221: bf16 gradients -> fp32 masters -> torch.optim.AdamW -> copy back),
its two-tier gradient clipping (train_qwen.py:1303-1319) and the index-logits clamp
(train_qwen.py:1343-1348), as two streaming passes over all parameters."""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from ._lib import PLZ_DT_BF16, PLZ_DT_FP32, call, query


class FusedAdamW:
    """AdamW(betas, eps, weight_decay) on fp32 masters for parameter groups.

    ``groups``: list of dicts with ``params``, ``lr``, ``clip_group`` (0 or 1: which of the two
    gradient-norm groups of ``step(max_norms=...)`` the group belongs to) and optional
    ``clamp`` = (lo, hi) applied to the updated values (changeable per step through
    ``set_clamp``). bf16 parameters get an fp32 master; fp32 parameters are their own master."""

    def __init__(self, groups, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0):
        self.betas, self.eps, self.weight_decay = betas, float(eps), float(weight_decay)
        self.groups = []
        self.entries = []  # (param, master or None, exp_avg, exp_avg_sq, group index)
        for gi, g in enumerate(groups):
            self.groups.append(dict(lr=float(g["lr"]), clip_group=int(g.get("clip_group", 0)),
                                    clamp=tuple(g.get("clamp") or (-math.inf, math.inf))))
            for p in g["params"]:
                if p.dtype not in (torch.bfloat16, torch.float32):
                    raise TypeError("FusedAdamW: parameters must be bf16 or fp32")
                master = p.detach().float().clone() if p.dtype == torch.bfloat16 else None
                self.entries.append((p, master, torch.zeros(p.shape, dtype=torch.float32,
                                                            device=p.device),
                                     torch.zeros(p.shape, dtype=torch.float32, device=p.device),
                                     gi))
        self.device = self.entries[0][0].device if self.entries else None
        self.step_count = 0
        self.last_norms = torch.zeros(2, dtype=torch.float32, device=self.device)
        self._ws = None

    def set_clamp(self, group_index: int, lo: float, hi: float):
        self.groups[group_index]["clamp"] = (float(lo), float(hi))

    def set_lr(self, group_index: int, lr: float):
        self.groups[group_index]["lr"] = float(lr)

    @torch.no_grad()
    def clamp_(self, group_index: int, lo: float, hi: float):
        """Clamp a group's parameters and masters now (outside a step)."""
        for p, master, _, _, gi in self.entries:
            if gi == group_index:
                if master is not None:
                    master.clamp_(lo, hi)
                    p.copy_(master)
                else:
                    p.clamp_(lo, hi)

    def step(self, max_norms=(0.0, 0.0)):
        """One step over every parameter with a gradient; max_norms[G] <= 0 disables clipping of
        group G. Returns the two groups' unclipped gradient norms (device tensor)."""
        live = [e for e in self.entries if e[0].grad is not None]
        if not live:
            return self.last_norms
        self.step_count += 1
        descs = (_lib.AdamWDesc * len(live))()
        for i, (p, master, m, v, gi) in enumerate(live):
            g = self.groups[gi]
            grad = p.grad
            if grad.dtype != p.dtype or not grad.is_contiguous():
                grad = grad.to(p.dtype).contiguous()
                p.grad = grad
            descs[i] = _lib.AdamWDesc(p.data_ptr(), grad.data_ptr(),
                                      master.data_ptr() if master is not None else None,
                                      m.data_ptr(), v.data_ptr(), p.numel(),
                                      PLZ_DT_BF16 if p.dtype == torch.bfloat16 else PLZ_DT_FP32,
                                      g["clip_group"], g["lr"], g["clamp"][0], g["clamp"][1],
                                      0.0, 0)
        total = _lib.lib().plz_adamw_plan(descs, len(live))
        if total < 0:
            raise _lib.PalettizeError("plz_adamw_plan failed: " +
                                      _lib.lib().plz_last_error().decode())
        raw = bytes(C.string_at(C.addressof(descs), C.sizeof(descs)))
        table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).pin_memory().to(
            self.device, non_blocking=True)
        need = query("plz_adamw_workspace", int(total))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        call("plz_adamw_step", table.data_ptr(), len(live), int(total), float(max_norms[0]),
             float(max_norms[1]), float(self.betas[0]), float(self.betas[1]), self.eps,
             self.weight_decay, self.step_count, self.last_norms.data_ptr(), self._ws.data_ptr(),
             self._ws.numel(), torch.cuda.current_stream(self.device).cuda_stream)
        self._table = table  # keep alive until the launch has consumed it
        return self.last_norms
