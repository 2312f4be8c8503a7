"""Fused optimizer step (plz_adamw_step): the reference's FP32MasterOptimizer
(train_qwen.py:154-221: bf16 gradients -> fp32 masters -> torch.optim.AdamW -> copy back),
its two-tier gradient clipping (train_qwen.py:1303-1319) and the index-logits clamp
(train_qwen.py:1343-1348), as two streaming passes over all parameters."""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from ._lib import PLZ_DT_BF16, PLZ_DT_FP32, PLZ_W_HARD_NOISY, call, query


class NextBuild:
    """Soft weights for the optimizer step to build from the logits it updates
    (plz_adamw_step_build): ``items`` lists (logits parameter, palette, w, noise_seed,
    noise_counter[, probs]) -- w [N, K] bf16 receives the weight plz_soft_build_w_batched_philox
    would build from the updated logits, drawing weight (n, k) at Philox counter offset +
    noise_counter + n*K + k under key noise_seed, and probs (fp16 [N, K, 4], optional) its P --
    and ``offset``, ``tau``, ``mode`` are the launch's. After the step, ``built`` holds the ids
    of the logits whose weight was built (a parameter without a gradient is not updated, so not
    built either)."""

    def __init__(self, items, offset: int, tau: float, mode: int = PLZ_W_HARD_NOISY):
        self.items = list(items)
        self.offset, self.tau, self.mode = int(offset), float(tau), int(mode)
        self.built = set()


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

    def step(self, max_norms=(0.0, 0.0), build: NextBuild | None = None, grad_sq=None):
        """One step over every parameter with a gradient; max_norms[G] <= 0 disables clipping of
        group G. With ``build``, the same pass also writes the soft weights it lists from the
        updated logits (plz_adamw_step_build); those parameters are updated after all others
        (the palettes the builds read among them). ``grad_sq`` (optional): {id(param): fp32
        tensor} with the sum of squares of every 512 consecutive elements of that parameter's
        current gradient (ops.soft_bwd_lora's grad_sq), which the clip norm then reads in place
        of the gradient. Returns the two groups' unclipped gradient norms (device tensor)."""
        grad_sq = grad_sq or {}
        live = [e for e in self.entries if e[0].grad is not None]
        if not live:
            return self.last_norms
        bmap = {}
        if build is not None:
            bmap = {id(it[0]): it for it in build.items}
            live = ([e for e in live if id(e[0]) not in bmap] +
                    [e for e in live if id(e[0]) in bmap])
        self.step_count += 1
        descs = (_lib.AdamWDesc * len(live))()
        for i, (p, master, m, v, gi) in enumerate(live):
            g = self.groups[gi]
            grad = p.grad
            if grad.dtype != p.dtype or not grad.is_contiguous():
                grad = grad.to(p.dtype).contiguous()
                p.grad = grad
            sq = grad_sq.get(id(p))
            if sq is not None and (sq.dtype != torch.float32 or not sq.is_contiguous() or
                                   sq.numel() * 512 != p.numel() or sq.device != p.device):
                raise ValueError("grad_sq: one fp32 sum per 512 elements of the parameter expected")
            descs[i] = _lib.AdamWDesc(p.data_ptr(), grad.data_ptr(),
                                      master.data_ptr() if master is not None else None,
                                      m.data_ptr(), v.data_ptr(), p.numel(),
                                      PLZ_DT_BF16 if p.dtype == torch.bfloat16 else PLZ_DT_FP32,
                                      g["clip_group"], g["lr"], g["clamp"][0], g["clamp"][1],
                                      0.0, 0, sq.data_ptr() if sq is not None else None)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if not bmap:
            total = _lib.lib().plz_adamw_plan(descs, len(live))
            if total < 0:
                raise _lib.PalettizeError("plz_adamw_plan failed: " +
                                          _lib.lib().plz_last_error().decode())
            table = self._upload(descs)
            ws = self._workspace(total)
            call("plz_adamw_step", table.data_ptr(), len(live), int(total), float(max_norms[0]),
                 float(max_norms[1]), float(self.betas[0]), float(self.betas[1]), self.eps,
                 self.weight_decay, self.step_count, self.last_norms.data_ptr(), ws.data_ptr(),
                 ws.numel(), stream)
            self._table = table  # keep alive until the launch has consumed it
            return self.last_norms
        builds = (_lib.BuildWDesc * len(live))()
        for i, e in enumerate(live):
            it = bmap.get(id(e[0]))
            if it is None:
                continue
            logits, palette, w, seed, counter = it[:5]
            pr = it[5] if len(it) > 5 else None
            N, K = w.shape
            builds[i] = _lib.BuildWDesc(logits.data_ptr(), None, palette.data_ptr(), w.data_ptr(),
                                        None, N, K, PLZ_DT_BF16, 0, 0,
                                        int(seed) & (2**64 - 1), int(counter) & (2**64 - 1),
                                        pr.data_ptr() if pr is not None else None)
        split = C.c_int64(0)
        total = _lib.lib().plz_adamw_plan_build(descs, builds, len(live), C.byref(split))
        if total < 0:
            raise _lib.PalettizeError("plz_adamw_plan_build failed: " +
                                      _lib.lib().plz_last_error().decode())
        table = self._upload(descs, builds)
        ws = self._workspace(total)
        nd = C.sizeof(descs)
        call("plz_adamw_step_build", table.data_ptr(), table.data_ptr() + nd, len(live),
             int(total), int(split.value), build.offset & (2**64 - 1), build.tau, build.mode,
             float(max_norms[0]), float(max_norms[1]), float(self.betas[0]),
             float(self.betas[1]), self.eps, self.weight_decay, self.step_count,
             self.last_norms.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        self._table = table
        build.built = {id(e[0]) for e in live if id(e[0]) in bmap}
        return self.last_norms

    def _upload(self, *tables):
        """The host tables, back to back, in one device buffer (through pinned memory)."""
        raw = b"".join(bytes(C.string_at(C.addressof(t), C.sizeof(t))) for t in tables)
        return torch.frombuffer(bytearray(raw), dtype=torch.uint8).pin_memory().to(
            self.device, non_blocking=True)

    def _workspace(self, total):
        need = query("plz_adamw_workspace", int(total))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws
