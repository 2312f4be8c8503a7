"""Benchmark of the MI355X LUT-linear hot path (BASELINE.json metric).

One step = one hard LUT-linear forward + backward (grad_x, grad_palette, LoRA grads) over
the seven Qwen-4B linear shapes at M = 16384 tokens (batch 32 x seq 512),
straight-through through the frozen 2-bit indices, LoRA rank 16 (32 on o and down).
`value` = sum over shapes of 6*M*K*N FLOP / step time (LoRA FLOP excluded, as BASELINE.json counts it),
the step's kernels issued on one stream as the library's autograd issues them: from 4096
rows the forward dequantises W once and runs the dense GEMM, and grad_x reuses that W; the
grad_palette GEMM also yields both LoRA weight gradients from its dW tiles; the LoRA row
products t = x A^T and gt = grad_y B run as their own HBM-bound kernels. The per-kernel
rooflines come from the same K steps run again with HIP events around every launch.

Also reported (same JSON line): the decode GEMV of config 2 (36 layers x 7 linears, M in
{1, 4, 16}, one grouped launch per M) in GB/s of packed indices + palettes, the roofline of
the dominant kernel (HIP events on the launch stream), and the reference's CPU PyTorch path
(gather + matmul, torch autograd) on the host cores: config 1 in full (median of 10), the gate
shape's fwd+bwd at M = 16384 once, and a one-layer CPU GEMV.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only hard|gemv]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-palettize_amd"))

# (name, K, N, LoRA rank) of the seven Qwen-4B linears
SHAPES = [("q", 2560, 4096, 16), ("k", 2560, 1024, 16), ("v", 2560, 1024, 16),
          ("o", 4096, 2560, 32), ("gate", 2560, 9728, 16), ("up", 2560, 9728, 16),
          ("down", 9728, 2560, 32)]
M_TRAIN = 16384
LAYERS = 36
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# HBM-side bytes per launch of each GEMM kind, averaged over the 7 shapes: rocprofv3 FETCH_SIZE x 2.0
# + WRITE_SIZE x 1.0, the factors that make a plain 1 GiB device copy read as 1 GiB each way (two
# --pmc runs of `bench.py --only hard --steps 1 --warmup 1 --no-cpu --calibration-copy`; counters,
# commands and algorithmic bytes in profiles/lut_gemm_traffic_m16384.txt).
# fwd counts its dequant_kernel launch too (from 4096 rows it dequantises W and runs the dense
# GEMM; grad_x runs on the same W); grad_palette includes the LoRA weight-gradient partials.
GEMM_TRAFFIC_BYTES = {"fwd": 1009.1e6, "grad_x": 962.8e6, "grad_palette": 905.7e6}
KERNEL_NAMES = {"fwd": "dequant_kernel + gemm2_kernel<OP_ROW, OP_ROW, EPI_BF16> (fwd)",
                "grad_x": "gemm2_kernel<OP_ROW, OP_COL, EPI_BF16> (grad_x on the forward's W)",
                "grad_palette": "gemm2_kernel<OP_COL, OP_COL, EPI_PAL> (grad_palette + LoRA "
                                "weight gradients)"}


def _make_weight(N, K, gen, device):
    import torch
    from palettize_hip import ops
    idx = torch.randint(0, 4, (N, K), generator=gen, device=device, dtype=torch.uint8)
    pal = torch.sort(torch.randn(N, K // 256, 4, generator=gen, device=device) * 0.02,
                     dim=-1).values.contiguous()
    return ops.pack_indices(idx), pal, idx


class HardStep:
    """Inputs resident in HBM; run() issues one fwd+bwd of all seven shapes."""

    def __init__(self, device, seed=0):
        import torch
        g = torch.Generator(device=device).manual_seed(seed)
        self.items = []
        for name, K, N, r in SHAPES:
            packed, pal, _ = _make_weight(N, K, g, device)
            x = torch.randn(M_TRAIN, K, generator=g, device=device).to(torch.bfloat16)
            gy = torch.randn(M_TRAIN, N, generator=g, device=device).to(torch.bfloat16)
            a = (torch.randn(r, K, generator=g, device=device) * 0.01).to(torch.bfloat16)
            b = (torch.randn(N, r, generator=g, device=device) * 0.01).to(torch.bfloat16)
            self.items.append(dict(name=name, K=K, N=N, r=r, packed=packed, pal=pal, x=x, gy=gy,
                                   a=a, b=b))
        self.flop = sum(6.0 * M_TRAIN * it["K"] * it["N"] for it in self.items)
        self.events = None

    def run(self, timed=False):
        import torch
        from palettize_hip import ops
        rec = self.events if timed else None
        for it in self.items:
            x, gy, a, b = it["x"], it["gy"], it["a"], it["b"]
            r = it["r"]
            e = self._mark(rec, "lora", it, 2.0 * M_TRAIN * it["K"] * r, M_TRAIN * it["K"] * 2)
            t = ops.lora_project(x, a, 1.0)
            self._close(e)
            # as the library's autograd (functional.LUTLinearFunction) runs it: where the
            # library dequantises W for the forward GEMM, that W serves grad_x too
            staged = ops.lut_linear_staged(M_TRAIN, it["N"], it["K"])
            e = self._mark(rec, "fwd", it)
            if staged:
                w = ops.dequant(it["packed"], it["pal"])
                ops.linear_fwd_dense(x, w, None, t, b)
            else:
                ops.lut_linear_fwd(x, it["packed"], it["pal"], None, t, b)
            self._close(e)
            e = self._mark(rec, "lora", it, 2.0 * M_TRAIN * it["N"] * r, M_TRAIN * it["N"] * 2)
            gt = ops.lora_grad_t(gy, b, 1.0)
            self._close(e)
            e = self._mark(rec, "grad_x", it)
            if staged:
                ops.linear_bwd_x_dense(gy, w, gt, a)
            else:
                ops.lut_linear_bwd_x(gy, it["packed"], it["pal"], gt, a)
            self._close(e)
            # grad_palette and both LoRA weight gradients from one dW GEMM, as the library's
            # backward runs it (functional.LUTLinearFunction)
            e = self._mark(rec, "grad_palette", it)
            ops.lut_linear_bwd_palette_lora(x, gy, it["packed"], a, b, 1.0,
                                            out_dtype=torch.bfloat16)
            self._close(e)

    @staticmethod
    def _mark(rec, kind, it, flop=None, nbytes=0):
        if rec is None:
            return None
        import torch
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        flop = 2.0 * M_TRAIN * it["K"] * it["N"] if flop is None else flop
        rec.setdefault(kind, []).append((s, e, flop, nbytes))
        return e

    @staticmethod
    def _close(e):
        if e is not None:
            e.record()


def kernel_rooflines(events):
    """Per kind: algorithmic FLOP (and activation bytes) / summed event time."""
    out = {}
    for kind, lst in events.items():
        ms = sum(s.elapsed_time(e) for s, e, _, _ in lst)
        fl = sum(f for _, _, f, _ in lst)
        nb = sum(b for _, _, _, b in lst)
        out[kind] = dict(ms=ms, launches=len(lst), tflops=fl / (ms * 1e-3) / 1e12,
                         gbs=nb / (ms * 1e-3) / 1e9)
    return out


def bench_gemv(device, reps=20):
    """Config 2: 36 layers x 7 linears per grouped launch. The top-level M1/M4/M16 entries are
    the library's default (GemvGroup layout "auto": the bit-plane GEMV up to 8 tokens, its
    x-prep kernel and the GEMV both timed; the dequantising decode-layout kernel above);
    "planes" and "decode" hold each kernel at every M for comparison. GB/s as the metric
    defines it: (packed indices + fp32 palettes) / time, 1,135,411,200 B per launch;
    stream_gbs: the bytes the layouts actually stream (bf16 lookup words, 8 B per row and
    256-k group in place of 16)."""
    import torch
    from palettize_hip import ops
    g = torch.Generator(device=device).manual_seed(1)
    weights = []
    wbytes = sbytes = 0
    for _ in range(LAYERS):
        for name, K, N, _r in SHAPES:
            packed, pal, _ = _make_weight(N, K, g, device)
            weights.append((packed, pal, K))
            wbytes += packed.numel() * 4 + pal.numel() * 4
            sbytes += packed.numel() * 4 + pal.numel() * 2
    res = {"planes": {}, "decode": {}}
    for M in (1, 4, 16):
        items = [(torch.randn(M, K, generator=g, device=device).to(torch.bfloat16), p, pl)
                 for p, pl, K in weights]
        for layout in ("planes", "decode"):
            grp = ops.GemvGroup(items, layout=layout)
            for _ in range(3):
                grp.run()
            torch.cuda.synchronize()
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                grp.run()
            e.record()
            torch.cuda.synchronize()
            ms = s.elapsed_time(e) / reps
            gbs = wbytes / (ms * 1e-3) / 1e9
            r = dict(us=round(ms * 1e3, 2), gbs=round(gbs, 1), frac=round(gbs / PEAK_HBM_GBS, 4),
                     stream_gbs=round(sbytes / (ms * 1e-3) / 1e9, 1))
            res[layout][f"M{M}"] = r
            if layout == ("planes" if M <= 8 else "decode"):  # what layout "auto" picks
                res[f"M{M}"] = dict(r, layout=layout)
            del grp
        del items
    res["weight_bytes"] = wbytes
    res["stream_bytes"] = sbytes
    return res


def bench_soft(device, reps=5):
    """Config 4: soft (Gumbel-softmax) fwd + bwd on the gate shape 2560 -> 9728 at M=16384;
    logits bf16 [N, K, 4] ~ N(0,1), Philox noise fp32 passed in, tau in {2.0, 0.5, 0.1}. The
    build keeps P (fp16) and the backward reads it, as the reference's forward saves P_aos
    for its backward (fused_lut_linear_cuda.py:903-905, 919, 952-959)."""
    import torch
    from palettize_hip import ops
    K, N = 2560, 9728
    g = torch.Generator(device=device).manual_seed(2)
    logits = torch.randn(N, K, 4, generator=g, device=device).to(torch.bfloat16)
    noise = ops.gumbel_philox((N, K, 4), seed=0, device=device)
    pal = torch.sort(torch.randn(N, K // 256, 4, generator=g, device=device) * 0.02, -1).values.contiguous()
    x = torch.randn(M_TRAIN, K, generator=g, device=device).to(torch.bfloat16)
    gy = torch.randn(M_TRAIN, N, generator=g, device=device).to(torch.bfloat16)
    probs = torch.empty((N, K, 4), dtype=torch.float16, device=device)
    out = {}
    ev = lambda: torch.cuda.Event(enable_timing=True)
    for tau in (2.0, 0.5, 0.1):
        times = {"build_w": 0.0, "fwd_gemm": 0.0, "grad_x": 0.0, "soft_bwd": 0.0}
        for rep in range(reps + 1):
            e = [ev() for _ in range(5)]
            e[0].record()
            w, _ = ops.soft_build_w(logits, noise, pal, tau, probs=probs)
            e[1].record()
            ops.linear_fwd_dense(x, w)
            e[2].record()
            ops.linear_bwd_x_dense(gy, w)
            e[3].record()
            ops.soft_bwd(x, gy, logits, noise, pal, tau, probs=probs)
            e[4].record()
            torch.cuda.synchronize()
            if rep:
                for i, k in enumerate(times):
                    times[k] += e[i].elapsed_time(e[i + 1]) / reps
        tot = sum(times.values())
        flop = 6.0 * M_TRAIN * K * N
        bw_bytes = 34.0 * N * K  # build-W: 8 B logits + 16 B noise in, 2 B W + 8 B P out per weight
        out[f"tau{tau}"] = dict(ms=round(tot, 3), tflops=round(flop / (tot * 1e-3) / 1e12, 1),
                                build_w_gbs=round(bw_bytes / (times["build_w"] * 1e-3) / 1e9, 1),
                                **{f"{k}_ms": round(v, 3) for k, v in times.items()})
    bw = out["tau0.5"]["build_w_gbs"]
    out["roofline_build_w"] = {"bound": "hbm", "achieved": bw, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                               "frac": round(bw / PEAK_HBM_GBS, 4)}
    return out


def bench_layer(device, steps=4, warmup=2):
    """Config 5: one palettized Qwen-4B-shaped decoder-layer training step at 32 x 512."""
    import torch
    from palettize_hip.layer import LayerConfig, LayerTrainer
    cfg = LayerConfig()
    tr = LayerTrainer(cfg, device, seed=0, lora_b_std=0.01)
    hs = torch.randn(32, 512, cfg.hidden, generator=torch.Generator(device=device).manual_seed(4),
                     device=device).to(torch.bfloat16)
    for _ in range(warmup):
        tr.step(hs)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    losses = []
    for _ in range(steps):
        loss, _ = tr.step(hs)
        losses.append(loss)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    # algorithmic FLOP of the step: student linears 6MKN (fwd, grad_x, dW), teacher 2MKN,
    # LoRA 6Mr(K+N), causal attention 4*B*Hq*S^2*D/2 for the teacher's forward and 3x that
    # for the student (fwd + bwd)
    B, S, M = 32, 512, 32 * 512
    h, q, kv, f = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.intermediate
    lin = [(h, q), (h, kv), (h, kv), (q, h), (h, f), (h, f), (f, h)]  # (K, N)
    flop = sum(8.0 * M * k * n + 6.0 * M * cfg.lora_rank * (k + n) for k, n in lin)
    flop += 4 * (4.0 * B * cfg.heads * S * S * cfg.head_dim / 2)
    tflops = flop / (ms * 1e-3) / 1e12
    return dict(ms_per_step=round(ms, 2), tokens_per_s=round(M / (ms * 1e-3), 1),
                tflops=round(tflops, 1), mfma_frac=round(tflops / PEAK_BF16_TFLOPS, 4),
                loss_first=round(float(losses[0]), 5), loss_last=round(float(losses[-1]), 5),
                config="hidden 2560, 32/8 heads x 128, SwiGLU 9728, 7 soft palettized linears + LoRA r16, batch 32 x 512")


def cpu_baseline():
    """The reference's CPU PyTorch path (PalettizedLinear's fallback, qwen_model.py:183-192:
    flat palette gather with the int64 _flat_idx buffer, x @ W^T, plus QwenLoRA's
    (x A^T) B^T, qwen_model.py:291-304; backward by torch autograd) on the host cores:
      * value: the gate shape (2560 -> 9728, LoRA r16) hard fwd + bwd at M = 16384, timed
        once after a warm-up at M = 512, in TFLOP/s of 6 M K N;
      * config1: the single hard forward of config 1 (M 512, K = N = 2560, LoRA r16,
        seed 0), median of 10 runs after 3 warm-ups;
      * gemv: one layer's seven linears at M = 1 (gather + matmul), GB/s of packed indices +
        fp32 palettes (31,539,200 B per layer); 36 layers = 36 x the per-layer time."""
    import statistics

    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from torch_ref import native_flat_idx, palettized_linear_cpu
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    bf = torch.bfloat16

    def weight(N, K, g):
        idx = torch.randint(0, 4, (N, K), generator=g, dtype=torch.uint8)
        pal = torch.sort(torch.randn(N, K // 256, 4, generator=g) * 0.02, -1).values
        return native_flat_idx(idx), pal.to(bf)

    # config 1
    g = torch.Generator().manual_seed(0)
    M1, K1, N1 = 512, 2560, 2560
    x1 = torch.randn(M1, K1, generator=g).to(bf)
    fi1, pal1 = weight(N1, K1, g)
    a1 = (0.01 * torch.randn(16, K1, generator=g)).to(bf)
    b1 = (0.01 * torch.randn(N1, 16, generator=g)).to(bf)
    times = []
    with torch.no_grad():
        for rep in range(13):
            t0 = time.perf_counter()
            palettized_linear_cpu(x1, pal1, fi1, None, a1, b1, 1.0)
            if rep >= 3:
                times.append(time.perf_counter() - t0)
    c1 = statistics.median(times)
    c1_flop = 2.0 * M1 * K1 * N1 + 2.0 * M1 * 16 * (K1 + N1)
    _log(f"cpu config1: {c1 * 1e3:.2f} ms")

    # config 3, gate shape, fwd + bwd once (warm-up at M = 512)
    K, N, r = 2560, 9728, 16
    fi, pal = weight(N, K, g)
    a = (0.01 * torch.randn(r, K, generator=g)).to(bf)
    b = (0.01 * torch.randn(N, r, generator=g)).to(bf)

    def fwd_bwd(M):
        x = torch.randn(M, K, generator=g).to(bf).requires_grad_(True)
        gy = torch.randn(M, N, generator=g).to(bf)
        ps = [t.detach().clone().requires_grad_(True) for t in (pal, a, b)]
        t0 = time.perf_counter()
        y = palettized_linear_cpu(x, ps[0], fi, None, ps[1], ps[2], 1.0)
        y.backward(gy)
        return time.perf_counter() - t0

    fwd_bwd(512)
    gate_s = fwd_bwd(M_TRAIN)
    gate_tflops = 6.0 * M_TRAIN * K * N / gate_s / 1e12
    _log(f"cpu gate fwd+bwd M={M_TRAIN}: {gate_s:.2f} s")
    del fi, pal

    # config 2: one layer's 7 GEMVs at M = 1
    layer = []
    wbytes = 0
    for name, K, N, _r in SHAPES:
        fi_l, pal_l = weight(N, K, g)
        layer.append((torch.randn(1, K, generator=g).to(bf), fi_l, pal_l))
        wbytes += N * K // 4 + N * (K // 256) * 16
    lt = []
    with torch.no_grad():
        for rep in range(4):
            t0 = time.perf_counter()
            for x, fi_l, pal_l in layer:
                palettized_linear_cpu(x, pal_l, fi_l)
            if rep:
                lt.append(time.perf_counter() - t0)
    layer_s = statistics.median(lt)
    _log(f"cpu gemv layer: {layer_s * 1e3:.1f} ms")
    return dict(value=round(gate_tflops, 5), unit="TFLOP/s", cores=cores, kind="port",
                sample=f"gate 2560->9728 hard fwd+bwd at M={M_TRAIN} (torch CPU bf16 gather + "
                       f"matmul + LoRA r16, autograd), timed once: {gate_s:.2f} s",
                config1=dict(ms_median=round(c1 * 1e3, 3), runs=10, warmup=3,
                             tflops=round(c1_flop / c1 / 1e12, 5)),
                gemv=dict(M=1, ms_per_layer=round(layer_s * 1e3, 3),
                          ms_36_layers=round(36 * layer_s * 1e3, 1),
                          gbs=round(wbytes / layer_s / 1e9, 3), weight_bytes_per_layer=wbytes,
                          note="one layer timed (median of 3 after 1 warm-up); 36 layers = 36x"))


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_attn(device, reps=10):
    """Causal grouped-query attention of the layer (B 32, S 512, 32 query / 8 kv heads x 128):
    forward (o, lse) and backward (dq, dk, dv), HIP-event time per call and FLOP rate
    (forward 4*B*Hq*S^2*D/2, backward 2.5x that)."""
    import torch
    from palettize_hip import ops
    B, S, Hq, Hkv, D = 32, 512, 32, 8, 128
    g = torch.Generator(device=device).manual_seed(4)
    q = torch.randn(B, S, Hq, D, generator=g, device=device).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, D, generator=g, device=device).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, D, generator=g, device=device).to(torch.bfloat16)
    go = torch.randn(B, S, Hq, D, generator=g, device=device).to(torch.bfloat16)
    flop = 4.0 * B * Hq * S * S * D / 2
    o, lse = ops.attn_fwd(q, k, v)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps * 1e3

    fwd_us = timed(lambda: ops.attn_fwd(q, k, v))
    bwd_us = timed(lambda: ops.attn_bwd(q, k, v, o, lse, go))
    return {"fwd_us": round(fwd_us, 1), "fwd_tflops": round(flop / fwd_us / 1e6, 1),
            "bwd_us": round(bwd_us, 1), "bwd_tflops": round(2.5 * flop / bwd_us / 1e6, 1),
            "config": "batch 32 x 512, 32/8 heads x 128, causal"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["hard", "gemv", "soft", "layer", "attn"], default=None)
    ap.add_argument("--calibration-copy", action="store_true",
                    help="first run a plain 1 GiB device copy (fp32 -> fp32), the reference "
                         "kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only: the LUT-linear path has no "
              "multi-GPU component (each rank would run these kernels on its own shard of the "
              "tokens or rows). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    from palettize_hip import _lib
    _lib.lib()

    out = {"metric": "LUT-linear fwd+bwd TFLOP/s @M=16384 (7 Qwen-4B shapes)",
           "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (uniform 2-bit indices, N(0,0.02) sorted fp32 palettes, N(0,1) bf16 activations)",
           "config": {"workload": "config3: hard fwd+bwd (grad_x, grad_palette, LoRA r16/r32) "
                                  "of q,k,v,o,gate,up,down at M=16384",
                      "M": M_TRAIN, "global_batch": 32, "seq_len": 512, "parallelism": "none (1 GPU)"}}

    if args.calibration_copy:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)  # reads 1 GiB, writes 1 GiB
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    if args.only in (None, "hard"):
        _log("hard: building inputs")
        step = HardStep(dev)
        for _ in range(args.warmup):
            step.run()
        torch.cuda.synchronize()
        # value: K steps bracketed by one event pair (no events between kernels: each one costs
        # a few microseconds of stream time). One stream, as the library's backward runs: the
        # grad_palette GEMM on a second stream beside grad_x measured slower (both GEMMs fill
        # the GPU and only contend).
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(args.steps):
            step.run()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        tflops = step.flop / (ms * 1e-3) / 1e12
        # per-kernel launch durations: one stream with an event pair around every kernel (no
        # other kernel shares the GPU)
        step.events = {}
        for _ in range(args.steps):
            step.run(timed=True)
        torch.cuda.synchronize()
        kr = kernel_rooflines(step.events)
        dom = max((k for k in kr if k != "lora"), key=lambda k: kr[k]["ms"])
        out.update(value=round(tflops, 2), ms_per_step=round(ms, 3))
        out["roofline"] = {"bound": "mfma", "kernel": KERNEL_NAMES[dom],
                           "achieved": round(kr[dom]["tflops"], 1), "peak": PEAK_BF16_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(kr[dom]["tflops"] / PEAK_BF16_TFLOPS, 4),
                           "traffic": GEMM_TRAFFIC_BYTES[dom], "traffic_unit": "bytes/launch"}
        out["kernels"] = {k: {"tflops": round(v["tflops"], 1),
                              "ms_per_step": round(v["ms"] / args.steps, 3)} for k, v in kr.items()}
        # the LoRA products are HBM-bound: activation bytes streamed per second
        out["kernels"]["lora"]["gbs"] = round(kr["lora"]["gbs"], 1)
        _log(f"hard: {ms:.3f} ms/step, {tflops:.1f} TFLOP/s")
        del step
        torch.cuda.empty_cache()
    if args.only in (None, "gemv"):
        out["gemv"] = bench_gemv(dev)
        _log(f"gemv: {out['gemv']}")
    if args.only in (None, "soft"):
        out["soft"] = bench_soft(dev)
        _log(f"soft: {out['soft']}")
        torch.cuda.empty_cache()
    if args.only in (None, "attn"):
        out["attn"] = bench_attn(dev)
        _log(f"attn: {out['attn']}")
        torch.cuda.empty_cache()
    if args.only in (None, "layer"):
        out["layer"] = bench_layer(dev)
        _log(f"layer: {out['layer']}")
        torch.cuda.empty_cache()
    if not args.no_cpu and args.only is None:
        out["cpu_baseline"] = cpu_baseline()
        _log("cpu baseline done")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
