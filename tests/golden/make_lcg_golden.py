"""Writes tests/golden/lcg_triton_golden.npz: input/output vectors of the reference's own
Gumbel LCG sampler, the one oracle function nothing else pins.

Run in the build container only (it needs /root/reference and triton's CPU interpreter):

    TRITON_INTERPRET=1 python tests/golden/make_lcg_golden.py

It imports /root/reference/scripts/triton_soft_forward.py and runs, on the CPU:
  * ``_gumbel_sample(seed, idx)`` (triton_soft_forward.py:51-66) through a one-line wrapper
    kernel, on idx 0..4095 and on 4096 seeded idx spread over [0, 2^31), for three seeds:
    the raw Gumbel noise of the reference's Triton sampler (int32 arithmetic);
  * ``compute_P_W_ste_kernel`` (triton_soft_forward.py:83-181) on fp16 logits (4, K, N) and
    a bf16 palette (G, 4), K = 32, N = 512, for two (seed, tau) pairs: P_aos (K, N, 4) fp16,
    W_soft and W_ste (K, N) bf16 -- the index mapping idx = (k*N + n)*4 + c, the softmax and
    the plain-logit argmax of the reference's preferred soft path.
Only the .npz is committed; nothing at test time reads the reference.
"""
from __future__ import annotations

import os
import sys

os.environ.setdefault("TRITON_INTERPRET", "1")

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

REF = "/root/reference/scripts"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lcg_triton_golden.npz")

SEEDS = (1, 7, 0x5EED1234)          # all < 2^31: the launcher passes int(step_seed) as int32
PW_CASES = ((3, 1.0), (0x5EED1234, 0.5))
K, N, GS = 32, 512, 256


ref_gumbel_sample = None  # the reference's _gumbel_sample, bound in main()


@triton.jit
def noise_kernel(out_ptr, idx_ptr, seed, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    idx = tl.load(idx_ptr + offs, mask=m, other=0)
    tl.store(out_ptr + offs, ref_gumbel_sample(seed, idx), mask=m)


def main():
    global ref_gumbel_sample
    if os.environ.get("TRITON_INTERPRET") != "1":
        raise SystemExit("run with TRITON_INTERPRET=1")
    sys.path.insert(0, REF)
    import triton_soft_forward as tsf
    ref_gumbel_sample = tsf._gumbel_sample

    rng = np.random.default_rng(20261202)
    idx = np.concatenate([np.arange(4096, dtype=np.int64),
                          rng.integers(0, 2**31, 4096, dtype=np.int64)]).astype(np.int32)
    idx_t = torch.from_numpy(idx)
    noise = {}
    for s in SEEDS:
        out = torch.empty(idx.size, dtype=torch.float32)
        noise_kernel[(idx.size // 256,)](out, idx_t, s, idx.size, BLOCK=256)
        noise[s] = out.numpy().copy()

    g = torch.Generator().manual_seed(7)
    logits = (torch.randn(4, K, N, generator=g) * 1.5).to(torch.float16)
    pal = torch.sort(torch.randn(N // GS, 4, generator=g) * 0.02, dim=-1).values.to(torch.bfloat16)
    pw = {}
    kern = tsf.compute_P_W_ste_kernel.fn  # the jitted kernel under its autotune wrapper
    for s, tau in PW_CASES:
        P = torch.empty((K, N, 4), dtype=torch.float16)
        ws = torch.empty((K, N), dtype=torch.bfloat16)
        wt = torch.empty((K, N), dtype=torch.bfloat16)
        grid = (triton.cdiv(K, 16), triton.cdiv(N, 32))
        kern[grid](logits, pal, P, ws, wt, K, N, N // GS, group_size=GS, tau=float(tau),
                   step_seed=int(s), BM=16, BN=32)
        pw[s] = (P.numpy().copy(), ws.view(torch.int16).numpy().view(np.uint16).copy(),
                 wt.view(torch.int16).numpy().view(np.uint16).copy())

    arrays = dict(idx=idx, seeds=np.array(SEEDS, np.int64),
                  pw_seeds=np.array([s for s, _ in PW_CASES], np.int64),
                  pw_taus=np.array([t for _, t in PW_CASES], np.float64),
                  logits=logits.numpy(),
                  palette_bits=pal.view(torch.int16).numpy().view(np.uint16))
    for s in SEEDS:
        arrays[f"noise_{s}"] = noise[s]
    for s, _ in PW_CASES:
        P, ws, wt = pw[s]
        arrays[f"P_aos_{s}"], arrays[f"W_soft_{s}"], arrays[f"W_ste_{s}"] = P, ws, wt
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
