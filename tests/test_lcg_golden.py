"""The oracle's LCG Gumbel samplers against the reference's own Triton sampler (CPU).

tests/golden/lcg_triton_golden.npz holds outputs of the reference's ``_gumbel_sample`` and
``compute_P_W_ste_kernel`` (triton_soft_forward.py:51-66, :83-181), written by
tests/golden/make_lcg_golden.py with triton's CPU interpreter (whose tl.log is numpy's fp32
log, so the oracle's numpy noise can be compared bit for bit).

* The Triton variant (int32, arithmetic shifts) must equal the golden noise on every draw.
* The CUDA variant (uint32, fused_lut_kernel.cu:1245-1256) must equal it wherever neither
  shifted intermediate has bit 31 set (there the two reference samplers agree by construction)
  and must differ almost everywhere else: a dropped or wrong constant, a wrong shift amount or
  a wrong seed/index combination breaks the first check on ~every element.
* The full soft build of the reference's preferred path (noise at idx = (k*N + n)*4 + c,
  softmax, plain-logit argmax, W_soft) must match through the oracle's layout mapping.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                    "lcg_triton_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def test_triton_variant_equals_reference_noise(gold):
    idx = gold["idx"].astype(np.uint32)
    for s in gold["seeds"]:
        want = gold[f"noise_{int(s)}"]
        got = O.gumbel_from_bits24(O.lcg_bits_i32(int(s), idx))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"seed {s}"
        assert np.array_equal(O.c_lcg_bits_i32(int(s), idx), O.lcg_bits_i32(int(s), idx))


def test_cuda_variant_equals_reference_where_shifts_agree(gold):
    idx = gold["idx"].astype(np.uint32)
    for s in gold["seeds"]:
        want = gold[f"noise_{int(s)}"]
        agree = O.lcg_variants_agree(int(s), idx)
        # bit 31 of two (nearly uniform) words clear: about a quarter of the draws
        assert 0.2 < agree.mean() < 0.3, agree.mean()
        got = O.gumbel_from_bits24(O.lcg_bits(int(s), idx))
        same = got.view(np.uint32) == want.view(np.uint32)
        assert same[agree].all(), f"seed {s}: {int((~same[agree]).sum())} agreeing draws differ"
        # where a shift sees bit 31 the samplers really differ (the golden is the int32 one)
        assert (~same[~agree]).mean() > 0.99
        assert np.array_equal(O.c_lcg_bits(int(s), idx), O.lcg_bits(int(s), idx))


def test_variant_noise_grids_use_reference_index(gold):
    """lcg_gumbel's [N, K, 4] grid draws element (n, k, c) at (k*N + n)*4 + c, in both
    variants and in both restatements (numpy fp32 log; C logf within 2 ulp)."""
    N, K = 24, 40
    for s in gold["seeds"]:
        for variant, bits in (("cuda", O.lcg_bits), ("triton", O.lcg_bits_i32)):
            grid = O.lcg_gumbel(int(s), N, K, variant)
            n, k, c = 5, 17, 3
            assert grid[n, k, c] == O.gumbel_from_bits24(bits(int(s), [(k * N + n) * 4 + c]))[0]
            assert np.allclose(O.c_gumbel_lcg(int(s), N, K, variant), grid, rtol=2e-6, atol=2e-6)


def test_soft_build_matches_reference_triton_path(gold):
    """P_aos, W_soft and W_ste of compute_P_W_ste_kernel from the oracle: Triton-variant
    noise, softmax((l + g) / tau), W_ste = palette[argmax of the plain logits]."""
    logits = gold["logits"].astype(np.float32)              # (4, K, N) fp16 values
    _, K, N = logits.shape
    pal_ref = O.bf16_to_f32(gold["palette_bits"])            # (G, 4), groups along N
    nat_logits = logits.transpose(2, 1, 0)                   # [N, K, 4]
    pal = np.repeat(pal_ref, 256, axis=0)[:N][:, None, :]    # [N, 1, 4]: row n -> group n//256
    for s, tau in zip(gold["pw_seeds"], gold["pw_taus"]):
        s = int(s)
        noise = O.lcg_gumbel(s, N, K, "triton")
        P, w_soft, w_ste = O.soft_weights(nat_logits, noise, pal, float(tau), O.W_HARD_PLAIN)
        P_ref = gold[f"P_aos_{s}"].astype(np.float64).transpose(1, 0, 2)   # [N, K, 4]
        # fp32 softmax rounded once to fp16 against fp64: within one fp16 ulp (2^-11 relative,
        # 2^-24 absolute below the normal range)
        ulp = np.maximum(np.abs(P) * 2.0 ** -10, 2.0 ** -24)
        assert np.all(np.abs(P_ref - P) <= ulp), f"seed {s}: P off by {np.abs(P_ref - P).max()}"
        ws_ref = O.bf16_to_f32(gold[f"W_soft_{s}"]).astype(np.float64).T
        assert np.all(np.abs(ws_ref - w_soft) <= np.abs(w_soft) * 2.0 ** -7 + 1e-9)
        want_ste = O.bf16_bits(w_ste.astype(np.float32)).T
        assert np.array_equal(gold[f"W_ste_{s}"], want_ste), f"seed {s}: W_ste"
        # the CUDA argmax (noisy P) is a different weight on a good share of positions here
        _, _, w_noisy = O.soft_weights(nat_logits, noise, pal, float(tau), O.W_HARD_NOISY)
        assert np.mean(O.bf16_bits(w_noisy.astype(np.float32)).T != want_ste) > 0.05
