"""GPU: the LoRA weight gradients computed inside the hard grad_palette GEMM
(plz_lut_linear_bwd_palette_lora) and the soft backward's dW GEMM (plz_soft_bwd_lora) against
the fp64 oracle of QwenLoRA's autograd (qwen_model.py:291-304): grad_A = s (gy B)^T x,
grad_B = s gy^T (x A^T). The palette (and logits) gradients of the same call must be
bit-equal to those of the call without LoRA, and the whole result bit-repeatable. Shapes cover
a ragged last row tile (N = 1032), a reduction shorter than one stage, split-M launches (the
soft backward's fp32 split rows among them) and every supported rank."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32, gen, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")


@pytest.mark.parametrize("M,N,K,rank,scale", [
    (512, 2560, 2560, 16, 2.0),   # config 1 shape
    (300, 1032, 768, 8, 1.0),
    (77, 136, 256, 24, 0.5),
    (2048, 256, 512, 32, 1.0),
    (4096, 1024, 2560, 16, 2.0),
])
def test_bwd_palette_lora(dev, M, N, K, rank, scale):
    idx, _ = make_weight(N, K, seed=M + N)
    p = ops.pack_indices(idx.to(dev))
    x = randn_bf16(M, K, seed=1).to(dev)
    gy = randn_bf16(M, N, seed=2).to(dev)
    a = randn_bf16(rank, K, seed=3, std=0.01).to(dev)
    b = randn_bf16(N, rank, seed=4, std=0.01).to(dev)
    gp, ga, gb = ops.lut_linear_bwd_palette_lora(x, gy, p, a, b, scale)
    assert torch.equal(gp, ops.lut_linear_bwd_palette(x, gy, p))
    wa, wb = O.lora_weight_grads(f32(x), f32(gy), f32(a), f32(b), scale)
    assert_close(f32(ga), wa, what="grad_a")
    assert_close(f32(gb), wb, what="grad_b")
    gp2, ga2, gb2 = ops.lut_linear_bwd_palette_lora(x, gy, p, a, b, scale)
    assert torch.equal(gp, gp2) and torch.equal(ga, ga2) and torch.equal(gb, gb2)
    # fp32 outputs: the same sums before the bf16 rounding
    _, fa, fb = ops.lut_linear_bwd_palette_lora(x, gy, p, a, b, scale, out_dtype=torch.float32)
    assert torch.equal(fa.to(torch.bfloat16), ga) and torch.equal(fb.to(torch.bfloat16), gb)


def test_bwd_palette_lora_agrees_with_the_separate_route(dev):
    """Against lora_weight_grads on t = s x A^T and gt = s gy B (bf16), the route the fused
    call replaces: equal within the bf16 rounding of t and gt."""
    M, N, K, r, s = 1024, 512, 1024, 16, 2.0
    idx, _ = make_weight(N, K, seed=5)
    p = ops.pack_indices(idx.to(dev))
    x = randn_bf16(M, K, seed=6).to(dev)
    gy = randn_bf16(M, N, seed=7).to(dev)
    a = randn_bf16(r, K, seed=8, std=0.01).to(dev)
    b = randn_bf16(N, r, seed=9, std=0.01).to(dev)
    _, ga, gb = ops.lut_linear_bwd_palette_lora(x, gy, p, a, b, s)
    t = ops.lora_project(x, a, s)
    gt = ops.lora_grad_t(gy, b, s)
    ra, rb = ops.lora_weight_grads(x, gy, t, gt, 1.0, out_dtype=torch.bfloat16)
    assert_close(f32(ga), f32(ra).astype(np.float64), max_rel=2e-2, min_cos=0.9999, what="grad_a")
    assert_close(f32(gb), f32(rb).astype(np.float64), max_rel=2e-2, min_cos=0.9999, what="grad_b")


def test_bwd_palette_lora_empty_reduction_gives_zeros(dev):
    N, K, r = 256, 512, 16
    idx, _ = make_weight(N, K, seed=10)
    p = ops.pack_indices(idx.to(dev))
    x = torch.empty(0, K, dtype=torch.bfloat16, device=dev)
    gy = torch.empty(0, N, dtype=torch.bfloat16, device=dev)
    a = randn_bf16(r, K, seed=11).to(dev)
    b = randn_bf16(N, r, seed=12).to(dev)
    gp, ga, gb = ops.lut_linear_bwd_palette_lora(x, gy, p, a, b, 1.0)
    assert not gp.any() and not ga.any() and not gb.any()


def _soft_case(N, K, seed):
    _, pal = make_weight(N, K, seed=seed)
    logits = torch.randn(N, K, 4, generator=gen(seed + 1)).to(torch.bfloat16)
    return logits, pal


@pytest.mark.parametrize("M,N,K,rank,scale,philox", [
    (512, 2560, 2560, 16, 2.0, True),    # config 1 shape, unsplit (fused soft epilogue)
    (300, 1032, 768, 8, 1.0, False),     # ragged last row tile, noise tensor
    (77, 136, 256, 24, 0.5, True),
    (1024, 512, 1024, 32, 1.0, False),   # 2 splits: fp32 dW rows + split epilogue
    (2048, 1024, 2560, 16, 2.0, True),   # 4 splits
])
def test_soft_bwd_lora(dev, M, N, K, rank, scale, philox):
    logits, pal = _soft_case(N, K, seed=M + N)
    logits, pal = logits.to(dev), pal.to(dev)
    noise = (ops.PhiloxNoise(seed=99, offset=M) if philox else
             ops.gumbel_philox((N, K, 4), seed=98, offset=0, device=dev))
    x = randn_bf16(M, K, seed=1).to(dev)
    gy = randn_bf16(M, N, seed=2).to(dev)
    a = randn_bf16(rank, K, seed=3, std=0.01).to(dev)
    b = randn_bf16(N, rank, seed=4, std=0.01).to(dev)
    gl, gp, ga, gb = ops.soft_bwd_lora(x, gy, logits, noise, pal, 0.5, a, b, scale)
    rl, rp = ops.soft_bwd(x, gy, logits, noise, pal, 0.5)
    assert torch.equal(gl, rl) and torch.equal(gp, rp)
    wa, wb = O.lora_weight_grads(f32(x), f32(gy), f32(a), f32(b), scale)
    assert_close(f32(ga), wa, what="grad_a")
    assert_close(f32(gb), wb, what="grad_b")
    out2 = ops.soft_bwd_lora(x, gy, logits, noise, pal, 0.5, a, b, scale)
    assert all(torch.equal(u, v) for u, v in zip((gl, gp, ga, gb), out2))
    _, _, fa, fb = ops.soft_bwd_lora(x, gy, logits, noise, pal, 0.5, a, b, scale,
                                     out_dtype=torch.float32)
    assert torch.equal(fa.to(torch.bfloat16), ga) and torch.equal(fb.to(torch.bfloat16), gb)
    # the squared-gradient sums of each 512 stored values (row n, 128 k), with every other
    # output unchanged
    sq = torch.full((N * K // 128,), float("nan"), device=dev)
    out3 = ops.soft_bwd_lora(x, gy, logits, noise, pal, 0.5, a, b, scale, grad_sq=sq)
    assert all(torch.equal(u, v) for u, v in zip((gl, gp, ga, gb), out3))
    want_sq = (f32(gl).astype(np.float64) ** 2).reshape(-1, 512).sum(1)
    assert np.allclose(f32(sq), want_sq, rtol=1e-5, atol=0)


def test_soft_bwd_lora_empty_reduction_gives_zeros(dev):
    N, K, r = 256, 512, 16
    logits, pal = _soft_case(N, K, seed=13)
    x = torch.empty(0, K, dtype=torch.bfloat16, device=dev)
    gy = torch.empty(0, N, dtype=torch.bfloat16, device=dev)
    a = randn_bf16(r, K, seed=14).to(dev)
    b = randn_bf16(N, r, seed=15).to(dev)
    sq = torch.full((N * K // 128,), float("nan"), device=dev)
    gl, gp, ga, gb = ops.soft_bwd_lora(x, gy, logits.to(dev), ops.PhiloxNoise(1, 0), pal.to(dev),
                                       0.5, a, b, 1.0, grad_sq=sq)
    assert not gl.any() and not gp.any() and not ga.any() and not gb.any() and not sq.any()
    rl, rp = ops.soft_bwd(x, gy, logits.to(dev), ops.PhiloxNoise(1, 0), pal.to(dev), 0.5)
    assert not rl.any() and not rp.any()


@pytest.mark.parametrize("M,N,K", [(300, 1032, 768), (2048, 1024, 2560)])
def test_soft_autograd_lora_weight_grads_ride_on_the_dw_gemm(dev, M, N, K):
    """soft_lut_linear with LoRA: the backward takes grad_A, grad_B from the soft dW GEMM
    (plz_soft_bwd_lora); logits and palette gradients equal ops.soft_bwd's from the same P bit
    for bit."""
    from palettize_hip import soft_lut_linear
    r, s, tau = 16, 2.0, 0.5
    logits, pal = _soft_case(N, K, seed=M)
    logits = logits.to(dev).requires_grad_()
    pal = pal.to(dev).requires_grad_()
    spec = ops.PhiloxNoise(seed=5, offset=17)
    x = randn_bf16(M, K, seed=21).to(dev).requires_grad_()
    a = randn_bf16(r, K, seed=22, std=0.01).to(dev).requires_grad_()
    b = randn_bf16(N, r, seed=23, std=0.01).to(dev).requires_grad_()
    gy = randn_bf16(M, N, seed=24).to(dev)
    y = soft_lut_linear(x, pal, logits, spec, tau, lora_a=a, lora_b=b, lora_scale=s)
    y.backward(gy)
    wa, wb = O.lora_weight_grads(f32(x.detach()), f32(gy), f32(a.detach()), f32(b.detach()), s)
    assert_close(f32(a.grad), wa, what="grad_a")
    assert_close(f32(b.grad), wb, what="grad_b")
    # the forward keeps its P (fp16) and the backward reads it: the same P built here
    probs = torch.empty((N, K, 4), dtype=torch.float16, device=dev)
    ops.soft_build_w(logits.detach(), spec, pal.detach(), tau, probs=probs)
    rl, rp = ops.soft_bwd(x.detach(), gy, logits.detach(), None, pal.detach(), tau, probs=probs)
    assert torch.equal(logits.grad, rl) and torch.equal(pal.grad, rp)
    assert bool(torch.isfinite(x.grad.float()).all())


def test_lora_grads_of_an_empty_weight_are_zero(dev):
    """N == 0: grad_A [r, K] is zero (no output row contributes); K == 0: grad_B [N, r] is zero
    (x A^T is zero). Both entries write them although the weight itself is empty."""
    from palettize_hip import _lib
    lib = _lib.lib()
    r, K, N, M = 16, 512, 256, 64
    s = torch.cuda.current_stream().cuda_stream
    for entry in ("plz_lut_linear_bwd_palette_lora", "plz_soft_bwd_lora"):
        ga = torch.full((r, K), float("nan"), dtype=torch.bfloat16, device=dev)
        gb = torch.full((N, r), float("nan"), dtype=torch.bfloat16, device=dev)
        for n, k, out_a, out_b in ((0, K, ga, None), (N, 0, None, gb)):
            pa = None if out_a is None else out_a.data_ptr()
            pb = None if out_b is None else out_b.data_ptr()
            if entry == "plz_lut_linear_bwd_palette_lora":
                rc = lib.plz_lut_linear_bwd_palette_lora(None, None, None, None, None, r, 1.0,
                                                         None, pa, pb, _lib.PLZ_DT_BF16, None, 0,
                                                         M, n, k, s)
            else:
                rc = lib.plz_soft_bwd_lora(None, None, None, _lib.PLZ_DT_BF16, None, 0, 0, None,
                                           None, 0.5, 0, None, None, r, 1.0, None, None, pa, pb,
                                           _lib.PLZ_DT_BF16, None, None, 0, M, n, k, s)
            assert rc == 0, lib.plz_last_error()
        torch.cuda.synchronize()
        assert bool((ga == 0).all()) and bool((gb == 0).all()), entry


@pytest.mark.parametrize("M,N,K,philox", [(512, 2560, 2560, True), (300, 1032, 768, False),
                                          (1024, 512, 1024, True)])
def test_soft_bwd_lora_from_saved_probs(dev, M, N, K, philox):
    """The forward's P saved by the build (SoftBuildGroup(want_probs=True), fp16 as the
    reference's P_aos) and read by the backward (soft_bwd_lora(probs=...)): P against the fp64
    softmax of logits + noise to fp16 rounding; the logits and palette gradients against those
    recomputed from the noise to the parity bar (P rounded to fp16 is the only difference), the
    LoRA weight gradients bit for bit; unsplit (M 512) and split (M 1024) dW."""
    from palettize_hip import _lib
    logits, pal = _soft_case(N, K, seed=M + 3 * N)
    logits, pal = logits.to(dev), pal.to(dev)
    tau = 0.5
    if philox:
        noise = ops.PhiloxNoise(seed=31, offset=7 * M)
        grp = ops.SoftBuildGroup([(logits, ops.PhiloxNoise(31, 0), pal)], _lib.PLZ_W_HARD_NOISY,
                                 want_probs=True)
        grp.run(tau, 7 * M)
        z = ops.gumbel_philox((N, K, 4), seed=31, offset=7 * M, device=dev)
    else:
        noise = ops.gumbel_philox((N, K, 4), seed=5, offset=0, device=dev)
        grp = ops.SoftBuildGroup([(logits, noise, pal)], _lib.PLZ_W_HARD_NOISY, want_probs=True)
        grp.run(tau)
        z = noise
    probs = grp.probs[0]
    a_ = (f32(logits).astype(np.float64) + f32(z)) / tau
    e = np.exp(a_ - a_.max(-1, keepdims=True))
    want_p = e / e.sum(-1, keepdims=True)
    assert np.all(np.abs(f32(probs) - want_p) <= 2.0 ** -10 * want_p + 2.0 ** -24)
    x = randn_bf16(M, K, seed=11).to(dev)
    gy = randn_bf16(M, N, seed=12).to(dev)
    a = randn_bf16(16, K, seed=13, std=0.01).to(dev)
    b = randn_bf16(N, 16, seed=14, std=0.01).to(dev)
    gl, gp, ga, gb = ops.soft_bwd_lora(x, gy, logits, noise, pal, tau, a, b, 1.0)
    gl2, gp2, ga2, gb2 = ops.soft_bwd_lora(x, gy, logits, noise, pal, tau, a, b, 1.0,
                                           probs=probs)
    assert torch.equal(ga, ga2) and torch.equal(gb, gb2)
    assert_close(f32(gl2), f32(gl).astype(np.float64), what="grad_logits from saved P")
    assert_close(f32(gp2), f32(gp).astype(np.float64), what="grad_palette from saved P")


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(512, 256, 512), (1024, 128, 768)])
@pytest.mark.parametrize("philox", [False, True])
def test_soft_bwd_probs_from_the_single_build(dev, M, N, K, philox):
    """The single-linear build's P (plz_soft_build_w(_philox) p_out) bit for bit the batched
    build's, and plz_soft_bwd_probs (P in place of logits and noise, the reference's
    grad_W + P_aos backward) bit for bit soft_bwd_lora(probs=...) in grad_logits and
    grad_palette, for fp16 logits too; unsplit (M 512) and split (M 1024) dW. The batched
    build's P and soft_bwd_lora(probs=...) are pinned against the fp64 softmax and the
    recomputing backward in test_soft_bwd_lora_from_saved_probs."""
    from palettize_hip import _lib
    logits, pal = _soft_case(N, K, seed=M + 5 * N)
    logits, pal = logits.to(dev), pal.to(dev)
    tau = 0.5
    for ldt in (torch.bfloat16, torch.float16):
        lg = logits.to(ldt)
        noise = (ops.PhiloxNoise(seed=17, offset=3 * N) if philox
                 else ops.gumbel_philox((N, K, 4), seed=5, offset=0, device=dev))
        p1 = torch.empty((N, K, 4), dtype=torch.float16, device=dev)
        w1, _ = ops.soft_build_w(lg, noise, pal, tau, _lib.PLZ_W_HARD_NOISY, probs=p1)
        if philox:
            grp = ops.SoftBuildGroup([(lg, ops.PhiloxNoise(17, 0), pal)], _lib.PLZ_W_HARD_NOISY,
                                     want_probs=True)
            grp.run(tau, 3 * N)
        else:
            grp = ops.SoftBuildGroup([(lg, noise, pal)], _lib.PLZ_W_HARD_NOISY, want_probs=True)
            grp.run(tau)
        assert torch.equal(p1, grp.probs[0]) and torch.equal(w1, grp.outputs[0][0])
        x = randn_bf16(M, K, seed=21).to(dev)
        gy = randn_bf16(M, N, seed=22).to(dev)
        a = randn_bf16(16, K, seed=23, std=0.01).to(dev)
        b = randn_bf16(N, 16, seed=24, std=0.01).to(dev)
        gl, gp, _, _ = ops.soft_bwd_lora(x, gy, lg, noise, pal, tau, a, b, 1.0, probs=p1)
        gl2, gp2 = ops.soft_bwd(x, gy, lg, None, pal, tau, probs=p1)
        assert gl2.dtype == ldt
        assert torch.equal(gl, gl2) and torch.equal(gp, gp2)
