"""GPU: NaN / Inf injected into the activations, gradients and logits propagate where the
mathematics puts them and nowhere else (the reference detects a non-finite loss and skips
the step, train_qwen.py:1282-1298, so the kernels must neither hide a NaN nor spread it).

Each case runs a clean launch and one with planted non-finite values, and checks that the
outputs the planted values reach are non-finite while every other output is bit-equal to the
clean launch (the kernels reduce in a fixed order, so untouched outputs do not move)."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import f32, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
layer = pytest.importorskip("palettize_hip.layer")
from palettize_hip import PLZ_W_HARD_NOISY, PLZ_W_SOFT  # noqa: E402

NAN, INF = float("nan"), float("inf")


def _weight(N, K, seed, dev):
    idx, pal = make_weight(N, K, seed=seed)
    return idx, ops.pack_indices(idx.to(dev)), pal.to(dev)


@pytest.mark.parametrize("M,N,K,staged", [(300, 1032, 768, True), (4096, 2560, 2560, True),
                                          (4096, 2560, 2560, False)])
def test_forward_rows_of_a_nonfinite_input_go_nonfinite(dev, M, N, K, staged):
    """staged: from 4096 rows W dequantised into the workspace and the dense GEMM; else the
    one-pass LUT GEMM."""
    _, p, pl = _weight(N, K, 1, dev)
    x = randn_bf16(M, K, seed=2).to(dev)
    clean = ops.lut_linear_fwd(x, p, pl, staged=staged)
    xb = x.clone()
    xb[3, 100] = NAN
    xb[M - 1, 5] = INF
    y = ops.lut_linear_fwd(xb, p, pl, staged=staged)
    bad = torch.zeros(M, dtype=torch.bool, device=dev)
    bad[3] = bad[M - 1] = True
    assert bool(torch.isnan(y[3]).all())
    assert not bool(torch.isfinite(y[M - 1]).any())  # +inf times palette values of both signs
    assert torch.equal(y[~bad], clean[~bad])
    gv = ops.lut_gemv(xb[:4].contiguous(), p, pl)  # the decode GEMV, rows 0..3 (NaN in row 3)
    assert bool(torch.isnan(gv[3]).all()) and bool(torch.isfinite(gv[:3]).all())


@pytest.mark.parametrize("M", [1, 5, 16])
def test_planes_gemv_tokens_of_a_nonfinite_input_go_nonfinite(dev, M):
    """The bit-plane GEMV: a NaN or +-inf in token t's x makes every output of token t
    non-finite (its e4m3 pieces are NaN); the other tokens are bit-equal to a clean launch (the
    scale of a group is set by its finite values only)."""
    N, K = 264, 768
    _, p, pl = _weight(N, K, 9, dev)
    pi, li = ops.gemv_pack_planes(p), ops.gemv_pack_palettes(pl)
    x = randn_bf16(M, K, seed=10).to(dev)
    clean = ops.lut_gemv_planes(x, pi, li, N)
    xb = x.clone()
    xb[M - 1, 300] = NAN if M % 2 else INF
    if M > 2:
        xb[1, 700] = -INF
    y = ops.lut_gemv_planes(xb, pi, li, N)
    bad = torch.zeros(M, dtype=torch.bool, device=dev)
    bad[M - 1] = True
    if M > 2:
        bad[1] = True
    assert not bool(torch.isfinite(y[bad]).any())
    assert torch.equal(y[~bad], clean[~bad])


@pytest.mark.parametrize("M", [512, 4096])  # the LUT GEMM; dequantised W + dense GEMM
def test_grad_x_rows_of_a_nonfinite_gradient_go_nonfinite(dev, M):
    N, K = 1024, 2560
    _, p, pl = _weight(N, K, 3, dev)
    gy = randn_bf16(M, N, seed=4).to(dev)
    clean = ops.lut_linear_bwd_x(gy, p, pl)
    g2 = gy.clone()
    g2[17, 9] = NAN
    gx = ops.lut_linear_bwd_x(g2, p, pl)
    assert bool(torch.isnan(gx[17]).all())
    rows = torch.arange(M, device=dev) != 17
    assert torch.equal(gx[rows], clean[rows])


def test_grad_palette_nan_reaches_only_its_column_group(dev):
    """x[m, k] = NaN makes dW[n, k] NaN for every row n: the class sum of group k // 256 that
    column k's index selects goes NaN in every row; other groups stay bit-equal."""
    M, N, K, k = 1024, 512, 1024, 300
    idx, p, _ = _weight(N, K, 5, dev)
    x = randn_bf16(M, K, seed=6).to(dev)
    gy = randn_bf16(M, N, seed=7).to(dev)
    clean = ops.lut_linear_bwd_palette(x, gy, p)
    xb = x.clone()
    xb[40, k] = NAN
    g = ops.lut_linear_bwd_palette(xb, gy, p)
    cls = idx[:, k].long().to(dev)
    hit = g[torch.arange(N, device=dev), k // 256, cls]
    assert bool(torch.isnan(hit).all())
    other = torch.ones(K // 256, dtype=torch.bool, device=dev)
    other[k // 256] = False
    assert torch.equal(g[:, other], clean[:, other])


def test_soft_build_w_with_a_nan_logit(dev):
    """A NaN logit makes that weight's P NaN: W_soft is NaN, and the hard pick, whose
    comparisons are all false against NaN, keeps the first entry (the first-max rule of
    fused_lut_kernel.cu:1998-2003 evaluated with IEEE comparisons). Other weights do not move."""
    N, K = 64, 512
    _, pal = make_weight(N, K, seed=8)
    logits = torch.randn(N, K, 4, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    noise = torch.from_numpy(O.gumbel_philox(N * K * 4, 10).reshape(N, K, 4))
    lg, nz, pl = logits.to(dev), noise.to(dev), pal.to(dev)
    w0, s0 = ops.soft_build_w(lg, nz, pl, 0.5, PLZ_W_HARD_NOISY, want_soft=True)
    lb = lg.clone()
    lb[7, 33, 2] = NAN
    w1, s1 = ops.soft_build_w(lb, nz, pl, 0.5, PLZ_W_HARD_NOISY, want_soft=True)
    ws, _ = ops.soft_build_w(lb, nz, pl, 0.5, PLZ_W_SOFT)
    assert bool(torch.isnan(s1[7, 33])) and bool(torch.isnan(ws[7, 33]))
    first = O.bf16_to_f32(O.bf16_bits(pal[7, 0, 0].numpy()))
    assert float(w1[7, 33].float()) == float(first)
    mask = torch.ones(N, K, dtype=torch.bool, device=dev)
    mask[7, 33] = False
    assert torch.equal(w1[mask], w0[mask]) and torch.equal(s1[mask], s0[mask])


def test_distillation_loss_of_a_nan_student_is_nan(dev):
    t = randn_bf16(2, 16, 256, seed=11).to(dev)
    s = randn_bf16(2, 16, 256, seed=12).to(dev)
    s[1, 3, 7] = NAN
    loss, l_cos = layer.compute_loss(s.requires_grad_(True), t)
    assert not bool(torch.isfinite(loss)) and not bool(torch.isfinite(l_cos))


def test_argument_errors_come_back_as_exceptions(dev):
    """Mis-shaped or misaligned tensors are refused before any launch."""
    _, p, pl = _weight(256, 512, 13, dev)
    x = randn_bf16(8, 512, seed=14).to(dev)
    with pytest.raises(ValueError):
        ops.lut_linear_fwd(x[:, :256].contiguous(), p, pl)
    odd = torch.empty(8 * 512 + 1, dtype=torch.bfloat16, device=dev)[1:].view(8, 512)
    odd.copy_(x)
    with pytest.raises(Exception, match="aligned"):
        ops.lut_linear_fwd(odd, p, pl)


def test_layer_step_skips_a_nonfinite_loss(dev):
    """LayerTrainer.step(skip_nonfinite=True) on an input holding a NaN: no update, gradients
    cleared, step counter advanced (train_qwen.py:1282-1298); a finite step after it trains."""
    cfg = layer.LayerConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512)
    tr = layer.LayerTrainer(cfg, dev, seed=3, lora_b_std=0.02)
    hs = randn_bf16(2, 16, 256, seed=15).to(dev)
    params = tr.logits + tr.others
    before = [q.detach().clone() for q in params]
    bad = hs.clone()
    bad[0, 4, 9] = NAN
    loss, _ = tr.step(bad, skip_nonfinite=True)
    assert not bool(torch.isfinite(loss)) and tr.skipped == 1 and tr.step_idx == 1
    assert all(q.grad is None for q in params)
    assert all(torch.equal(q, b) for q, b in zip(params, before))
    loss, _ = tr.step(hs, skip_nonfinite=True)
    assert bool(torch.isfinite(loss)) and tr.skipped == 1 and tr.step_idx == 2
    assert any(not torch.equal(q, b) for q, b in zip(params, before))
