"""GPU parity: LoRA products, RMSNorm, SwiGLU, autograd Functions and the drop-in API."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32, gen, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
layer = pytest.importorskip("palettize_hip.layer")
import palettize_hip as P  # noqa: E402
from palettize_hip import fused_lut_linear_cuda as FL  # noqa: E402


@pytest.mark.parametrize("M,L,rank", [(1, 8, 8), (77, 520, 24), (1000, 264, 16), (130, 4104, 32),
                                      (16384, 2560, 16), (4096, 9728, 32)])
def test_lora_project_and_grad_t(dev, M, L, rank):
    """t = s x A^T (A [r, L]) and gt = s grad_y B (B [L, r]): ragged rows, reduction lengths
    that are not multiples of 32 or 256, every supported rank, and the full C3 shapes."""
    x = randn_bf16(M, L, seed=M + L)
    a = randn_bf16(rank, L, seed=rank, std=0.05)
    t = ops.lora_project(x.to(dev), a.to(dev), 0.5)
    assert t.shape == (M, rank)
    assert_close(f32(t), 0.5 * (f32(x).astype(np.float64) @ f32(a).T), what="lora t")
    b = randn_bf16(L, rank, seed=rank + 1, std=0.05)
    gt = ops.lora_grad_t(x.to(dev), b.to(dev), 2.0)
    assert_close(f32(gt), 2.0 * (f32(x).astype(np.float64) @ f32(b)), what="lora gt")


@pytest.mark.parametrize("M,N,K,rank", [(1000, 264, 512, 16), (1000, 264, 512, 32),
                                        (1, 8, 8, 8), (77, 520, 264, 24),
                                        (16384, 9728, 2560, 16), (16384, 2560, 9728, 32)])
def test_lora_weight_grads(dev, M, N, K, rank):
    x = randn_bf16(M, K, seed=1)
    gy = randn_bf16(M, N, seed=2)
    t = randn_bf16(M, rank, seed=3)
    gt = randn_bf16(M, rank, seed=4)
    ga, gb = ops.lora_weight_grads(x.to(dev), gy.to(dev), t.to(dev), gt.to(dev), 0.5)
    assert_close(f32(ga), f32(gt).T.astype(np.float64) @ f32(x), max_rel=1e-4, what="grad_a")
    assert_close(f32(gb), 0.5 * f32(gy).T.astype(np.float64) @ f32(t), max_rel=1e-4, what="grad_b")


@pytest.mark.parametrize("rows,cols", [(64, 2560), (300, 128), (17, 4096), (3, 128), (5000, 256),
                                       (70001, 128), (2049, 2560)])
def test_rmsnorm(dev, rows, cols):
    x = randn_bf16(rows, cols, seed=rows)
    w = (1 + 0.1 * torch.randn(cols, generator=gen(1))).to(torch.bfloat16)
    y, rstd = ops.rmsnorm_fwd(x.to(dev), w.to(dev), 1e-6)
    want, want_r = O.rmsnorm_fwd(f32(x), f32(w), 1e-6)
    # fp32 rsqrt against the fp64 oracle can flip the rounding of bf16(x r) by one ulp in rare
    # elements (a few in 9M): every element within two bf16 ulps, at least 99% exact
    d = np.abs(f32(y) - want)
    assert np.all(d <= np.abs(want) * 2.0 ** -6 + 1e-30) and np.mean(d == 0) > 0.99
    assert np.allclose(f32(rstd), want_r, rtol=1e-5)
    gy = randn_bf16(rows, cols, seed=rows + 1)
    gx, gw = ops.rmsnorm_bwd(x.to(dev), w.to(dev), rstd, gy.to(dev))
    wgx, wgw = O.rmsnorm_bwd(f32(x), f32(w), f32(gy), 1e-6)
    assert_close(f32(gx), wgx, what="rmsnorm grad_x")
    assert_close(f32(gw), wgw, max_rel=1e-4, what="rmsnorm grad_w")


@pytest.mark.parametrize("rows,cols", [(64, 2560), (300, 128), (17, 4096), (5000, 256), (2049, 2560)])
def test_add_rmsnorm_is_add_then_norm_bit_for_bit(dev, rows, cols):
    """plz_add_rmsnorm_fwd / plz_rmsnorm_bwd_add against the ops they fuse (torch's bf16 add,
    plz_rmsnorm_fwd, plz_rmsnorm_bwd's grad_x then torch's bf16 add), every bit; and the layer's
    autograd path against the unfused modules."""
    a = randn_bf16(rows, cols, seed=rows).to(dev)
    b = randn_bf16(rows, cols, seed=rows + 7, std=0.5).to(dev)
    w = (1 + 0.1 * torch.randn(cols, generator=gen(3))).to(torch.bfloat16).to(dev)
    s, y, rstd = ops.add_rmsnorm_fwd(a, b, w, 1e-6)
    ws = a + b
    wy, wr = ops.rmsnorm_fwd(ws, w, 1e-6)
    assert torch.equal(s.view(torch.int16), ws.view(torch.int16))
    assert torch.equal(y.view(torch.int16), wy.view(torch.int16)) and torch.equal(rstd, wr)
    gy = randn_bf16(rows, cols, seed=rows + 1).to(dev)
    ga = randn_bf16(rows, cols, seed=rows + 2).to(dev)
    gx = ops.rmsnorm_bwd_add(s, w, rstd, gy, ga)
    wgx, _ = ops.rmsnorm_bwd(ws, w, wr, gy)
    assert torch.equal(gx.view(torch.int16), (wgx + ga).view(torch.int16))
    # the layer's fused path (frozen weight) against add + RMSNorm module, through autograd
    norm = layer.RMSNorm(cols, 1e-6, dev)
    norm.weight.data.copy_(w)
    a1, b1 = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    a2, b2 = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    s1, y1 = layer.add_rmsnorm(norm, a1, b1)
    s2 = a2 + b2
    y2 = norm(s2)
    torch.autograd.backward([s1, y1], [ga, gy])
    torch.autograd.backward([s2, y2], [ga, gy])
    for u, v in ((a1.grad, a2.grad), (b1.grad, b2.grad)):
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))


def test_swiglu(dev):
    n = 8 * 4096
    g = randn_bf16(n, seed=1, std=3.0)
    u = randn_bf16(n, seed=2)
    h = ops.swiglu_fwd(g.to(dev), u.to(dev))
    want = O.swiglu_fwd(f32(g), f32(u))
    d = np.abs(f32(h) - want)
    assert np.all(d <= np.abs(want) * 2.0 ** -7) and np.mean(d == 0) > 0.99
    gh = randn_bf16(n, seed=3)
    gg, gu = ops.swiglu_bwd(g.to(dev), u.to(dev), gh.to(dev))
    wg, wu = O.swiglu_bwd(f32(g), f32(u), f32(gh))
    assert_close(f32(gg), wg, what="swiglu grad_gate")
    assert_close(f32(gu), wu, what="swiglu grad_up")


def test_swiglu_concatenated_layout(dev):
    """The fused gate/up projection's layout [rows, 2F] = [gate | up]: swiglu_fwd_cat and
    swiglu_bwd_cat are bit for bit the flat kernels on the separated halves, and the oracle's
    SwiGLU holds for them as for the flat ones."""
    rows, F = 96, 520
    gu = torch.cat([randn_bf16(rows, F, seed=11, std=3.0), randn_bf16(rows, F, seed=12)], 1)
    g, u = gu[:, :F].contiguous(), gu[:, F:].contiguous()
    h = ops.swiglu_fwd_cat(gu.to(dev))
    assert torch.equal(h, ops.swiglu_fwd(g.to(dev), u.to(dev)))
    want = O.swiglu_fwd(f32(g), f32(u))
    assert np.all(np.abs(f32(h) - want) <= np.abs(want) * 2.0 ** -7)
    gh = randn_bf16(rows, F, seed=13)
    grad = ops.swiglu_bwd_cat(gu.to(dev), gh.to(dev))
    gg, gup = ops.swiglu_bwd(g.to(dev), u.to(dev), gh.to(dev))
    assert torch.equal(grad[:, :F], gg) and torch.equal(grad[:, F:], gup)
    with pytest.raises(ValueError):
        ops.swiglu_bwd_cat(gu.to(dev), gh[:, :-8].contiguous().to(dev))


@pytest.mark.parametrize("M,N,K,r", [(16384, 2560, 9728, 16), (300, 1032, 768, 0),
                                     (2048, 512, 1024, 32)])
def test_grad_x_gemm_with_swiglu_backward_epilogue(dev, M, N, K, r):
    """plz_linear_bwd_x_dense_swiglu: [grad_gate | grad_up] bit for bit plz_linear_bwd_x_dense
    (with LoRA) followed by the SwiGLU backward over the pre-activations, on the layer's down
    shape (split last-wave tiles) and on a ragged edge."""
    gy = randn_bf16(M, N, seed=41).to(dev)
    w = (randn_bf16(N, K, seed=42).float() * 0.02).to(torch.bfloat16).to(dev)
    pre = randn_bf16(M, 2 * K, seed=43, std=2.0).to(dev)
    gt = randn_bf16(M, r, seed=44).to(dev) if r else None
    la = randn_bf16(r, K, seed=45, std=0.01).to(dev) if r else None
    got = ops.linear_bwd_x_dense_swiglu(gy, w, pre, gt, la)
    want = ops.swiglu_bwd_cat(pre, ops.linear_bwd_x_dense(gy, w, gt, la))
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,N,K,r,bias", [(300, 1032, 768, 0, False), (2048, 1024, 512, 16, True),
                                          (16384, 2560, 9728, 16, False), (4096, 2560, 2560, 0, True)])
def test_dense_gemm_with_residual_epilogue(dev, M, N, K, r, bias):
    """plz_linear_fwd_dense_residual: y = residual + x W^T (+ bias) (+ LoRA) bit for bit the
    dense GEMM followed by a bf16 tensor add, on whole tiles, a ragged edge and the split
    last-wave tiles (the layer's down shape); rows of y never written stay untouched."""
    x = randn_bf16(M, K, seed=31).to(dev)
    w = (randn_bf16(N, K, seed=32).float() * 0.02).to(torch.bfloat16).to(dev)
    res = randn_bf16(M, N, seed=33).to(dev)
    b = randn_bf16(N, 1, seed=34).reshape(N).to(dev) if bias else None
    t = randn_bf16(M, r, seed=35).to(dev) if r else None
    lb = randn_bf16(N, r, seed=36, std=0.01).to(dev) if r else None
    y = ops.linear_fwd_dense(x, w, b, t, lb, residual=res)
    want = ops.linear_fwd_dense(x, w, b, t, lb) + res
    assert torch.equal(y, want)
    # the residual may alias nothing else but may be any bf16 values, inf and nan included
    res2 = res.clone()
    res2[0, :8] = torch.tensor([float("inf"), float("-inf"), float("nan"), 0.0, -0.0, 1e30,
                                -1e-30, 3.0], dtype=torch.bfloat16)
    y2 = ops.linear_fwd_dense(x, w, b, t, lb, residual=res2)
    want2 = ops.linear_fwd_dense(x, w, b, t, lb) + res2
    assert torch.equal(y2.isnan(), want2.isnan())
    assert torch.equal(torch.nan_to_num(y2), torch.nan_to_num(want2))


@pytest.mark.parametrize("M,F,K,r", [(300, 384, 512, 32), (64, 128, 2560, 16),
                                     (2048, 9728, 2560, 32), (513, 640, 264, 0)])
def test_gate_up_gemm_with_swiglu_epilogue(dev, M, F, K, r):
    """plz_linear_fwd_dense_swiglu_cat on a [Wg; Wu] weight as stored: its pre-activations are
    the unsplit plz_linear_fwd_dense output (no workspace, so the same reduction order) and its
    h is swiglu_fwd_cat of them, every bit, with and without LoRA, for ragged row tiles, an odd
    count of 128-row halves (F = 384, 640), a single tile (which the dense forward would split
    over K when given its workspace) and the Qwen-4B gate/up shape; and the pre-activations
    against fp64."""
    x = randn_bf16(M, K, seed=M + F).to(dev)
    w = randn_bf16(2 * F, K, seed=K + 1, std=0.03).to(dev)
    t = b = None
    if r:
        t = randn_bf16(M, r, seed=3).to(dev)
        b = randn_bf16(2 * F, r, seed=4, std=0.05).to(dev)
    want_y = torch.empty((M, 2 * F), dtype=torch.bfloat16, device=dev)
    ops.call("plz_linear_fwd_dense", x.data_ptr(), w.data_ptr(), None, ops._ptr(t), ops._ptr(b),
             r, want_y.data_ptr(), None, 0, M, 2 * F, K, ops._stream(x))
    want_h = ops.swiglu_fwd_cat(want_y)
    y, h = ops.linear_fwd_dense_swiglu_cat(x, w, t, b)
    assert torch.equal(y.view(torch.int16), want_y.view(torch.int16))
    assert torch.equal(h.view(torch.int16), want_h.view(torch.int16))
    none, h2 = ops.linear_fwd_dense_swiglu_cat(x, w, t, b, keep_pre=False)
    assert none is None and torch.equal(h2.view(torch.int16), want_h.view(torch.int16))
    xs, ws = f32(x).astype(np.float64), f32(w).astype(np.float64)
    ref = xs @ ws.T + (f32(t).astype(np.float64) @ f32(b).T if r else 0.0)
    assert_close(f32(y), ref, what="gate/up pre-activations")


@pytest.mark.parametrize("M,r,train_pal", [(256, 16, True), (4096, 16, True), (4096, 32, False)])
def test_lut_linear_autograd_with_lora(dev, M, r, train_pal):
    """From 4096 rows the forward dequantises W once and grad_x reuses it; with the palette
    trained the LoRA weight gradients come from the grad_palette GEMM, else from their own
    kernel."""
    N, K = 384, 512
    idx, pal = make_weight(N, K, seed=5)
    x = randn_bf16(M, K, seed=6).to(dev).requires_grad_(True)
    pal_d = pal.to(dev).requires_grad_(train_pal)
    A = randn_bf16(r, K, seed=7, std=0.05).to(dev).requires_grad_(True)
    B = randn_bf16(N, r, seed=8, std=0.05).to(dev).requires_grad_(True)
    packed = ops.pack_indices(idx.to(dev))
    y = P.lut_linear(x, packed, pal_d, None, A, B, 2.0)
    gy = randn_bf16(M, N, seed=9).to(dev)
    y.backward(gy)
    W = O.dequant(idx.numpy(), pal.numpy()).astype(np.float64)
    xs, As, Bs, gys = f32(x), f32(A), f32(B), f32(gy)
    assert_close(f32(y), xs @ W.T + 2.0 * (xs @ As.T) @ Bs.T, what="y")
    gt = 2.0 * gys @ Bs
    assert_close(f32(x.grad), gys @ W + gt @ As, what="grad_x")
    if train_pal:
        assert_close(f32(pal_d.grad), O.grad_palette(xs, gys, idx.numpy()), max_rel=1e-3,
                     what="grad_palette")
    else:
        assert pal_d.grad is None
    assert_close(f32(A.grad), gt.T @ xs, what="grad_A")
    assert_close(f32(B.grad), gys.T @ (2.0 * xs @ As.T), what="grad_B")


def test_dropin_fused_lut_linear_reference_layout(dev):
    # reference layout: indices (K, N) int8, palette (G, 4) bf16 per 256 output channels
    M, K, N, GS = 96, 640, 512, 256   # K not a multiple of 256 exercises the padding
    g = gen(21)
    idx_kn = torch.randint(0, 4, (K, N), generator=g, dtype=torch.int8)
    pal = torch.sort(torch.randn(N // GS, 4, generator=g) * 0.02, -1).values.to(torch.bfloat16)
    bias = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    x = randn_bf16(M, K, seed=22)
    xd = x.to(dev).requires_grad_(True)
    pd = pal.to(dev).requires_grad_(True)
    bd = bias.to(dev).requires_grad_(True)
    y = FL.fused_lut_linear(xd, pd, idx_kn.to(dev), bd, GS)
    W = O.reference_weight(idx_kn.numpy().astype(np.uint8), f32(pal), GS).astype(np.float64)
    assert_close(f32(y), f32(x) @ W + f32(bias), what="drop-in y")
    gy = randn_bf16(M, N, seed=23)
    y.backward(gy.to(dev))
    assert_close(f32(xd.grad), f32(gy) @ W.T, what="drop-in grad_x")
    assert pd.grad.dtype == torch.bfloat16 and pd.grad.shape == (N // GS, 4)
    dW = f32(x).T.astype(np.float64) @ f32(gy)          # (K, N)
    want = np.zeros((N // GS, 4))
    cls = idx_kn.numpy().astype(np.int64)
    for gg in range(N // GS):
        for c in range(4):
            sl = slice(gg * GS, (gg + 1) * GS)
            want[gg, c] = dW[:, sl][cls[:, sl] == c].sum()
    assert_close(f32(pd.grad), want, what="drop-in grad_palette")
    assert_close(f32(bd.grad), f32(gy).sum(0), what="drop-in grad_bias")


def test_dropin_soft_reference_layout(dev):
    M, K, N, GS, tau = 64, 512, 256, 256, 0.5
    g = gen(31)
    logits = torch.randn(4, K, N, generator=g).to(torch.float16)
    pal = torch.sort(torch.randn(N // GS, 4, generator=g) * 0.02, -1).values.to(torch.bfloat16)
    x = randn_bf16(M, K, seed=32)
    xd = x.to(dev).requires_grad_(True)
    pd = pal.to(dev).requires_grad_(True)
    ld = logits.to(dev).requires_grad_(True)
    seed_before = FL._SOFT_STEP_SEED
    y = FL.fused_lut_linear_soft(xd, pd, ld, None, GS, tau)
    seed = (seed_before + 1) & 0xFFFFFFFF
    # oracle: LCG noise with the reference indexing, native layout
    noise = O.c_gumbel_lcg(seed, N, K)
    lg_nk4 = f32(logits).transpose(2, 1, 0)
    pal_nat = O.expand_reference_palette(f32(pal), N, K, GS)
    _, _, w_hard = O.soft_weights(lg_nk4, noise, pal_nat, tau, O.W_HARD_NOISY)
    assert_close(f32(y), f32(x) @ O.bf16_round(w_hard.astype(np.float32)).T.astype(np.float64),
                 what="drop-in soft y")
    gy = randn_bf16(M, N, seed=33)
    y.backward(gy.to(dev))
    gl, gp = O.soft_backward(f32(x), f32(gy), lg_nk4, noise, pal_nat, tau)
    assert ld.grad.shape == (4, K, N) and ld.grad.dtype == torch.float16
    assert_close(f32(ld.grad), gl.transpose(2, 1, 0), what="drop-in grad_logits")
    want_gp = gp.reshape(N // GS, GS, -1, 4).sum(axis=(1, 2))
    assert_close(f32(pd.grad), want_gp, what="drop-in soft grad_palette")


@pytest.mark.parametrize("ste", [True, False], ids=["ste", "pure-soft"])
def test_dropin_soft_supplied_noise(dev, ste):
    """fused_lut_linear_soft(..., noise=, ste=): noise in the logits' (4, K, N) layout replaces
    the LCG draw (the step seed does not advance); ste=False puts W_soft in the forward. The
    backward is the same STE backward either way."""
    M, K, N, GS, tau = 64, 512, 256, 256, 0.7
    g = gen(41)
    logits = torch.randn(4, K, N, generator=g).to(torch.float16)
    pal = torch.sort(torch.randn(N // GS, 4, generator=g) * 0.02, -1).values.to(torch.bfloat16)
    noise_ref = torch.from_numpy(O.gumbel_philox(4 * K * N, seed=42).reshape(4, K, N))
    x = randn_bf16(M, K, seed=43)
    xd = x.to(dev).requires_grad_(True)
    pd = pal.to(dev).requires_grad_(True)
    ld = logits.to(dev).requires_grad_(True)
    seed_before = FL._SOFT_STEP_SEED
    y = FL.fused_lut_linear_soft(xd, pd, ld, None, GS, tau, noise=noise_ref.to(dev), ste=ste)
    assert FL._SOFT_STEP_SEED == seed_before
    lg_nk4 = f32(logits).transpose(2, 1, 0)
    noise = noise_ref.numpy().transpose(2, 1, 0)
    pal_nat = O.expand_reference_palette(f32(pal), N, K, GS)
    mode = O.W_HARD_NOISY if ste else O.W_SOFT
    _, _, w_fwd = O.soft_weights(lg_nk4, noise, pal_nat, tau, mode)
    assert_close(f32(y), f32(x) @ O.bf16_round(w_fwd.astype(np.float32)).T.astype(np.float64),
                 what="drop-in soft y (supplied noise)")
    gy = randn_bf16(M, N, seed=44)
    y.backward(gy.to(dev))
    gl, gp = O.soft_backward(f32(x), f32(gy), lg_nk4, noise, pal_nat, tau)
    assert_close(f32(ld.grad), gl.transpose(2, 1, 0), what="drop-in grad_logits (supplied noise)")
    want_gp = gp.reshape(N // GS, GS, -1, 4).sum(axis=(1, 2))
    assert_close(f32(pd.grad), want_gp, what="drop-in soft grad_palette (supplied noise)")


@pytest.mark.parametrize("M,N,K", [(300, 256, 512), (64, 1024, 256)])
def test_dense_swiglu_epilogue(dev, M, N, K):
    """Gate and up in one GEMM with the SwiGLU in the epilogue: the HF bf16 formula against the
    oracle, and bit for bit the unfused dense GEMMs + plz_swiglu_fwd (no tail split here, so
    both accumulate every output in the same order)."""
    x = randn_bf16(M, K, seed=51)
    wg = randn_bf16(N, K, seed=52, std=0.05)
    wu = randn_bf16(N, K, seed=53, std=0.05)
    xd, wgd, wud = x.to(dev), wg.to(dev), wu.to(dev)
    h = ops.linear_fwd_dense_swiglu(xd, ops.swiglu_weight(wgd, wud))
    assert h.shape == (M, N)
    g = O.bf16_round((f32(x).astype(np.float64) @ f32(wg).T).astype(np.float32))
    u = O.bf16_round((f32(x).astype(np.float64) @ f32(wu).T).astype(np.float32))
    want = O.bf16_round(O.silu(g).astype(np.float32)) * u
    assert_close(f32(h), want, what="fused SwiGLU")
    assert ops.query("plz_linear_fwd_dense_workspace", M, N, K) == 0
    ref = ops.swiglu_fwd(ops.linear_fwd_dense(xd, wgd), ops.linear_fwd_dense(xd, wud))
    assert torch.equal(h, ref)
