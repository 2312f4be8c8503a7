"""GPU parity: Gumbel noise, soft build-W, fused soft backward (through the C ABI)."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32, gen, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
from palettize_hip import PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN, PLZ_W_SOFT  # noqa: E402


def test_gumbel_philox_matches_oracle(dev):
    n = 1 << 16
    g = ops.gumbel_philox((n,), seed=(3 << 32) | 17, offset=5, device=dev)
    want = O.c_gumbel_philox(n, (3 << 32) | 17, 5)
    assert np.allclose(f32(g), want, rtol=2e-6, atol=2e-6)


def test_gumbel_lcg_matches_reference_hash(dev):
    N, K, seed = 40, 512, 12345
    g = ops.gumbel_lcg(N, K, seed, device=dev)
    want = O.c_gumbel_lcg(seed, N, K)
    assert np.allclose(f32(g), want, rtol=2e-6, atol=2e-6)


def _soft_inputs(N, K, seed, dtype=torch.bfloat16, logit_std=1.0):
    _, pal = make_weight(N, K, seed=seed)
    logits = (torch.randn(N, K, 4, generator=gen(seed + 1)) * logit_std).to(dtype)
    noise = torch.from_numpy(O.gumbel_philox(N * K * 4, seed=seed).reshape(N, K, 4))
    return logits, noise, pal


@pytest.mark.parametrize("mode", [PLZ_W_SOFT, PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN])
@pytest.mark.parametrize("tau", [2.0, 0.5, 0.1])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_soft_build_w(dev, mode, tau, dtype):
    N, K = 64, 512
    logits, noise, pal = _soft_inputs(N, K, seed=int(tau * 10) + mode, dtype=dtype)
    w, ws = ops.soft_build_w(logits.to(dev), noise.to(dev), pal.to(dev), tau, mode, want_soft=True)
    P, w_soft, w_fwd = O.soft_weights(f32(logits), noise.numpy(), pal.numpy(), tau, mode)
    got = w.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.bf16_bits(w_fwd.astype(np.float32))
    def near(bits, ref):
        # fp32 (GPU) vs fp64 (oracle) softmax, each rounded once to bf16: within one bf16
        # ulp of the reference, or a tiny absolute slack where the weight crosses zero
        v = O.bf16_to_f32(bits).astype(np.float64)
        return np.all(np.abs(v - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6 * np.abs(ref).max())

    if mode == PLZ_W_SOFT:
        assert near(got, w_fwd)
    elif mode == PLZ_W_HARD_PLAIN:
        # argmax of the bf16/fp16 logits themselves: exact, ties to the first index
        assert np.array_equal(got, want)
    else:
        # argmax of the noisy P: a bit-exact palette copy, except where the top two of
        # (logit + noise) / tau are so close that fp32 (GPU) and fp64 (oracle) may order them
        # differently (the GPU's P rounds both to the same value and takes the first)
        z = (f32(logits).astype(np.float64) + noise.numpy()) / tau
        top2 = np.sort(z, axis=-1)[..., -2:]
        gap = top2[..., 1] - top2[..., 0]
        tie = gap <= 1e-5 * (1.0 + np.abs(top2[..., 1]))
        bad = got != want
        assert not np.any(bad & ~tie), (
            f"{int(np.sum(bad & ~tie))} hard weights differ away from a near tie "
            f"(smallest gap {gap[bad].min() if bad.any() else 0:.3e})")
    assert near(ws.view(torch.int16).cpu().numpy().view(np.uint16), w_soft)


@pytest.mark.parametrize("mode", [PLZ_W_SOFT, PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN])
def test_soft_build_w_batched_matches_single(dev, mode):
    """One launch over linears of different shapes and logit dtypes equals the per-linear
    builds bit for bit, on two consecutive runs with different tau."""
    shapes = [(64, 512, torch.bfloat16), (8, 256, torch.float16), (136, 768, torch.bfloat16),
              (1024, 2560, torch.bfloat16)]
    items = []
    for i, (N, K, dt) in enumerate(shapes):
        lg, nz, pl = _soft_inputs(N, K, seed=40 + i, dtype=dt)
        items.append((lg.to(dev), nz.to(dev), pl.to(dev)))
    grp = ops.SoftBuildGroup(items, mode, want_soft=True)
    for tau in (0.7, 2.0):
        outs = grp.run(tau)
        for (lg, nz, pl), (w, ws) in zip(items, outs):
            w1, ws1 = ops.soft_build_w(lg, nz, pl, tau, mode, want_soft=True)
            assert torch.equal(w, w1) and torch.equal(ws, ws1)


@pytest.mark.parametrize("mode", [PLZ_W_SOFT, PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN])
def test_soft_build_w_batched_philox(dev, mode):
    """Descriptors without a noise tensor draw Philox noise in the kernel from their own key at
    the launch's counter offset: each output equals the single-linear plz_soft_build_w_philox
    bit for bit, and the oracle's build from the oracle's Philox noise (the reference's
    per-layer decorrelated in-kernel draw, fused_lut_kernel.cu:2071-2211)."""
    shapes = [(64, 512, torch.bfloat16, 11), (8, 256, torch.float16, 12),
              (136, 768, torch.bfloat16, (3 << 32) | 5), (1024, 2560, torch.bfloat16, 14)]
    items, host = [], []
    for i, (N, K, dt, seed) in enumerate(shapes):
        lg, _, pl = _soft_inputs(N, K, seed=60 + i, dtype=dt)
        items.append((lg.to(dev), ops.PhiloxNoise(seed, 0), pl.to(dev)))
        host.append((lg, pl, seed))
    grp = ops.SoftBuildGroup(items, mode, want_soft=True)
    for tau, offset in ((0.7, 0), (2.0, 1 << 32), (0.1, (5 << 32) + 12345)):
        outs = grp.run(tau, offset)
        for j, ((lg, nz, pl), (w, ws)) in enumerate(zip(items, outs)):
            w1, ws1 = ops.soft_build_w(lg, ops.PhiloxNoise(nz.seed, offset), pl, tau, mode,
                                       want_soft=True)
            assert torch.equal(w, w1) and torch.equal(ws, ws1), f"linear {j} tau {tau}"
            if j == 2:  # the oracle, from its own Philox noise
                lgc, plc, seed = host[j]
                N, K = lgc.shape[:2]
                noise = O.gumbel_philox(N * K * 4, seed, offset).reshape(N, K, 4)
                _, w_soft, w_fwd = O.soft_weights(f32(lgc), noise, plc.numpy(), tau, mode)
                got = O.bf16_to_f32(w.view(torch.int16).cpu().numpy().view(np.uint16))
                if mode == PLZ_W_SOFT:
                    assert np.allclose(got, w_fwd, rtol=2.0 ** -7, atol=1e-6)
                elif mode == PLZ_W_HARD_PLAIN:
                    want = O.bf16_to_f32(O.bf16_bits(w_fwd.astype(np.float32)))
                    assert np.array_equal(got, want)
                else:
                    # bit-exact except where the top two of (logit + noise) / tau are a near
                    # tie that fp32 (GPU) and fp64 (oracle) may order differently
                    want = O.bf16_to_f32(O.bf16_bits(w_fwd.astype(np.float32)))
                    z = (f32(lgc).astype(np.float64) + noise) / tau
                    top2 = np.sort(z, axis=-1)[..., -2:]
                    tie = top2[..., 1] - top2[..., 0] <= 1e-5 * (1.0 + np.abs(top2[..., 1]))
                    bad = got != want
                    assert not np.any(bad & ~tie), f"{int(np.sum(bad & ~tie))} differ off a tie"
                soft = O.bf16_to_f32(ws.view(torch.int16).cpu().numpy().view(np.uint16))
                assert np.allclose(soft, w_soft, rtol=2.0 ** -7, atol=1e-6)
    assert grp.generation == 3


@pytest.mark.parametrize("tau", [2.0, 0.5, 0.1])
@pytest.mark.parametrize("scaled", [False, True])
def test_soft_bwd(dev, tau, scaled):
    M, N, K = 192, 256, 512
    logits, noise, pal = _soft_inputs(N, K, seed=3)
    x = randn_bf16(M, K, seed=4)
    gy = randn_bf16(M, N, seed=5)
    gl, gp = ops.soft_bwd(x.to(dev), gy.to(dev), logits.to(dev), noise.to(dev), pal.to(dev), tau,
                          scaled)
    want_gl, want_gp = O.soft_backward(f32(x), f32(gy), f32(logits), noise.numpy(), pal.numpy(),
                                       tau, scaled)
    assert_close(f32(gl), want_gl, what="grad_logits")
    assert_close(f32(gp), want_gp, max_rel=1e-3, min_cos=0.99999, what="grad_palette")


@pytest.mark.parametrize("M,N,K", [(2048, 1024, 2560), (1100, 256, 512), (4160, 264, 768)])
def test_soft_bwd_split_reduction(dev, M, N, K):
    """Output grids too small for the GPU split the reduction over M; the last split of each
    tile sums the partials in a fixed order and runs the epilogue (ragged M: a partial stage
    in the last split; N = 264: a ragged tile row)."""
    pal_bytes = N * (K // 128) * 16
    assert ops.query("plz_soft_bwd_workspace", M, N, K) > pal_bytes, "expected a split launch"
    logits, noise, pal = _soft_inputs(N, K, seed=M)
    x = randn_bf16(M, K, seed=M + 1)
    gy = randn_bf16(M, N, seed=M + 2)
    args = (x.to(dev), gy.to(dev), logits.to(dev), noise.to(dev), pal.to(dev), 0.5)
    gl, gp = ops.soft_bwd(*args)
    want_gl, want_gp = O.soft_backward(f32(x), f32(gy), f32(logits), noise.numpy(), pal.numpy(),
                                       0.5)
    assert_close(f32(gl), want_gl, what="grad_logits (split)")
    assert_close(f32(gp), want_gp, max_rel=1e-3, min_cos=0.99999, what="grad_palette (split)")
    gl2, gp2 = ops.soft_bwd(*args)
    assert torch.equal(gl, gl2) and torch.equal(gp, gp2), "split soft backward must be deterministic"


def test_soft_bwd_fp16_logits(dev):
    M, N, K = 64, 128, 256
    logits, noise, pal = _soft_inputs(N, K, seed=8, dtype=torch.float16)
    x = randn_bf16(M, K, seed=9)
    gy = randn_bf16(M, N, seed=10)
    gl, gp = ops.soft_bwd(x.to(dev), gy.to(dev), logits.to(dev), noise.to(dev), pal.to(dev), 0.5)
    assert gl.dtype == torch.float16
    want_gl, want_gp = O.soft_backward(f32(x), f32(gy), f32(logits), noise.numpy(), pal.numpy(), 0.5)
    assert_close(f32(gl), want_gl, what="grad_logits fp16")
    assert_close(f32(gp), want_gp, max_rel=1e-3, min_cos=0.99999, what="grad_palette")


def test_dense_linear_matches_oracle(dev):
    M, N, K = 200, 264, 512
    w = randn_bf16(N, K, seed=1, std=0.02)
    x = randn_bf16(M, K, seed=2)
    gy = randn_bf16(M, N, seed=3)
    y = ops.linear_fwd_dense(x.to(dev), w.to(dev))
    assert_close(f32(y), f32(x).astype(np.float64) @ f32(w).T, what="dense fwd")
    gx = ops.linear_bwd_x_dense(gy.to(dev), w.to(dev))
    assert_close(f32(gx), f32(gy).astype(np.float64) @ f32(w), what="dense grad_x")


def test_gumbel_philox_finite_and_bounded_at_scale(dev):
    # 2^28 draws: a mapping that lets u reach 0 or 1 would show ~16 infinities here
    n = 1 << 28
    g = ops.gumbel_philox((n,), seed=0x5EED, offset=0, device=dev)
    assert bool(torch.isfinite(g).all())
    lo, hi = float(g.min()), float(g.max())
    # u in [2^-24, 1 - 2^-24]  =>  noise in [-log(24 ln 2), -log(-log(1 - 2^-24))]
    assert -2.82 < lo and hi < 16.64 + 1e-3
    del g


def test_soft_bwd_full_gate_shape_sampled_rows(dev):
    # gate_proj of the layer config (N=9728, K=2560) with Philox noise made on the GPU;
    # every output must be finite, and sampled output rows match the oracle
    M, N, K, tau = 256, 9728, 2560, 0.5
    _, pal = make_weight(N, K, seed=21)
    logits = (torch.randn(N, K, 4, generator=gen(22)) * 2.0).to(torch.bfloat16)
    noise = ops.gumbel_philox((N, K, 4), seed=1234, offset=0, device=dev)
    x = randn_bf16(M, K, seed=23)
    gy = randn_bf16(M, N, seed=24)
    gl, gp = ops.soft_bwd(x.to(dev), gy.to(dev), logits.to(dev), noise, pal.to(dev), tau)
    assert bool(torch.isfinite(gl).all()) and bool(torch.isfinite(gp).all())
    rows = torch.tensor([0, 1, 255, 256, 4097, 7777, 9600, N - 1])
    nz = noise[rows.to(dev)].cpu().numpy()
    want_gl, want_gp = O.soft_backward(f32(x), f32(gy[:, rows]), f32(logits[rows]), nz,
                                       pal[rows].numpy(), tau)
    assert_close(f32(gl[rows.to(dev)]), want_gl, what="grad_logits sampled rows")
    assert_close(f32(gp[rows.to(dev)]), want_gp, max_rel=1e-3, min_cos=0.99999,
                 what="grad_palette sampled rows")


@pytest.mark.parametrize("mode", [PLZ_W_SOFT, PLZ_W_HARD_NOISY, PLZ_W_HARD_PLAIN])
def test_soft_build_w_philox_draws_the_tensor_noise(dev, mode):
    """Noise drawn inside build-W equals plz_gumbel_philox's tensor bit for bit, so W too."""
    N, K = 264, 768
    logits, _, pal = _soft_inputs(N, K, seed=41)
    spec = ops.PhiloxNoise(seed=0xABCDEF123, offset=977)
    noise = spec.materialize(N, K, dev)
    w1, s1 = ops.soft_build_w(logits.to(dev), noise, pal.to(dev), 0.5, mode, want_soft=True)
    w2, s2 = ops.soft_build_w(logits.to(dev), spec, pal.to(dev), 0.5, mode, want_soft=True)
    assert torch.equal(w1, w2) and torch.equal(s1, s2)


@pytest.mark.parametrize("M,N,K", [(192, 256, 512), (2048, 1024, 2560)])
def test_soft_bwd_philox_matches_tensor_noise(dev, M, N, K):
    """The backward's epilogue redraws the forward's Philox noise: identical to passing the
    materialised noise (fused epilogue and split-over-M paths)."""
    logits, _, pal = _soft_inputs(N, K, seed=M)
    x = randn_bf16(M, K, seed=M + 1)
    gy = randn_bf16(M, N, seed=M + 2)
    spec = ops.PhiloxNoise(seed=77, offset=12345)
    noise = spec.materialize(N, K, dev)
    a = ops.soft_bwd(x.to(dev), gy.to(dev), logits.to(dev), noise, pal.to(dev), 0.5)
    b = ops.soft_bwd(x.to(dev), gy.to(dev), logits.to(dev), spec, pal.to(dev), 0.5)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
