"""GPU parity at BASELINE.json config 4, at its size: the soft (Gumbel-softmax) forward and backward
on the gate shape (K = 2560 -> N = 9728) at M = 16384, logits bf16 [N, K, 4] ~ N(0, 1), Gumbel
noise fp32 from a seeded Philox stream passed in as a tensor, tau in {2.0, 0.5, 0.1} -- the
calls the benchmark times (build-W, the dense forward and grad_x on W, the fused soft
backward), plus the soft backward that also returns the LoRA weight gradients.

Outputs are checked on sampled rows against the fp64 oracle at the north-star bar: W_hard bit
for bit except at near ties of (logit + noise) / tau, W_soft within one bf16 ulp, y / grad_x /
grad_logits / grad_palette at max-rel-err 1e-2 and cosine 0.9999 (grad_palette at 1e-3), the
LoRA weight gradients over all M rows at the same bar.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
from palettize_hip import PLZ_W_HARD_NOISY  # noqa: E402

M, K, N = 16384, 2560, 9728
ROWS_N = [0, 1, 255, 256, 257, 4097, 7777, 9600, N - 1]
ROWS_M = [0, 1, 127, 128, 8191, 12345, M - 257, M - 1]


@pytest.fixture(scope="module")
def c4(dev):
    g = torch.Generator(device=dev).manual_seed(2)
    logits = torch.randn(N, K, 4, generator=g, device=dev).to(torch.bfloat16)
    noise = ops.gumbel_philox((N, K, 4), seed=0, device=dev)
    pal = torch.sort(torch.randn(N, K // 256, 4, generator=g, device=dev) * 0.02,
                     -1).values.contiguous()
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    gy = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    rn = torch.tensor(ROWS_N, device=dev)
    return dict(logits=logits, noise=noise, pal=pal, x=x, gy=gy, rn=rn,
                lg_r=f32(logits[rn]), nz_r=noise[rn].cpu().numpy().astype(np.float64),
                pal_r=pal[rn].cpu().numpy(), x64=f32(x).astype(np.float64))


def _hard_bits_ok(got_bits, want_w, lg, nz, tau):
    want = O.bf16_bits(want_w.astype(np.float32))
    z = (lg.astype(np.float64) + nz) / tau
    top2 = np.sort(z, axis=-1)[..., -2:]
    tie = top2[..., 1] - top2[..., 0] <= 1e-5 * (1.0 + np.abs(top2[..., 1]))
    bad = got_bits != want
    return int(np.sum(bad & ~tie))


@pytest.mark.parametrize("tau", [2.0, 0.5, 0.1])
def test_config4_forward(dev, c4, tau):
    w, ws = ops.soft_build_w(c4["logits"], c4["noise"], c4["pal"], tau, PLZ_W_HARD_NOISY,
                             want_soft=True)
    _, w_soft, w_hard = O.soft_weights(c4["lg_r"], c4["nz_r"], c4["pal_r"], tau, O.W_HARD_NOISY)
    got = w[c4["rn"]].view(torch.int16).cpu().numpy().view(np.uint16)
    assert _hard_bits_ok(got, w_hard, c4["lg_r"], c4["nz_r"], tau) == 0, f"tau {tau}: W_hard"
    soft = O.bf16_to_f32(ws[c4["rn"]].view(torch.int16).cpu().numpy().view(np.uint16))
    assert np.all(np.abs(soft - w_soft) <= np.abs(w_soft) * 2.0 ** -7 + 1e-6 * np.abs(w_soft).max())
    # y on sampled rows m (all N) and sampled columns n (all M) against the GPU's own W
    y = ops.linear_fwd_dense(c4["x"], w)
    Wd = f32(w).astype(np.float64)
    rm = torch.tensor(ROWS_M, device=dev)
    assert_close(f32(y[rm]), c4["x64"][ROWS_M] @ Wd.T, what=f"tau {tau}: y rows")
    assert_close(f32(y[:, c4["rn"]]), c4["x64"] @ Wd[ROWS_N].T, what=f"tau {tau}: y columns")
    gx = ops.linear_bwd_x_dense(c4["gy"], w)
    assert_close(f32(gx[rm]), f32(c4["gy"][rm]).astype(np.float64) @ Wd,
                 what=f"tau {tau}: grad_x rows")


@pytest.mark.parametrize("tau", [2.0, 0.5, 0.1])
def test_config4_backward(dev, c4, tau):
    gl, gp = ops.soft_bwd(c4["x"], c4["gy"], c4["logits"], c4["noise"], c4["pal"], tau)
    assert bool(torch.isfinite(gl).all()) and bool(torch.isfinite(gp).all())
    gy_r = f32(c4["gy"][:, c4["rn"]])
    want_gl, want_gp = O.soft_backward(c4["x64"], gy_r, c4["lg_r"], c4["nz_r"], c4["pal_r"], tau)
    assert_close(f32(gl[c4["rn"]]), want_gl, what=f"tau {tau}: grad_logits rows")
    assert_close(f32(gp[c4["rn"]]), want_gp, max_rel=1e-3, min_cos=0.99999,
                 what=f"tau {tau}: grad_palette rows")
    gl2, gp2 = ops.soft_bwd(c4["x"], c4["gy"], c4["logits"], c4["noise"], c4["pal"], tau)
    assert torch.equal(gl, gl2) and torch.equal(gp, gp2), "soft backward must be deterministic"


def test_config4_backward_lora(dev, c4):
    """plz_soft_bwd_lora at the gate shape, M = 16384, rank 16: logits and palette gradients
    bit-equal to plz_soft_bwd, grad_A / grad_B against the fp64 oracle over all rows."""
    tau, scale, r = 0.5, 2.0, 16
    g = torch.Generator(device=dev).manual_seed(3)
    a = (torch.randn(r, K, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    b = (torch.randn(N, r, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    gl, gp, ga, gb = ops.soft_bwd_lora(c4["x"], c4["gy"], c4["logits"], c4["noise"], c4["pal"],
                                       tau, a, b, scale)
    gl0, gp0 = ops.soft_bwd(c4["x"], c4["gy"], c4["logits"], c4["noise"], c4["pal"], tau)
    assert torch.equal(gl, gl0) and torch.equal(gp, gp0)
    want_a, want_b = O.lora_weight_grads(c4["x64"], f32(c4["gy"]), f32(a), f32(b), scale)
    assert_close(f32(ga), want_a, what="soft grad_A (M=16384)")
    assert_close(f32(gb), want_b, what="soft grad_B (M=16384)")
