"""GPU parity at BASELINE.json config 3: hard forward, grad_x and grad_palette at M = 16384 on all
seven Qwen-4B linear shapes, LoRA rank 16 (32 on o and down), through the C ABI.

These are the launch geometries the benchmark times: 640- and 2432-tile launches whose last
partial wave is split over the reduction, the split-M grad_palette GEMM (up to 32 ways) and
down's 38 palette groups along K. The forward and grad_x run both of their schedules:
staged (W dequantised into the workspace, then the dense GEMM: what the query's workspace
selects at this M) and the one-pass LUT GEMMs (a workspace for the tail partials only). Outputs are checked on sampled rows against the fp64 oracle
(rows of y and grad_x; output rows n of grad_palette, which need only gy[:, n]^T x), at the
north-star bar (max-rel-err 1e-2, cosine 0.9999); grad_palette must also be bit-repeatable.
Inputs are drawn on the GPU from a seeded generator and copied to the host for the oracle.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")

M = 16384
# (name, K, N, LoRA rank) as in BASELINE.json config 3
SHAPES = [("q", 2560, 4096, 16), ("k", 2560, 1024, 16), ("v", 2560, 1024, 16),
          ("o", 4096, 2560, 32), ("gate", 2560, 9728, 16), ("up", 2560, 9728, 16),
          ("down", 9728, 2560, 32)]


def _rows(n_total, extra_seed):
    """First, last and tile-boundary rows plus a few seeded random ones (sorted, unique)."""
    fixed = [0, 1, 127, 128, 255, 256, 257, n_total // 2 + 3, n_total - 1800, n_total - 600,
             n_total - 257, n_total - 256, n_total - 129, n_total - 1]
    rnd = np.random.default_rng(extra_seed).integers(0, n_total, 6).tolist()
    return sorted({r for r in fixed + rnd if 0 <= r < n_total})


@pytest.fixture(scope="module")
def problems(dev):
    out = {}
    for i, (name, K, N, r) in enumerate(SHAPES):
        g = torch.Generator(device=dev).manual_seed(100 + i)
        idx = torch.randint(0, 4, (N, K), generator=g, device=dev, dtype=torch.uint8)
        pal = torch.sort(torch.randn(N, K // 256, 4, generator=g, device=dev) * 0.02,
                         dim=-1).values.contiguous()
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        gy = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
        a = (torch.randn(r, K, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        b = (torch.randn(N, r, generator=g, device=dev) * 0.01).to(torch.bfloat16)
        out[name] = dict(K=K, N=N, r=r, idx=idx, pal=pal, x=x, gy=gy, a=a, b=b,
                         packed=ops.pack_indices(idx))
    return out


@pytest.mark.parametrize("staged", [True, False])
@pytest.mark.parametrize("name", [s[0] for s in SHAPES])
def test_config3_forward(dev, problems, name, staged):
    p = problems[name]
    rows = torch.tensor(_rows(M, 1), device=dev)
    t = ops.lora_project(p["x"], p["a"], 1.0)
    y = ops.lut_linear_fwd(p["x"], p["packed"], p["pal"], None, t, p["b"], staged=staged)
    W = O.dequant(p["idx"].cpu().numpy(), p["pal"].cpu().numpy())
    xr = f32(p["x"][rows])
    want = O.lut_linear_fwd(xr, W) + O.lora_forward(xr, f32(p["a"]), f32(p["b"]), 1.0)
    assert_close(f32(y[rows]), want, what=f"{name} y (M={M}, staged={staged})")


@pytest.mark.parametrize("staged", [True, False])
@pytest.mark.parametrize("name", [s[0] for s in SHAPES])
def test_config3_grad_x(dev, problems, name, staged):
    p = problems[name]
    rows = torch.tensor(_rows(M, 2), device=dev)
    gt = ops.lora_grad_t(p["gy"], p["b"], 1.0)
    gx = ops.lut_linear_bwd_x(p["gy"], p["packed"], p["pal"], gt, p["a"], staged=staged)
    W = O.dequant(p["idx"].cpu().numpy(), p["pal"].cpu().numpy())
    gyr = f32(p["gy"][rows]).astype(np.float64)
    want = O.grad_x(gyr, W) + (gyr @ f32(p["b"]).astype(np.float64)) @ f32(p["a"])
    assert_close(f32(gx[rows]), want, what=f"{name} grad_x (M={M}, staged={staged})")


@pytest.mark.parametrize("name", [s[0] for s in SHAPES])
def test_config3_grad_palette(dev, problems, name):
    p = problems[name]
    g1 = ops.lut_linear_bwd_palette(p["x"], p["gy"], p["packed"])
    g2 = ops.lut_linear_bwd_palette(p["x"], p["gy"], p["packed"])
    assert torch.equal(g1, g2), f"{name}: grad_palette must be bit-repeatable"
    ns = torch.tensor(_rows(p["N"], 3), device=dev)
    x64 = f32(p["x"]).astype(np.float64)
    gyc = f32(p["gy"][:, ns]).astype(np.float64)
    want = O.grad_palette(x64, gyc, p["idx"][ns].cpu().numpy())
    assert_close(f32(g1[ns]), want, what=f"{name} grad_palette (M={M})")


@pytest.mark.parametrize("name", [s[0] for s in SHAPES])
def test_config3_grad_palette_lora(dev, problems, name):
    """The entry the benchmark times (plz_lut_linear_bwd_palette_lora): grad_palette bit-equal
    to the plain entry's, and grad_A [r, K] / grad_B [N, r] (rank 16; 32 on o and down) from
    the dW tiles of every split-M part, summed in fixed order, against the fp64 oracle over all
    M = 16384 rows at the north-star bar; bit-repeatable."""
    p = problems[name]
    scale = 2.0
    gp, ga, gb = ops.lut_linear_bwd_palette_lora(p["x"], p["gy"], p["packed"], p["a"], p["b"],
                                                 scale, out_dtype=torch.bfloat16)
    gp2, ga2, gb2 = ops.lut_linear_bwd_palette_lora(p["x"], p["gy"], p["packed"], p["a"], p["b"],
                                                    scale, out_dtype=torch.bfloat16)
    assert torch.equal(gp, gp2) and torch.equal(ga, ga2) and torch.equal(gb, gb2), \
        f"{name}: LoRA grad_palette entry must be bit-repeatable"
    assert torch.equal(gp, ops.lut_linear_bwd_palette(p["x"], p["gy"], p["packed"])), \
        f"{name}: palette output differs from plz_lut_linear_bwd_palette"
    want_a, want_b = O.lora_weight_grads(f32(p["x"]), f32(p["gy"]), f32(p["a"]), f32(p["b"]),
                                         scale)
    assert_close(f32(ga), want_a, what=f"{name} grad_A (M={M}, r={p['r']})")
    assert_close(f32(gb), want_b, what=f"{name} grad_B (M={M}, r={p['r']})")
