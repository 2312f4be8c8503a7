"""GPU parity: packing, dequant, hard LUT-linear forward / backward, GEMV (through the C ABI)."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import gen, assert_close, f32, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")


def _packed(idx, dev):
    return ops.pack_indices(idx.to(dev))


@pytest.mark.parametrize("N,K", [(8, 256), (24, 512), (2560, 2560), (1032, 768)])
def test_pack_unpack_bit_exact(dev, N, K):
    idx, _ = make_weight(N, K, seed=N + K)
    p = _packed(idx, dev)
    assert np.array_equal(p.cpu().numpy(), O.pack_native(idx.numpy()))
    assert torch.equal(ops.unpack_indices(p).cpu(), idx)


@pytest.mark.parametrize("N,K", [(8, 256), (2560, 2560), (1032, 768), (4096, 2560)])
def test_dequant_bit_exact(dev, N, K):
    idx, pal = make_weight(N, K, seed=7 * N + K)
    w = ops.dequant(_packed(idx, dev), pal.to(dev))
    got = w.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, O.dequant_bits(idx.numpy(), pal.numpy()))


def test_dequant_rounds_fp32_palette_to_nearest_even(dev):
    # palette entries on, just below and just above bf16 rounding ties (even and odd bases)
    N, K = 8, 256
    idx = torch.arange(4, dtype=torch.uint8).repeat(N, K // 4)
    vals = []
    for n in range(N):
        b = (0x3C00 + 2 * n + (n % 2)) << 16
        vals += [b | 0x8000, b | 0x7FFF, b | 0x8001, (b + 0x10000) | 0x8000]
    pal = torch.from_numpy(np.array(vals, np.uint32).view(np.float32).reshape(N, 1, 4).copy())
    w = ops.dequant(_packed(idx, dev), pal.to(dev)).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(w, O.dequant_bits(idx.numpy(), pal.numpy()))


def test_dequant_rounding_special_values(dev):
    # fp32 denormals (rounding to bf16 denormals, up to the smallest normal, and ties),
    # negative ties, overflow to inf, +-inf, +-0, the largest finite values, and a
    # random sweep over all exponents; NaN must stay NaN
    special = [0x00000001, 0x00007FFF, 0x00008000, 0x00018000, 0x0000FFFF, 0x007FFFFF,
               0x007F8000, 0x80008000, 0x80018000, 0x807FFFFF, 0xBC018000, 0xBC028000,
               0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000,
               0x00000000, 0x80000000, 0x7F7EFFFF, 0x3F808000, 0x3F818000, 0x3F80FFFF]
    rnd = np.random.default_rng(5).integers(0, 2**32, size=4096 - len(special) - 4,
                                            dtype=np.uint64).astype(np.uint32)
    rnd = rnd[((rnd >> 23) & 0xFF) != 0xFF]  # finite only
    bits = np.concatenate([np.array(special, np.uint32), rnd,
                           np.zeros(4096 - len(special) - rnd.size - 4, np.uint32),
                           np.array([0x7FC00000, 0x7F800001, 0xFFC12345, 0x7FFFFFFF], np.uint32)])
    N, K = 64, 4096  # N * K/256 * 4 = 4096 palette entries, each selected by some weight
    pal = torch.from_numpy(bits.view(np.float32).reshape(N, K // 256, 4).copy())
    idx = torch.arange(4, dtype=torch.uint8).repeat(N, K // 4)
    w = ops.dequant(_packed(idx, dev), pal.to(dev)).view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.dequant_bits(idx.numpy(), pal.numpy())
    nan = np.isnan(O.bf16_to_f32(want))
    assert np.array_equal(w[~nan], want[~nan])
    assert np.all(np.isnan(O.bf16_to_f32(w[nan])))


def _oracle_problem(M, N, K, seed, rank=0):
    idx, pal = make_weight(N, K, seed=seed)
    x = randn_bf16(M, K, seed=seed + 1)
    W = O.dequant(idx.numpy(), pal.numpy())
    lora = None
    if rank:
        a = randn_bf16(rank, K, seed=seed + 2, std=0.01)
        b = randn_bf16(N, rank, seed=seed + 3, std=0.01)
        lora = (a, b)
    return idx, pal, x, W, lora


@pytest.mark.parametrize("M,N,K,rank", [
    (512, 2560, 2560, 16),   # config 1 shape
    (1, 256, 256, 0), (3, 1032, 768, 8), (129, 384, 512, 16), (300, 136, 1024, 32),
    (4097, 1032, 768, 8),
])
def test_lut_linear_fwd(dev, M, N, K, rank):
    """From 4096 rows the call dequantises W into its workspace and runs the dense GEMM."""
    idx, pal, x, W, lora = _oracle_problem(M, N, K, seed=M + N + K, rank=rank)
    bias = randn_bf16(N, seed=5, std=0.1) if M % 2 else None
    args = {}
    t_ref = None
    if rank:
        a, b = lora
        t = ops.lora_project(x.to(dev), a.to(dev), 1.0)
        t_ref = f32(a)  # oracle recomputes t from x
        assert_close(f32(t), O.bf16_round(f32(x) @ f32(a).T), what="lora t")
        args = dict(lora_t=t, lora_b=b.to(dev))
    y = ops.lut_linear_fwd(x.to(dev), _packed(idx, dev), pal.to(dev),
                           None if bias is None else bias.to(dev), **args)
    want = O.lut_linear_fwd(f32(x), W, None if bias is None else f32(bias))
    if rank:
        want = want + O.lora_forward(f32(x), t_ref, f32(lora[1]), 1.0)
    assert_close(f32(y), want, what="y")
    if M >= 4096:  # the one-pass LUT GEMM on the same problem
        y1 = ops.lut_linear_fwd(x.to(dev), _packed(idx, dev), pal.to(dev),
                                None if bias is None else bias.to(dev), staged=False, **args)
        assert_close(f32(y1), want, what="y (LUT GEMM)")


@pytest.mark.parametrize("M,N,K,rank", [(512, 2560, 2560, 16), (1, 256, 256, 0),
                                        (77, 1032, 768, 8), (256, 384, 1024, 32),
                                        (4096, 1032, 768, 8)])
def test_lut_linear_bwd_x(dev, M, N, K, rank):
    """From 4096 rows the call dequantises W into its workspace and runs the dense GEMM."""
    idx, pal, _, W, lora = _oracle_problem(M, N, K, seed=3 * M + N, rank=rank)
    gy = randn_bf16(M, N, seed=9)
    args = {}
    want = O.grad_x(f32(gy), W)
    if rank:
        a, b = lora
        gt = ops.lora_grad_t(gy.to(dev), b.to(dev), 2.0)
        assert_close(f32(gt), 2.0 * f32(gy) @ f32(b), what="lora gt")
        args = dict(lora_gt=gt, lora_a=a.to(dev))
        want = want + f32(gt) @ f32(a)
    gx = ops.lut_linear_bwd_x(gy.to(dev), _packed(idx, dev), pal.to(dev), **args)
    assert_close(f32(gx), want, what="grad_x")
    if M >= 4096:  # the one-pass LUT GEMM on the same problem
        g1 = ops.lut_linear_bwd_x(gy.to(dev), _packed(idx, dev), pal.to(dev), staged=False, **args)
        assert_close(f32(g1), want, what="grad_x (LUT GEMM)")


@pytest.mark.parametrize("M,N,K", [(512, 2560, 2560), (1, 256, 256), (77, 1032, 768),
                                   (2048, 128, 512), (64, 1024, 2560)])
def test_lut_linear_bwd_palette(dev, M, N, K):
    idx, pal, x, _, _ = _oracle_problem(M, N, K, seed=M * 5 + K)
    gy = randn_bf16(M, N, seed=11)
    g1 = ops.lut_linear_bwd_palette(x.to(dev), gy.to(dev), _packed(idx, dev))
    want = O.grad_palette(f32(x), f32(gy), idx.numpy())
    assert_close(f32(g1), want, max_rel=1e-3, min_cos=0.99999, what="grad_palette")
    g2 = ops.lut_linear_bwd_palette(x.to(dev), gy.to(dev), _packed(idx, dev))
    assert torch.equal(g1, g2), "grad_palette must be deterministic"


def test_bias_grad(dev):
    gy = randn_bf16(333, 136, seed=3)
    assert_close(f32(ops.bias_grad(gy.to(dev))), O.grad_bias(f32(gy)), max_rel=1e-5,
                 min_cos=0.999999)


def test_empty_inputs(dev):
    idx, pal = make_weight(16, 256, seed=1)
    p, pl = _packed(idx, dev), pal.to(dev)
    x = torch.empty(0, 256, dtype=torch.bfloat16, device=dev)
    assert ops.lut_linear_fwd(x, p, pl).shape == (0, 16)
    g = ops.lut_linear_bwd_palette(x, torch.empty(0, 16, dtype=torch.bfloat16, device=dev), p)
    assert torch.count_nonzero(g) == 0
    # empty reductions of the other kernels are zero-filled too (by a kernel, not a memset)
    e = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
    for dt in (torch.float32, torch.bfloat16):
        ga, gb = ops.lora_weight_grads(e(0, 256), e(0, 128), e(0, 16), e(0, 16), 2.0, dt)
        assert ga.shape == (16, 256) and gb.shape == (128, 16)
        assert torch.count_nonzero(ga) == 0 and torch.count_nonzero(gb) == 0
    _, gw = ops.rmsnorm_bwd(e(0, 320), torch.ones(320, dtype=torch.bfloat16, device=dev),
                            torch.empty(0, device=dev),
                            e(0, 320))
    assert gw.shape == (320,) and torch.count_nonzero(gw) == 0


# ---- decode GEMV ----------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("N,K", [(1024, 2560), (2560, 9728), (264, 512)])
def test_gemv(dev, M, N, K):
    idx, pal = make_weight(N, K, seed=M * 31 + N)
    x = randn_bf16(M, K, seed=M)
    y = ops.lut_gemv(x.to(dev), _packed(idx, dev), pal.to(dev))
    want = O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy()))
    assert_close(f32(y), want, what=f"gemv M={M}")


@pytest.mark.parametrize("M,N,K", [(5, 264, 256), (13, 8, 768), (9, 136, 1280), (16, 2560, 9728)])
def test_gemv_ragged(dev, M, N, K):
    """Token counts of every LDS x-slice size, K ending mid-stage, N not a multiple of the
    128-row work item."""
    idx, pal = make_weight(N, K, seed=M * 7 + K)
    x = randn_bf16(M, K, seed=M + 1)
    y = ops.lut_gemv(x.to(dev), _packed(idx, dev), pal.to(dev))
    want = O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy()))
    assert_close(f32(y), want, what=f"gemv M={M} N={N} K={K}")


def _single_gemv(x, p, pl, decode):
    if decode == "planes":
        return ops.lut_gemv_planes(x, ops.gemv_pack_planes(p), ops.gemv_pack_palettes(pl),
                                   p.shape[0])
    if decode:
        return ops.lut_gemv_decode(x, ops.gemv_pack_indices(p), ops.gemv_pack_palettes(pl),
                                   p.shape[0])
    return ops.lut_gemv(x, p, pl)


def _layout(decode):
    return "planes" if decode == "planes" else ("decode" if decode else "native")


@pytest.mark.parametrize("decode", [False, True, "planes"],
                         ids=["native", "decode-layout", "planes-layout"])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_grouped_many_linears(dev, M, decode):
    """A grouped launch over 3 x 7 Qwen-4B shapes plus empty linears: every output equals the
    single-linear launch on the same layout bit for bit, and sampled ones match the oracle."""
    shapes = [(4096, 2560), (1024, 2560), (1024, 2560), (2560, 4096), (9728, 2560),
              (9728, 2560), (2560, 9728)]
    items, idxs = [], []
    for layer in range(3):
        for i, (N, K) in enumerate(shapes):
            idx, pal = make_weight(N, K, seed=1000 + 7 * layer + i)
            x = randn_bf16(M, K, seed=2000 + 7 * layer + i)
            items.append((x.to(dev), _packed(idx, dev), pal.to(dev)))
            idxs.append((idx, pal, x))
        items.append((randn_bf16(M, 256, seed=7).to(dev), torch.zeros(0, 16, dtype=torch.int32, device=dev),
                      torch.zeros(0, 1, 4, device=dev)))
        idxs.append(None)
    grp = ops.GemvGroup(items, layout=_layout(decode))
    outs = grp.run()
    for j, ((x, p, pl), y) in enumerate(zip(items, outs)):
        if idxs[j] is None:
            assert y.shape[1] == 0
            continue
        assert torch.equal(y, _single_gemv(x, p, pl, decode)), f"linear {j}"
        if j % 5 == 0:
            idx, pal, xc = idxs[j]
            want = O.lut_linear_fwd(f32(xc), O.dequant(idx.numpy(), pal.numpy()))
            assert_close(f32(y), want, what=f"grouped gemv linear {j}")


def test_gemv_pack_palettes_layout(dev):
    """Decode palette layout: the bf16 lookup words [ceil(N/128)][K/256][128][lo, hi], rows past
    N zero, word for word as the oracle builds them."""
    N, K = 300, 768
    pal = torch.randn(N, K // 256, 4, generator=gen(3))
    got = ops.gemv_pack_palettes(pal.to(dev)).cpu().numpy().view(np.uint32)
    want = O.gemv_palette_luts(pal.numpy())
    assert got.size >= want.size and np.array_equal(got[:want.size], want)


@pytest.mark.parametrize("decode", [False, True, "planes"],
                         ids=["native", "decode-layout", "planes-layout"])
def test_gemv_grouped_matches_single(dev, decode):
    shapes = [(4096, 2560), (1024, 2560), (2560, 4096), (264, 512), (9728, 2560)]
    M = 4
    items, wants = [], []
    for i, (N, K) in enumerate(shapes):
        idx, pal = make_weight(N, K, seed=100 + i)
        x = randn_bf16(M, K, seed=200 + i)
        items.append((x.to(dev), _packed(idx, dev), pal.to(dev)))
        wants.append(O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy())))
    grp = ops.GemvGroup(items, layout=_layout(decode))
    outs = grp.run()
    for (x, p, pl), y, want in zip(items, outs, wants):
        assert_close(f32(y), want, what="grouped gemv")
        assert torch.equal(y, _single_gemv(x, p, pl, decode))


def test_gemv_pack_indices_layout(dev):
    """plz_gemv_pack_indices equals the oracle's decode layout word for word (ragged N: padded
    rows are zero)."""
    N, K = 300, 768
    idx, _ = make_weight(N, K, seed=4)
    got = ops.gemv_pack_indices(_packed(idx, dev)).cpu().numpy().view(np.uint32)
    want = O.gemv_decode_layout(idx.numpy())
    assert got.size >= want.size and np.array_equal(got[:want.size], want)


@pytest.mark.parametrize("layout", [True, "planes"], ids=["decode-layout", "planes-layout"])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 2560), (4, 1024, 2560), (16, 2560, 9728),
                                   (5, 264, 256), (13, 8, 768), (1, 136, 1280), (2, 256, 512),
                                   (7, 128, 256), (8, 384, 1024), (9, 256, 768), (15, 136, 512)])
def test_gemv_decode_layout(dev, M, N, K, layout):
    """The GEMV on the decode and planes layouts (indices and palettes) against the oracle,
    including token counts of every x-slice and A-operand size and N not a multiple of the
    128-row item."""
    idx, pal = make_weight(N, K, seed=M * 3 + N + K)
    x = randn_bf16(M, K, seed=M + 2)
    y = _single_gemv(x.to(dev), _packed(idx, dev), pal.to(dev), layout)
    want = O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy()))
    assert_close(f32(y), want, what=f"{_layout(layout)} gemv M={M} N={N} K={K}")


def test_gemv_pack_planes_layout(dev):
    """plz_gemv_pack_planes equals the oracle's planes layout word for word (ragged N: padded
    rows are zero)."""
    N, K = 300, 768
    idx, _ = make_weight(N, K, seed=5)
    got = ops.gemv_pack_planes(_packed(idx, dev)).cpu().numpy().view(np.uint32)
    want = O.gemv_planes_layout(idx.numpy())
    assert got.size >= want.size and np.array_equal(got[:want.size], want)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_planes_x_dynamic_range(dev, M):
    """x rows spanning many binades inside one 256-k group (an outlier 2^12 times the rest,
    tiny values, exact zeros, negative zero): the two e4m3 pieces under the group's scale keep
    the bit-plane GEMV at the parity bar against the fp64 oracle."""
    N, K = 256, 1024
    idx, pal = make_weight(N, K, seed=77)
    g = gen(78)
    x = torch.randn(M, K, generator=g)
    x[:, 5] = 4096.0
    x[:, 300:320] *= 1e-6
    x[:, 600:640] = 0.0
    x[:, 700] = -0.0
    x[0, 900] = -3000.0
    x = x.to(torch.bfloat16)
    y = _single_gemv(x.to(dev), _packed(idx, dev), pal.to(dev), "planes")
    want = O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy()))
    assert_close(f32(y), want, what=f"planes gemv dynamic range M={M}")


@pytest.mark.parametrize("M", [2048, 8192])
def test_tail_split_gemms(dev, M):
    """Launches whose last wave is partial split those tiles over the reduction (fp32 partials
    in a workspace, summed by a second kernel): M=2048 splits every tile 3 ways, M=8192 the
    last 64 of 320 tiles 4 ways. Sampled rows cover whole and split tiles; LoRA and bias ride
    on the first part."""
    N = K = 2560
    assert ops.query("plz_lut_linear_fwd_workspace", M, N, K) > 0
    assert ops.query("plz_lut_linear_bwd_x_workspace", M, N, K) > 0
    idx, pal, x, W, (a, b) = _oracle_problem(M, N, K, seed=M, rank=16)
    bias = randn_bf16(N, seed=3, std=0.1)
    gy = randn_bf16(M, N, seed=4)
    rows = torch.tensor([0, 1, 255, 777, M // 2 + 3, M - 1800, M - 257, M - 256, M - 1])
    p, pl = _packed(idx, dev), pal.to(dev)
    t = ops.lora_project(x.to(dev), a.to(dev), 1.0)
    y = ops.lut_linear_fwd(x.to(dev), p, pl, bias.to(dev), lora_t=t, lora_b=b.to(dev))
    xr = f32(x[rows])
    want = O.lut_linear_fwd(xr, W, f32(bias)) + O.lora_forward(xr, f32(a), f32(b), 1.0)
    assert_close(f32(y[rows.to(dev)]), want, what="fwd (tail split)")
    y1 = ops.lut_linear_fwd(x.to(dev), p, pl, bias.to(dev), lora_t=t, lora_b=b.to(dev),
                            staged=False)
    assert_close(f32(y1[rows.to(dev)]), want, what="fwd (LUT GEMM, tail split)")
    gt = ops.lora_grad_t(gy.to(dev), b.to(dev), 1.0)
    gx = ops.lut_linear_bwd_x(gy.to(dev), p, pl, lora_gt=gt, lora_a=a.to(dev))
    want = O.grad_x(f32(gy[rows]), W) + f32(gt[rows.to(dev)]) @ f32(a)
    assert_close(f32(gx[rows.to(dev)]), want, what="grad_x (tail split)")
    g1 = ops.lut_linear_bwd_x(gy.to(dev), p, pl, lora_gt=gt, lora_a=a.to(dev), staged=False)
    assert_close(f32(g1[rows.to(dev)]), want, what="grad_x (LUT GEMM, tail split)")
    # the dense GEMMs of the soft path on the dequantised weight
    wd = ops.dequant(p, pl)
    yd = ops.linear_fwd_dense(x.to(dev), wd, bias.to(dev))
    assert_close(f32(yd[rows.to(dev)]), O.lut_linear_fwd(xr, W, f32(bias)), what="dense fwd")
    gd = ops.linear_bwd_x_dense(gy.to(dev), wd)
    assert_close(f32(gd[rows.to(dev)]), O.grad_x(f32(gy[rows]), W), what="dense grad_x")
    # deterministic: the split sums its parts in a fixed order
    y2 = ops.lut_linear_fwd(x.to(dev), p, pl, bias.to(dev), lora_t=t, lora_b=b.to(dev))
    assert torch.equal(y, y2)


@pytest.mark.parametrize("M", [1, 8, 9])
def test_gemv_group_auto_layout(dev, M):
    """The default grouped layout: the bit-plane kernel up to 8 tokens, the decode kernel
    above; either way the oracle's outputs."""
    shapes = [(1024, 2560), (264, 512)]
    items, wants = [], []
    for i, (N, K) in enumerate(shapes):
        idx, pal = make_weight(N, K, seed=300 + i)
        x = randn_bf16(M, K, seed=400 + i)
        items.append((x.to(dev), _packed(idx, dev), pal.to(dev)))
        wants.append(O.lut_linear_fwd(f32(x), O.dequant(idx.numpy(), pal.numpy())))
    grp = ops.GemvGroup(items)
    assert grp.layout == (ops._lib.PLZ_GEMV_PLANES if M <= 8 else ops._lib.PLZ_GEMV_DECODE)
    for y, want in zip(grp.run(), wants):
        assert_close(f32(y), want, what=f"auto-layout gemv M={M}")
