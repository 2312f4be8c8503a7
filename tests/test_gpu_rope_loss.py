"""GPU parity of the layer-step kernels around the linears: RoPE forward/backward (bit-exact
against the torch expression of HF Qwen3's rotate_half embedding), the fused per-head norm +
RoPE (bit-exact against the two kernels it replaces) and the distillation loss of
train_qwen.py:229-249 (against torch autograd of the same expression in fp32 on the CPU)."""
import pytest
import torch

from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
layer = pytest.importorskip("palettize_hip.layer")
ops = pytest.importorskip("palettize_hip.ops")


def _rope_cpu(x, cos, sin):
    xf = x.float()
    d = xf.shape[-1] // 2
    rot = torch.cat([-xf[..., d:], xf[..., :d]], dim=-1)
    return (xf * cos[None, :, None, :] + rot * sin[None, :, None, :]).to(x.dtype)


@pytest.mark.parametrize("B,S,H,D", [(2, 37, 4, 128), (1, 512, 8, 64), (3, 16, 32, 128)])
def test_rope_bit_exact(dev, B, S, H, D):
    g = torch.Generator().manual_seed(B * S + H)
    x = (torch.randn(B, S, H, D, generator=g) * 3).to(torch.bfloat16)
    cos, sin = layer.rope_tables(S, D, 1e6, "cpu")
    y = ops.rope_fwd(x.to(dev), cos.to(dev), sin.to(dev)).cpu()
    assert torch.equal(y.view(torch.int16), _rope_cpu(x, cos, sin).view(torch.int16))
    # backward: torch autograd through the same expression
    xr = x.clone().requires_grad_(True)
    gy = (torch.randn(B, S, H, D, generator=g)).to(torch.bfloat16)
    _rope_cpu(xr, cos, sin).backward(gy)
    gx = ops.rope_bwd(gy.to(dev), cos.to(dev), sin.to(dev)).cpu()
    assert torch.equal(gx.view(torch.int16), xr.grad.view(torch.int16))
    # the autograd wrapper the layer uses
    xg = x.to(dev).requires_grad_(True)
    layer.apply_rope(xg, cos.to(dev), sin.to(dev)).backward(gy.to(dev))
    assert torch.equal(xg.grad.cpu().view(torch.int16), xr.grad.view(torch.int16))


@pytest.mark.parametrize("B,S,H", [(2, 37, 3), (1, 512, 32), (3, 16, 8)])
def test_head_norm_rope_is_norm_then_rope_bit_for_bit(dev, B, S, H):
    """The fused per-head RMSNorm + RoPE (plz_head_norm_rope_fwd / _bwd) against the two kernels
    it replaces (plz_rmsnorm_fwd then plz_rope_fwd; plz_rope_bwd then plz_rmsnorm_bwd), each
    pinned above and in test_gpu_misc: every output bit, with a non-unit norm weight and a row
    count that leaves a partial workgroup (B S H not a multiple of 16)."""
    D = 128
    g = torch.Generator().manual_seed(B * S * H)
    x = (torch.randn(B, S, H, D, generator=g) * 2).to(torch.bfloat16).to(dev)
    w = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev)
    gy = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).to(dev)
    cos, sin = layer.rope_tables(S, D, 1e6, dev)
    eps = 1e-6
    n, rstd = ops.rmsnorm_fwd(x.view(-1, D), w, eps)
    want = ops.rope_fwd(n.view(B, S, H, D), cos, sin)
    y, rstd2 = ops.head_norm_rope_fwd(x, w, cos, sin, eps)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    assert torch.equal(rstd2, rstd)
    gn = ops.rope_bwd(gy, cos, sin)
    want_gx, _ = ops.rmsnorm_bwd(x.view(-1, D), w, rstd, gn.view(-1, D))
    gx = ops.head_norm_rope_bwd(x, w, rstd2, cos, sin, gy)
    assert torch.equal(gx.view(-1, D).view(torch.int16), want_gx.view(torch.int16))
    # the layer's autograd path (frozen weight) against the unfused modules
    norm = layer.RMSNorm(D, eps, dev)
    norm.weight.data.copy_(w)
    xa, xb = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    layer.norm_rope(norm, xa, cos, sin).backward(gy)
    layer.apply_rope(norm(xb), cos, sin).backward(gy)
    assert torch.equal(xa.grad.view(torch.int16), xb.grad.view(torch.int16))


def _loss_cpu(s, t, w_cos=0.5, w_mse=0.5):
    sf, tf = s.float(), t.float()
    tot = w_cos + w_mse
    cos_per = torch.nn.functional.cosine_similarity(sf.flatten(0, 1), tf.flatten(0, 1), dim=-1,
                                                    eps=1e-4)
    l_cos = (1 - cos_per).mean()
    t_var = (tf * tf).mean().clamp(min=1e-6)
    l_mse = ((sf - tf) ** 2).mean() / t_var
    return (w_cos / tot) * l_cos + (w_mse / tot) * l_mse, l_cos


@pytest.mark.parametrize("B,S,Dm,w", [(2, 64, 256, (0.5, 0.5)), (4, 512, 2560, (0.5, 0.5)),
                                      (1, 100, 2560, (1.0, 3.0))])
def test_distill_loss_matches_torch(dev, B, S, Dm, w):
    g = torch.Generator().manual_seed(S + Dm)
    t = torch.randn(B, S, Dm, generator=g).to(torch.bfloat16)
    s = (t.float() + 0.3 * torch.randn(B, S, Dm, generator=g)).to(torch.bfloat16)
    sr = s.clone().requires_grad_(True)
    want, want_cos = _loss_cpu(sr, t, *w)
    want.backward()
    sg = s.to(dev).requires_grad_(True)
    loss, l_cos = layer.compute_loss(sg, t.to(dev), *w)
    lv, lc, wv, wc = (float(v.detach()) for v in (loss, l_cos, want, want_cos))
    assert abs(lv - wv) <= 1e-5 * abs(wv) + 1e-7
    assert abs(lc - wc) <= 1e-5 * abs(wc) + 1e-7
    (2.0 * loss).backward()
    assert_close(f32(sg.grad.cpu()), 2.0 * f32(sr.grad), what="grad_student")


def test_distill_loss_identical_inputs(dev):
    # s == t: l_cos = 0, l_mse = 0, gradient 0
    t = torch.randn(2, 8, 128).to(torch.bfloat16).to(dev)
    s = t.clone().requires_grad_(True)
    loss, l_cos = layer.compute_loss(s, t)
    assert abs(float(loss.detach())) < 1e-6 and abs(float(l_cos.detach())) < 1e-6
    loss.backward()
    assert float(s.grad.float().abs().max()) < 1e-6


def test_distill_loss_near_zero_student_rows(dev):
    """Rows whose student norm is below the cosine eps (1e-4) -- the zero-initialised
    correction layer train_qwen.py:233 guards against -- and all-zero student rows: loss and
    gradient follow torch's F.cosine_similarity, which clamps |s| and |t| separately."""
    g = torch.Generator().manual_seed(11)
    B, S, D = 2, 24, 256
    t = torch.randn(B, S, D, generator=g).to(torch.bfloat16)
    s = (t.float() + 0.5 * torch.randn(B, S, D, generator=g))
    tiny = torch.zeros(B, S, dtype=torch.bool)
    tiny[0, 3:9] = True
    tiny[1, 17] = True
    s[tiny] = torch.randn(int(tiny.sum()), D, generator=g) * 1e-7
    zero = torch.zeros(B, S, dtype=torch.bool)
    zero[1, 0:4] = True
    s[zero] = 0.0
    s = s.to(torch.bfloat16)
    sr = s.clone().requires_grad_(True)
    want, want_cos = _loss_cpu(sr, t)
    want.backward()
    sg = s.to(dev).requires_grad_(True)
    loss, l_cos = layer.compute_loss(sg, t.to(dev))
    lv, lc, wv, wc = (float(v.detach()) for v in (loss, l_cos, want, want_cos))
    assert abs(lv - wv) <= 1e-5 * abs(wv)
    assert abs(lc - wc) <= 1e-5 * abs(wc)
    loss.backward()
    got = f32(sg.grad.cpu())
    ref = f32(sr.grad)
    normal = ~(tiny | zero)
    for mask, what in ((tiny, "tiny rows"), (zero, "zero rows"), (normal, "normal rows")):
        assert_close(got[mask.numpy()], ref[mask.numpy()], what=f"grad_student {what}")
