"""GPU parity of the causal grouped-query attention kernels against fp32 attention on the CPU
(the math of torch scaled_dot_product_attention(is_causal=True) with repeated k/v heads)."""
import math

import numpy as np
import pytest
import torch

from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")


def _ref(q, k, v):
    B, S, Hq, D = q.shape
    G = Hq // k.shape[2]
    qf = q.float().transpose(1, 2)
    kf = k.float().repeat_interleave(G, dim=2).transpose(1, 2)
    vf = v.float().repeat_interleave(G, dim=2).transpose(1, 2)
    s = (qf @ kf.transpose(-1, -2)) / math.sqrt(D)
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    o = torch.softmax(s, dim=-1) @ vf
    return o.transpose(1, 2), lse


def _inputs(B, S, Hq, Hkv, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, S, Hq, 128, generator=g) * std).to(torch.bfloat16)
    k = (torch.randn(B, S, Hkv, 128, generator=g) * std).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, 128, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,S,Hq,Hkv,std", [(2, 256, 8, 2, 1.0), (1, 512, 4, 4, 1.0),
                                            (1, 128, 32, 8, 3.0), (1, 1024, 16, 2, 1.0)])
def test_attn_fwd_matches_fp32(dev, B, S, Hq, Hkv, std):
    q, k, v = _inputs(B, S, Hq, Hkv, seed=S + Hq, std=std)
    o, lse = ops.attn_fwd(q.to(dev), k.to(dev), v.to(dev))
    want_o, want_lse = _ref(q, k, v)
    assert_close(f32(o), want_o.numpy(), what="attention output")
    assert np.allclose(f32(lse), want_lse.numpy(), rtol=1e-4, atol=1e-4)


def _ref_grads(q, k, v, go):
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    o, _ = _ref(qf, kf, vf)
    o.backward(go.float())
    return qf.grad, kf.grad, vf.grad


@pytest.mark.parametrize("B,S,Hq,Hkv,std", [(2, 256, 8, 2, 1.0), (1, 512, 4, 4, 1.0),
                                            (1, 128, 32, 8, 3.0), (1, 384, 6, 1, 1.0),
                                            (1, 1024, 16, 2, 1.0)])
def test_attn_bwd_matches_fp32(dev, B, S, Hq, Hkv, std):
    """dQ, dK, dV (dK / dV summed over the query heads of each kv head) against fp32 autograd
    of the same attention; P and dS enter the products as bf16, as in the forward."""
    q, k, v = _inputs(B, S, Hq, Hkv, seed=7 * S + Hq, std=std)
    go = torch.randn(B, S, Hq, 128, generator=torch.Generator().manual_seed(S)).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o, lse = ops.attn_fwd(qd, kd, vd)
    gq, gk, gv = ops.attn_bwd(qd, kd, vd, o, lse, go.to(dev))
    want = _ref_grads(q, k, v, go)
    for got, ref, nm in zip((gq, gk, gv), want, ("grad_q", "grad_k", "grad_v")):
        assert got.shape == ref.shape
        assert_close(f32(got), ref.numpy(), what=nm)
    again = ops.attn_bwd(qd, kd, vd, o, lse, go.to(dev))
    assert all(torch.equal(a, b) for a, b in zip((gq, gk, gv), again)), "backward must be deterministic"


def test_attn_bwd_layer_shape_sampled_heads(dev):
    """The layer's shape (seq 512, 32 query / 8 kv heads, batch 2): every gradient finite, and
    kv head 5 with its four query heads matches fp32 autograd."""
    B, S, Hq, Hkv = 2, 512, 32, 8
    q, k, v = _inputs(B, S, Hq, Hkv, seed=99)
    go = torch.randn(B, S, Hq, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o, lse = ops.attn_fwd(qd, kd, vd)
    gq, gk, gv = ops.attn_bwd(qd, kd, vd, o, lse, go.to(dev))
    assert all(bool(torch.isfinite(t).all()) for t in (gq, gk, gv))
    hs = slice(20, 24)
    want = _ref_grads(q[:, :, hs].contiguous(), k[:, :, 5:6].contiguous(),
                      v[:, :, 5:6].contiguous(), go[:, :, hs].contiguous())
    for got, ref, nm in zip((gq[:, :, hs], gk[:, :, 5:6], gv[:, :, 5:6]), want,
                            ("grad_q", "grad_k", "grad_v")):
        assert_close(f32(got), ref.numpy(), what=nm + " (layer shape)")


@pytest.mark.parametrize("growth", [1.0, -1.0], ids=["rising-scores", "falling-scores"])
def test_attn_running_max_jumps(dev, growth):
    """Key norms that grow (or shrink) along the sequence make every later kv block move the
    running max by far more than the lazy-rescale threshold (2^8) or never move it: both
    branches of the online softmax, forward and backward, against fp32."""
    B, S, Hq, Hkv = 1, 512, 4, 2
    q, k, v = _inputs(B, S, Hq, Hkv, seed=11)
    ramp = torch.exp(growth * torch.linspace(-1.5, 1.5, S)).view(1, S, 1, 1)
    k = (k.float() * ramp).to(torch.bfloat16)
    go = torch.randn(B, S, Hq, 128, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o, lse = ops.attn_fwd(qd, kd, vd)
    want_o, want_lse = _ref(q, k, v)
    assert_close(f32(o), want_o.numpy(), what="attention output")
    assert np.allclose(f32(lse), want_lse.numpy(), rtol=1e-4, atol=1e-3)
    grads = ops.attn_bwd(qd, kd, vd, o, lse, go.to(dev))
    for got, ref, nm in zip(grads, _ref_grads(q, k, v, go), ("grad_q", "grad_k", "grad_v")):
        assert_close(f32(got), ref.numpy(), what=nm)
