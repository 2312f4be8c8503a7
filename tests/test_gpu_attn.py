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
                                            (1, 128, 32, 8, 3.0)])
def test_attn_fwd_matches_fp32(dev, B, S, Hq, Hkv, std):
    q, k, v = _inputs(B, S, Hq, Hkv, seed=S + Hq, std=std)
    o, lse = ops.attn_fwd(q.to(dev), k.to(dev), v.to(dev))
    want_o, want_lse = _ref(q, k, v)
    assert_close(f32(o), want_o.numpy(), what="attention output")
    assert np.allclose(f32(lse), want_lse.numpy(), rtol=1e-4, atol=1e-4)
