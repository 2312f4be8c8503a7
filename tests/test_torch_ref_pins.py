"""CPU pins of oracle/torch_ref.py, the torch restatement the layer-step parity tests and the
CPU baseline rely on. Each function is checked against something independent of its own
formula:

  * rmsnorm_ref, rope_ref, layer.rope_tables, the MLP and attention inside
    teacher_forward_ref / layer_forward_ref: HF transformers' Qwen3 modules
    (models/qwen3/modeling_qwen3.py: Qwen3RMSNorm, Qwen3RotaryEmbedding,
    apply_rotary_pos_emb, Qwen3DecoderLayer with eager attention), built from a local
    Qwen3Config with the same weights -- never from_pretrained;
  * compute_loss_ref: closed forms of train_qwen.py:229-249 on planted inputs (s = t,
    s = -t, s = c t, all-zero student rows) and torch's F.cosine_similarity eps semantics;
  * SoftLinearRef: the numpy oracle (oracle.soft_weights / soft_backward, themselves pinned by
    finite differences in test_oracle.py);
  * palettized_linear_cpu: the oracle's dequantiser and fp64 products.
"""
import numpy as np
import pytest
import torch

import oracle as O
import torch_ref as R
from helpers import assert_close, make_weight

hf = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
from transformers import Qwen3Config  # noqa: E402


class Cfg:
    hidden, heads, kv_heads, head_dim, intermediate = 256, 4, 2, 64, 512
    eps, rope_theta = 1e-6, 1e6


def _hf_config(cfg=Cfg):
    c = Qwen3Config(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                    num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
                    head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, hidden_act="silu",
                    attention_bias=False, max_position_embeddings=4096,
                    rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta})
    c._attn_implementation = "eager"
    return c


def _bf(t):
    return t.to(torch.bfloat16).float()


def _causal_mask(S):
    m = torch.full((S, S), float("-inf")).triu(1)
    return m[None, None]


def test_rmsnorm_ref_is_hf_qwen3_rmsnorm_bit_for_bit():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(3, 17, 256, generator=g) * 4).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(256, generator=g)).to(torch.bfloat16)
    norm = hf.Qwen3RMSNorm(256, eps=1e-6).to(torch.bfloat16)  # a bf16 model's norm
    with torch.no_grad():
        norm.weight.copy_(w)
    want = norm(x)  # bf16 in, bf16 weight: HF rounds the normalised value, then the product
    got = R.rmsnorm_ref(x.float(), w.float(), 1e-6)
    assert torch.equal(got, want.float())


@pytest.mark.parametrize("S,D", [(37, 64), (512, 128)])
def test_rope_ref_and_layer_tables_are_hf_rotary_bit_for_bit(S, D):
    from palettize_hip import layer
    cfg = type("C", (Cfg,), {"head_dim": D})
    rot = hf.Qwen3RotaryEmbedding(_hf_config(cfg))
    pos = torch.arange(S)[None]
    g = torch.Generator().manual_seed(S)
    x = _bf(torch.randn(2, S, 3, D, generator=g) * 2)          # [B, S, H, D]
    cos, sin = rot(x, pos)                                     # fp32 [1, S, D]
    c_tab, s_tab = layer.rope_tables(S, D, Cfg.rope_theta, "cpu")
    assert torch.equal(c_tab, cos[0]) and torch.equal(s_tab, sin[0])
    q_hf, _ = hf.apply_rotary_pos_emb(x.transpose(1, 2), x.transpose(1, 2), cos, sin)
    assert torch.equal(R.rope_ref(x, S, Cfg.rope_theta), _bf(q_hf.transpose(1, 2)))


def _teacher_weights(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    h, hd = cfg.hidden, cfg.head_dim
    dims = {"q_proj": (cfg.heads * hd, h), "k_proj": (cfg.kv_heads * hd, h),
            "v_proj": (cfg.kv_heads * hd, h), "o_proj": (h, cfg.heads * hd),
            "gate_proj": (cfg.intermediate, h), "up_proj": (cfg.intermediate, h),
            "down_proj": (h, cfg.intermediate)}
    w = {n: _bf(torch.randn(*s, generator=g) * 0.05) for n, s in dims.items()}
    for n, d in (("input_layernorm", h), ("post_attention_layernorm", h), ("q_norm", hd),
                 ("k_norm", hd)):
        w[n] = _bf(1 + 0.2 * torch.randn(d, generator=g))
    return w


def _hf_layer(w, cfg=Cfg):
    layer = hf.Qwen3DecoderLayer(_hf_config(cfg), layer_idx=0).float().eval()
    with torch.no_grad():
        at, mlp = layer.self_attn, layer.mlp
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(at, n).weight.copy_(w[n])
        for n in ("gate_proj", "up_proj", "down_proj"):
            getattr(mlp, n).weight.copy_(w[n])
        at.q_norm.weight.copy_(w["q_norm"])
        at.k_norm.weight.copy_(w["k_norm"])
        layer.input_layernorm.weight.copy_(w["input_layernorm"])
        layer.post_attention_layernorm.weight.copy_(w["post_attention_layernorm"])
    return layer


def _hf_forward(layer, hs, cfg=Cfg):
    S = hs.shape[1]
    rot = hf.Qwen3RotaryEmbedding(_hf_config(cfg))
    pe = rot(hs, torch.arange(S)[None])
    with torch.no_grad():
        return layer(hs, attention_mask=_causal_mask(S), position_embeddings=pe)


def test_teacher_forward_ref_is_hf_qwen3_decoder_layer():
    """The teacher restatement (bf16 rounding between ops) against HF's fp32 decoder layer with
    the same bf16 weights: only the intermediate roundings differ. A dropped residual, the
    q/k norms left out, a RoPE sign or the wrong kv-head mapping each move the output far
    outside this bar."""
    w = _teacher_weights(Cfg, 1)
    hs = _bf(torch.randn(2, 48, Cfg.hidden, generator=torch.Generator().manual_seed(2)))
    want = _hf_forward(_hf_layer(w), hs)
    got = R.teacher_forward_ref(w, hs, Cfg)
    assert_close(got.numpy(), want.numpy(), max_rel=2e-2, min_cos=0.99995, what="teacher layer")
    # residual-free part, the update the layer adds, at the same bar (so a residual does not
    # mask an error in the attention or MLP branch)
    assert_close((got - hs).numpy(), (want - hs).numpy(), max_rel=3e-2, min_cos=0.9999,
                 what="teacher update")


def test_layer_forward_ref_is_hf_layer_with_merged_weights():
    """The student restatement with one-hot logits (W_hard = the palette entry of each index,
    whatever the noise) and LoRA equals HF's decoder layer whose weights are W_hard + s B A."""
    cfg = Cfg
    g = torch.Generator().manual_seed(5)
    h, hd = cfg.hidden, cfg.head_dim
    shapes = {"q_proj": (cfg.heads * hd, h), "k_proj": (cfg.kv_heads * hd, h),
              "v_proj": (cfg.kv_heads * hd, h), "o_proj": (h, cfg.heads * hd),
              "gate_proj": (cfg.intermediate, h), "up_proj": (cfg.intermediate, h),
              "down_proj": (h, cfg.intermediate)}
    p, noises, merged = {}, {}, {}
    scale = 2.0
    for i, (name, (N, K)) in enumerate(shapes.items()):
        idx, pal = make_weight(N, K, seed=10 + i, std=0.05)
        logits = torch.where(torch.nn.functional.one_hot(idx.long(), 4).bool(),
                             torch.tensor(10.0), torch.tensor(-10.0))
        a = _bf(torch.randn(16, K, generator=g) * 0.02)
        b = _bf(torch.randn(N, 16, generator=g) * 0.02)
        p[name] = dict(palette=pal, logits=logits, lora_a=a, lora_b=b, lora_scale=scale)
        noises[name] = torch.from_numpy(O.gumbel_philox(N * K * 4, 20 + i).reshape(N, K, 4))
        W = torch.from_numpy(O.dequant(idx.numpy(), pal.numpy()))
        merged[name] = W + scale * b @ a
    norms = _teacher_weights(cfg, 3)
    for n in ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm"):
        p[n] = norms[n]
        merged[n] = norms[n]
    hs = _bf(torch.randn(2, 32, h, generator=g))
    got = R.layer_forward_ref(p, hs, noises, 1.0, cfg)
    want = _hf_forward(_hf_layer(merged), hs)
    assert_close(got.detach().numpy(), want.numpy(), max_rel=2e-2, min_cos=0.99995,
                 what="student layer")
    assert_close((got.detach() - hs).numpy(), (want - hs).numpy(), max_rel=3e-2, min_cos=0.9999,
                 what="student update")


def test_compute_loss_ref_closed_forms():
    """train_qwen.py:229-249 with weights 0.5 / 0.5: loss = 0.5 mean_rows(1 - cos) +
    0.5 mean((s - t)^2) / max(mean(t^2), 1e-6)."""
    g = torch.Generator().manual_seed(0)
    t = torch.randn(2, 5, 64, generator=g)
    assert float(R.compute_loss_ref(t.clone(), t)) == pytest.approx(0.0, abs=1e-6)
    # s = -t: cos = -1 -> l_cos = 2; (s - t)^2 = 4 t^2 -> l_mse = 4
    assert float(R.compute_loss_ref(-t, t)) == pytest.approx(0.5 * 2 + 0.5 * 4, rel=1e-6)
    # s = c t, c > 0: cos = 1; l_mse = (c - 1)^2
    assert float(R.compute_loss_ref(3 * t, t)) == pytest.approx(0.5 * 4, rel=1e-6)
    # all-zero student: cos = 0 per row (torch clamps |s| to eps), l_mse = 1
    assert float(R.compute_loss_ref(torch.zeros_like(t), t)) == pytest.approx(1.0, rel=1e-6)
    # a zero teacher: t_var clamps to 1e-6
    s = torch.full((1, 2, 4), 1e-3)
    loss = R.compute_loss_ref(s, torch.zeros_like(s))
    assert float(loss) == pytest.approx(0.5 * 1.0 + 0.5 * 1e-6 / 1e-6, rel=1e-5)
    # the eps clamps |s| and |t| separately: |s| = 2e-6, |t| = 200 gives cos = s.t / (1e-4 * 200)
    s = torch.full((1, 1, 4), 1e-6)
    t = torch.full((1, 1, 4), 100.0)
    l_cos = 2 * float(R.compute_loss_ref(s, t)) - float((s - t).pow(2).mean() / t.pow(2).mean())
    assert l_cos == pytest.approx(1 - 4e-4 / (1e-4 * 200), rel=1e-5)


@pytest.mark.parametrize("tau", [2.0, 0.5, 0.1])
def test_soft_linear_ref_matches_numpy_oracle(tau):
    g = torch.Generator().manual_seed(int(tau * 10))
    M, N, K = 24, 16, 512
    _, pal = make_weight(N, K, seed=3)
    logits = _bf(torch.randn(N, K, 4, generator=g))
    noise = torch.from_numpy(O.gumbel_philox(N * K * 4, 7).reshape(N, K, 4))
    x = _bf(torch.randn(M, K, generator=g)).requires_grad_(True)
    gy = _bf(torch.randn(M, N, generator=g))
    palr = pal.clone().requires_grad_(True)
    lg = logits.clone().requires_grad_(True)
    y = R.SoftLinearRef.apply(x, palr, lg, noise, tau)
    y.backward(gy)
    _, _, w_hard = O.soft_weights(logits.numpy(), noise.numpy(), pal.numpy(), tau)
    w_hard = O.bf16_to_f32(O.bf16_bits(w_hard.astype(np.float32)))
    assert_close(y.detach().numpy(), x.detach().numpy().astype(np.float64) @ w_hard.T, what="y")
    assert_close(x.grad.numpy(), gy.numpy().astype(np.float64) @ w_hard, what="grad_x")
    gl, gp = O.soft_backward(x.detach().numpy(), gy.numpy(), logits.numpy(), noise.numpy(),
                             pal.numpy(), tau)
    assert_close(lg.grad.numpy(), gl, max_rel=1e-4, min_cos=0.999999, what="grad_logits")
    assert_close(palr.grad.numpy(), gp, max_rel=1e-4, min_cos=0.999999, what="grad_palette")


def test_palettized_linear_cpu_matches_oracle():
    M, N, K, r = 33, 64, 512, 16
    idx, pal = make_weight(N, K, seed=8)
    g = torch.Generator().manual_seed(9)
    x = _bf(torch.randn(M, K, generator=g))
    a = _bf(torch.randn(r, K, generator=g) * 0.01)
    b = _bf(torch.randn(N, r, generator=g) * 0.01)
    bias = _bf(torch.randn(N, generator=g) * 0.1)
    # bf16 operands, as the baseline runs it: the palette is rounded to bf16 on the way in
    bf = torch.bfloat16
    y = R.palettized_linear_cpu(x.to(bf), pal, R.native_flat_idx(idx), bias.to(bf), a.to(bf),
                                b.to(bf), 2.0)
    W = O.dequant(idx.numpy(), pal.numpy())
    want = O.lut_linear_fwd(x.numpy(), W, bias.numpy()) + O.lora_forward(x.numpy(), a.numpy(),
                                                                       b.numpy(), 2.0)
    assert y.dtype == bf
    assert_close(y.float().numpy(), want, what="cpu path")
