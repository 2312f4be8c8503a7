"""GPU parity of the reference's two soft samplers and its batched soft build, through the
C ABI and the drop-in module.

* plz_gumbel_lcg / plz_gumbel_lcg_triton against the reference's own Triton sampler outputs
  (tests/golden/lcg_triton_golden.npz, written from triton_soft_forward.py:51-66 by
  tests/golden/make_lcg_golden.py): every draw of the Triton variant, and the draws of the
  CUDA variant where the two reference samplers agree by construction. The GPU's logf and the
  golden's numpy log may differ by an ulp, so floats are compared at 2e-6; the discrete check
  below is bit-exact.
* A wrong bit anywhere in a hash changes its noise, and with it the argmax of the noisy
  softmax: the hard-noisy build from the GPU noise of each variant must equal the oracle's
  build from the oracle's noise bit for bit, except at near ties of (logit + noise) / tau.
* fused_lut_linear_soft(semantics="triton") against the oracle (forward: palette of the plain
  logits' argmax; backward from the Triton-variant noise of the module's own step counter).
* fused_compute_P_W_batched (fused_lut_linear_cuda.py:1016-1077): the reference's test pattern
  (test_batched_compute_pw.py:199-246: batched layer i == the single-layer build at seed
  step_seed ^ (i * 0x9E3779B9), group size 16) and the oracle (P within one fp16 ulp, W_soft
  within one bf16 ulp).
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
from palettize_hip import PLZ_W_HARD_NOISY  # noqa: E402
from palettize_hip import fused_lut_linear_cuda as FL  # noqa: E402
from palettize_hip.qwen_model import PalettizedLinear  # noqa: E402

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                    "lcg_triton_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def test_gumbel_lcg_variants_against_reference_golden(dev, gold):
    # a 32 x 32 grid draws idx (k*32 + n)*4 + c = 0..4095, the golden's first 4096 entries
    N = K = 32
    nk = O.lcg_index(N, K).ravel()
    for s in gold["seeds"]:
        s = int(s)
        want = gold[f"noise_{s}"][:4096]
        tri = f32(ops.gumbel_lcg(N, K, s, device=dev, variant="triton")).ravel()
        assert np.allclose(tri, want[nk], rtol=2e-6, atol=2e-6), f"triton variant, seed {s}"
        cud = f32(ops.gumbel_lcg(N, K, s, device=dev)).ravel()
        agree = O.lcg_variants_agree(s, nk)
        assert np.allclose(cud[agree], want[nk][agree], rtol=2e-6, atol=2e-6), f"cuda, seed {s}"
        assert np.allclose(cud, O.c_gumbel_lcg(s, N, K).ravel(), rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("variant", ["cuda", "triton"])
def test_gumbel_lcg_hard_build_is_bit_exact(dev, variant):
    N, K, seed, tau = 256, 1024, 0x5EED1234, 0.5
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(N, K, 4, generator=g).to(torch.bfloat16)
    pal = torch.sort(torch.randn(N, K // 256, 4, generator=g) * 0.02, dim=-1).values
    noise = ops.gumbel_lcg(N, K, seed, device=dev, variant=variant)
    w, _ = ops.soft_build_w(logits.to(dev), noise, pal.to(dev), tau, PLZ_W_HARD_NOISY)
    want_noise = O.lcg_gumbel(seed, N, K, variant).astype(np.float64)
    _, _, w_fwd = O.soft_weights(f32(logits), want_noise, pal.numpy(), tau, O.W_HARD_NOISY)
    got = w.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.bf16_bits(w_fwd.astype(np.float32))
    z = (f32(logits).astype(np.float64) + want_noise) / tau
    top2 = np.sort(z, axis=-1)[..., -2:]
    tie = top2[..., 1] - top2[..., 0] <= 1e-5 * (1.0 + np.abs(top2[..., 1]))
    bad = got != want
    assert not np.any(bad & ~tie), f"{int(np.sum(bad & ~tie))} hard weights differ"
    # the noise decides the pick on a large share of weights (a wrong hash would show)
    am_plain = np.argmax(f32(logits), axis=-1)
    am_noisy = np.argmax(z, axis=-1)
    assert np.mean(am_plain != am_noisy) > 0.3


def test_dropin_soft_triton_semantics(dev):
    M, K, N, GS, tau = 64, 512, 512, 256, 1.0
    g = torch.Generator().manual_seed(21)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    logits = (torch.randn(4, K, N, generator=g) * 1.5).to(torch.float16)
    pal = torch.sort(torch.randn(N // GS, 4, generator=g) * 0.02, dim=-1).values.to(torch.bfloat16)
    gy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    ld = logits.to(dev).requires_grad_(True)
    pd = pal.to(dev).requires_grad_(True)
    FL._TRITON_STEP_SEED = 40
    cuda_seed = FL._SOFT_STEP_SEED
    y = FL.fused_lut_linear_soft(xd, pd, ld, None, GS, tau, semantics="triton")
    assert FL._TRITON_STEP_SEED == 41 and FL._SOFT_STEP_SEED == cuda_seed
    y.backward(gy.to(dev))
    nat_l = f32(logits).transpose(2, 1, 0)                       # [N, K, 4]
    nat_p = np.repeat(f32(pal), GS, axis=0)[:, None, :].repeat(K // 256, axis=1)
    noise = O.lcg_gumbel(41, N, K, "triton").astype(np.float64)
    _, _, w_ste = O.soft_weights(nat_l, noise, nat_p, tau, O.W_HARD_PLAIN)
    w_ste = O.bf16_round(w_ste.astype(np.float32))
    assert_close(f32(y), f32(x).astype(np.float64) @ w_ste.T, what="triton-semantics y")
    gl, gp = O.soft_backward(f32(x), f32(gy), nat_l, noise, nat_p, tau)
    assert_close(f32(ld.grad).transpose(2, 1, 0), gl, what="triton-semantics grad_logits")
    gp_ref = gp.sum(axis=1).reshape(N // GS, GS, 4).sum(axis=1)
    assert_close(f32(pd.grad), gp_ref, what="triton-semantics grad_palette")
    assert_close(f32(xd.grad), f32(gy).astype(np.float64) @ w_ste, what="triton-semantics grad_x")


def test_palettized_linear_soft_semantics_flags(dev):
    lin = torch.nn.Linear(256, 256, bias=False)
    idx = torch.randint(0, 4, (256, 256), generator=torch.Generator().manual_seed(3)).to(dev)
    a = PalettizedLinear(lin, idx, 1, 4, 256, False, use_soft_indices=True)
    b = PalettizedLinear(lin, idx, 1, 4, 256, False, use_soft_indices=True,
                         soft_semantics="triton")
    assert (a._use_cuda, a._use_triton) == (True, False)
    assert (b._use_cuda, b._use_triton) == (False, True)
    with pytest.raises(ValueError):
        PalettizedLinear(lin, idx, 1, 4, 256, False, soft_semantics="cutlass")


def _pw_oracle(logits, pal_bits, gs, tau, seed):
    """(P [K, N, 4], W_soft [K, N]) of the reference's batched kernel from the oracle."""
    lg = logits.astype(np.float32)                                # (4, K, N)
    _, K, N = lg.shape
    nat_l = lg.transpose(2, 1, 0)                                 # [N, K, 4]
    per_row = np.repeat(O.bf16_to_f32(pal_bits), gs, axis=0)[:N]  # [N, 4]
    nat_p = np.repeat(per_row[:, None, :], max(1, -(-K // 256)), axis=1)
    noise = O.lcg_gumbel(seed, N, K, "cuda").astype(np.float64)
    P, w_soft, _ = O.soft_weights(nat_l, noise, nat_p, tau, O.W_SOFT)
    return P.transpose(1, 0, 2), w_soft.T


def test_fused_compute_P_W_batched_reference_pattern(dev):
    """test_batched_compute_pw.py:199-246 on this build: shapes (K, N) (32, 64), (16, 32),
    (48, 64), group size 16, tau 0.5, step seed 12345."""
    mod = FL._get_module()
    torch.manual_seed(0)
    shapes, GS, tau, seed = [(32, 64), (16, 32), (48, 64)], 16, 0.5, 12345
    logits_list = [torch.randn(4, K, N, dtype=torch.float16, device=dev) for K, N in shapes]
    palette_list = [torch.randn(N // GS, 4, dtype=torch.bfloat16, device=dev) for _, N in shapes]
    flat = mod.fused_compute_P_W_batched(logits_list, palette_list, GS, tau, seed)
    assert len(flat) == 6
    for i, ((K, N), lg, pl) in enumerate(zip(shapes, logits_list, palette_list)):
        layer_seed = (seed ^ (i * 0x9E3779B9)) & 0xFFFFFFFF
        x_dummy = torch.zeros(1, K, dtype=torch.bfloat16, device=dev)
        P1, W1 = mod.fused_lut_linear_soft_fwd_aos(x_dummy, pl, lg, GS, tau, layer_seed)
        P, W = flat[2 * i], flat[2 * i + 1]
        assert P.shape == (K, N, 4) and W.shape == (K, N)
        assert torch.equal(P, P1) and torch.equal(W, W1), f"layer {i}"
        Pr, Wr = _pw_oracle(lg.cpu().numpy(), pl.view(torch.int16).cpu().numpy().view(np.uint16),
                            GS, tau, layer_seed)
        Pg = P.float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(Pg - Pr) <= np.maximum(np.abs(Pr) * 2.0 ** -10, 2.0 ** -24)), i
        Wg = W.float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(Wg - Wr) <= np.abs(Wr) * 2.0 ** -7 + 1e-6 * np.abs(Wr).max()), i
    with pytest.raises(ValueError, match="G mismatch"):
        mod.fused_compute_P_W_batched(logits_list[:1], [palette_list[1]], GS, tau, seed)


def test_fused_compute_P_W_batched_on_student(dev):
    """Walks a module for soft PalettizedLinears (skipping hard ones and non-palettized
    modules), at Qwen-like shapes, odd group sizes rejected."""
    g = torch.Generator().manual_seed(5)

    def pl(K, N, soft=True):
        lin = torch.nn.Linear(K, N, bias=False)
        idx = torch.randint(0, 4, (K, N), generator=g)
        pal = torch.sort(torch.randn(N // 256, 4, generator=g) * 0.02, -1).values
        m = PalettizedLinear(lin, idx, N // 256, 4, 256, False, initial_palette=pal,
                             use_soft_indices=soft).to(dev)
        if soft:  # logits off the one-hot init, so the noise matters
            with torch.no_grad():
                m.index_logits.copy_((torch.randn(4, K, N, generator=g) * 1.5).half())
        return m

    student = torch.nn.Module()
    student.q = pl(2560, 1024)
    student.frozen = pl(256, 512, soft=False)
    student.other = torch.nn.Linear(8, 8)
    student.down = pl(1024, 2560)
    out = FL.fused_compute_P_W_batched(student, 0.5, 777)
    assert len(out) == 2
    for i, m in enumerate((student.q, student.down)):
        P, W = out[i]
        K, N = m.index_logits.shape[1:]
        assert P.shape == (K, N, 4) and P.dtype == torch.float16 and W.dtype == torch.bfloat16
        seed = (777 ^ (i * 0x9E3779B9)) & 0xFFFFFFFF
        # the oracle on the first 64 input rows k (all N): a cut of whole rows keeps every
        # element's draw index (k*N + n)*4 + c
        rows = slice(0, 64)
        Pr, Wr = _pw_oracle(m.index_logits.detach()[:, rows].cpu().numpy(),
                            m.palette.detach().view(torch.int16).cpu().numpy().view(np.uint16),
                            256, 0.5, seed)
        Pg = P[rows].float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(Pg - Pr) <= np.maximum(np.abs(Pr) * 2.0 ** -10, 2.0 ** -24)), i
        Wg = W[rows].float().cpu().numpy().astype(np.float64)
        assert np.all(np.abs(Wg - Wr) <= np.abs(Wr) * 2.0 ** -7 + 1e-6 * np.abs(Wr).max()), i
    assert FL.fused_compute_P_W_batched(torch.nn.Linear(4, 4), 1.0, 1) == []
    student.down.group_size = 128
    with pytest.raises(ValueError, match="must share group_size"):
        FL.fused_compute_P_W_batched(student, 0.5, 777)
