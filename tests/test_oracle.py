"""Pins the CPU oracle (oracle/oracle.py, oracle/plz_oracle.c) before it is trusted.

Each oracle function is checked against something its own formula does not restate:
the reference's known-answer bytes, a second restatement in C or in Python integers,
published test vectors, finite differences, brute force on tiny inputs, closed forms,
torch library routines, or distribution moments.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O


# ---- packing: reference known answers (verify_2bit_format.py:50-109) ------------------
def test_pack_idx2_known_answers():
    assert O.pack_idx2([0, 1, 2, 3]) == bytes([0xE4])
    assert O.pack_idx2([3, 0, 1, 2]) == bytes([0x93])
    assert O.pack_idx2([1, 2, 3]) == bytes([0x39])  # padded last byte


def test_pack_idx2_matches_coreml_bit_packing():
    # Apple's pack_elements_into_bits as restated in verify_2bit_format.py:91-95
    def apple(elements, nbits):
        e = np.array(elements, dtype=np.uint8)
        bits = np.unpackbits(e.reshape(-1, 1), bitorder="little", axis=-1)[:, :nbits]
        return np.packbits(bits.flatten(), bitorder="little").tobytes()

    rng = np.random.default_rng(123)
    for n in (4, 100, 1000, 4096):
        v = rng.integers(0, 4, n, dtype=np.uint8)
        assert O.pack_idx2(v) == apple(v, 2)
    rt = O.unpack_idx2(O.pack_idx2(v), v.size)
    assert np.array_equal(rt, v)


def test_native_packing_is_idx2_bytes_and_c_agrees():
    rng = np.random.default_rng(0)
    idx = rng.integers(0, 4, (7, 512), dtype=np.uint8)
    p = O.pack_native(idx)
    for r in range(idx.shape[0]):
        assert p[r].tobytes() == O.pack_idx2(idx[r])
    # word 0 of a row holds k = 0..15 with k at bits 2k
    q = int(p[0, 0].view(np.uint32))
    assert [(q >> (2 * k)) & 3 for k in range(16)] == list(idx[0, :16])
    assert np.array_equal(O.c_pack(idx), p)
    assert np.array_equal(O.unpack_native(p), idx)
    assert np.array_equal(O.c_unpack(p), idx)


# ---- bf16 rounding vs torch's conversion ------------------------------------------------
def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    base = rng.standard_normal(20000).astype(np.float32) * np.float32(0.02)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 3.3895314e38, -3.4e38, 1e-40, -1e-40, 6e-39,
                         np.inf, -np.inf, 1.00390625, 1.01171875], np.float32)
    # exact ties: bf16 value + half an ulp, both parities
    ties = (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([base, specials, ties, -ties])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_bits(x), ref)
    L = O.clib()
    assert all(L.orc_f2bf(float(v)) == int(r) for v, r in zip(x[:3000], ref[:3000]))
    n = O.bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(O.bf16_to_f32(n)[0])


# ---- dequant: the flat gather -----------------------------------------------------------
def test_dequant_decodes_row_group_and_index():
    # palette entry (n, g, c) holds a distinct small integer -> exact in bf16; decoding the
    # dequantised value must recover (n, k // 256, idx[n, k]) for every weight.
    N, K = 6, 768
    G = K // 256
    rng = np.random.default_rng(2)
    idx = rng.integers(0, 4, (N, K), dtype=np.uint8)
    code = (np.arange(N)[:, None, None] * G + np.arange(G)[None, :, None]) * 4 + np.arange(4)
    pal = code.astype(np.float32)
    w = O.dequant(idx, pal).astype(np.int64)
    n_, g_, c_ = w // (4 * G), (w // 4) % G, w % 4
    assert np.array_equal(n_, np.repeat(np.arange(N)[:, None], K, 1))
    assert np.array_equal(g_, np.repeat((np.arange(K) // 256)[None, :], N, 0))
    assert np.array_equal(c_, idx)
    assert np.array_equal(O.c_dequant_bits(O.pack_native(idx), pal), O.dequant_bits(idx, pal))


def test_reference_layout_embeds_by_palette_expansion():
    # the reference's (K, N) gather with a palette per 256 output channels equals the native
    # dequant of the transposed indices with the expanded palette
    rng = np.random.default_rng(3)
    K, N, GS = 512, 512, 256
    idx_kn = rng.integers(0, 4, (K, N), dtype=np.uint8)
    pal_ref = np.sort(rng.normal(0, 0.02, (N // GS, 4)).astype(np.float32), axis=1)
    w_ref = O.reference_weight(idx_kn, pal_ref, GS)               # (K, N)
    w_nat = O.dequant(idx_kn.T, O.expand_reference_palette(pal_ref, N, K, GS))  # (N, K)
    assert np.array_equal(w_ref, w_nat.T)


# ---- hard linear ------------------------------------------------------------------------
def _tiny_problem(seed=4, M=3, N=8, K=512):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, 4, (N, K), dtype=np.uint8)
    pal = np.sort(rng.normal(0, 0.02, (N, K // 256, 4)), axis=-1).astype(np.float32)
    x = rng.standard_normal((M, K))
    gy = rng.standard_normal((M, N))
    return idx, pal, x, gy


def test_hard_forward_brute_force():
    idx, pal, x, _ = _tiny_problem()
    M, K = x.shape
    N = idx.shape[0]
    W = O.dequant(idx, pal)
    y = O.lut_linear_fwd(x, W)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += x[m, k] * float(O.bf16_round(pal[n, k // 256, idx[n, k]]))
            assert abs(s - y[m, n]) < 1e-9


def test_grad_palette_finite_difference():
    # L(pal) = sum(gy * (x W(pal)^T)) is linear in pal: the difference quotient is exact.
    idx, pal, x, gy = _tiny_problem(seed=5)
    pal64 = pal.astype(np.float64)
    N, G = idx.shape[0], pal.shape[1]

    def loss(p):
        W = np.asarray(p)[np.arange(N)[:, None], (np.arange(idx.shape[1]) // 256)[None, :], idx]
        return float((gy * (x @ W.T)).sum())

    g = O.grad_palette(x, gy, idx)
    h = 1e-3
    for n in range(N):
        for gg in range(G):
            for c in range(4):
                p1 = pal64.copy()
                p1[n, gg, c] += h
                fd = (loss(p1) - loss(pal64)) / h
                assert abs(fd - g[n, gg, c]) < 1e-8 * max(1.0, abs(fd))


def test_grad_palette_single_class_is_group_sum():
    idx, pal, x, gy = _tiny_problem(seed=6)
    idx[:] = 2
    g = O.grad_palette(x, gy, idx)
    dW = gy.T @ x
    assert np.allclose(g[:, :, 2], dW.reshape(dW.shape[0], -1, 256).sum(-1))
    assert np.all(g[:, :, [0, 1, 3]] == 0)


def test_grad_x_finite_difference():
    idx, pal, x, gy = _tiny_problem(seed=7)
    W = O.dequant(idx, pal).astype(np.float64)
    g = O.grad_x(gy, W)
    h = 1e-4
    for (m, k) in [(0, 0), (1, 300), (2, 511)]:
        x1 = x.copy()
        x1[m, k] += h
        fd = ((gy * (x1 @ W.T)).sum() - (gy * (x @ W.T)).sum()) / h
        assert abs(fd - g[m, k]) < 1e-7


# ---- Gumbel noise -------------------------------------------------------------------------
def test_lcg_hash_three_restatements():
    seed = 0x12345677
    idx = np.array([0, 1, 2, 3, 1000, 2**31 - 1, 2**32 - 4, 0xDEADBEEF], dtype=np.uint32)

    def py(seed, i):  # Python integers, explicit mod 2^32
        m = 0xFFFFFFFF
        x = (seed ^ ((i * 0x9E3779B9) & m)) & m
        x ^= x >> 13
        x = (x * 1103515245 + 12345) & m
        x ^= x >> 17
        x = (x * 1103515245 + 12345) & m
        return x & 0xFFFFFF

    want = np.array([py(seed, int(i)) for i in idx], np.uint32)
    assert np.array_equal(O.lcg_bits(seed, idx), want)
    assert np.array_equal(O.c_lcg_bits(seed, idx), want)
    a = O.lcg_gumbel(7, 3, 40)
    b = O.c_gumbel_lcg(7, 3, 40)
    assert np.allclose(a, b, rtol=1e-6, atol=1e-6)


def test_gumbel_moments():
    # Gumbel(0, 1): mean = Euler-Mascheroni, variance = pi^2 / 6
    for noise in (O.lcg_gumbel(3, 64, 1024).ravel(), O.gumbel_philox(262144, seed=11)):
        assert abs(noise.mean() - 0.5772157) < 0.01
        assert abs(noise.var() - math.pi ** 2 / 6) < 0.03


def test_gumbel_from_bits_is_finite_at_the_extremes():
    # the largest and smallest 32-bit draws must map strictly inside (0, 1): no inf noise
    g = O.gumbel_from_bits(np.array([0, 1, 0x1FF, 0xFFFFFE00, 0xFFFFFFFF], np.uint32))
    assert np.all(np.isfinite(g))
    assert g[-1] > 15.0 and g[0] < -2.5


def test_philox_random123_known_answers():
    kat = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in kat:
        assert tuple(int(v) for v in O.philox4x32_10(np.array([ctr], np.uint32), key)[0]) == want
        assert tuple(int(v) for v in O.c_philox(np.array(ctr, np.uint32), np.array(key, np.uint32))) == want
    a = O.gumbel_philox(4096, seed=(5 << 32) | 9, offset=77)
    b = O.c_gumbel_philox(4096, seed=(5 << 32) | 9, offset=77)
    assert np.allclose(a, b, rtol=1e-6, atol=1e-6)


# ---- soft path ------------------------------------------------------------------------------
def _soft_problem(seed=8, N=4, K=256, tau=0.7):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((N, K, 4))
    noise = O.lcg_gumbel(seed, N, K).astype(np.float64)
    pal = np.sort(rng.normal(0, 0.02, (N, K // 256, 4)), axis=-1)
    return logits, noise, pal, tau


def test_soft_forward_closed_forms():
    logits, noise, pal, tau = _soft_problem()
    P, ws, wh = O.soft_weights(logits, noise, pal, tau, O.W_HARD_NOISY)
    assert np.allclose(P.sum(-1), 1.0)
    lo, hi = pal.min(-1)[:, :, None], pal.max(-1)[:, :, None]
    N, K = ws.shape
    assert np.all(ws >= np.repeat(lo, 256, 1)[:, :K, 0] - 1e-12)
    assert np.all(ws <= np.repeat(hi, 256, 1)[:, :K, 0] + 1e-12)
    # equal logits + noise -> uniform P whatever tau
    P1, _, _ = O.soft_weights(np.zeros_like(logits), np.zeros_like(noise), pal, 5.0)
    assert np.allclose(P1, 0.25)
    # equal palette entries -> W_soft = c
    palc = np.full_like(pal, 0.0125)
    _, ws_c, wh_c = O.soft_weights(logits, noise, palc, tau)
    assert np.allclose(ws_c, 0.0125) and np.allclose(wh_c, 0.0125)
    # saturated one-hot logits (+-10) at tau = 0.1 -> W_soft == W_hard == pal[onehot]
    onehot = np.random.default_rng(9).integers(0, 4, (N, K))
    l10 = np.where(np.arange(4)[None, None, :] == onehot[..., None], 10.0, -10.0)
    _, ws_s, wh_s = O.soft_weights(l10, noise, pal, 0.1, O.W_HARD_PLAIN)
    want = np.take_along_axis(np.repeat(pal, 256, 1)[:, :K], onehot[..., None], -1)[..., 0]
    assert np.allclose(wh_s, want) and np.allclose(ws_s, want, atol=1e-12)


def test_soft_argmax_first_max_wins():
    pal = np.arange(4, dtype=np.float64).reshape(1, 1, 4) * np.ones((1, 1, 4))
    logits = np.zeros((1, 256, 4))
    logits[0, 0] = [1.0, 3.0, 3.0, 0.0]   # tie between 1 and 2 -> 1
    logits[0, 1] = [2.0, 2.0, 2.0, 2.0]   # all equal -> 0
    _, _, wh = O.soft_weights(logits, np.zeros_like(logits), pal, 1.0, O.W_HARD_PLAIN)
    assert wh[0, 0] == 1.0 and wh[0, 1] == 0.0


def test_soft_backward_finite_difference_and_reference_scale():
    # L(logits, pal) = sum dW * W_soft: the true gradient wrt logits carries 1/tau; the
    # reference's formula omits it (fused_lut_kernel.cu:1914-1917).
    logits, noise, pal, tau = _soft_problem(seed=10, N=2, K=256, tau=0.5)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 256))
    gy = rng.standard_normal((3, 2))
    dW = gy.T @ x

    def loss(lg, p):
        _, ws, _ = O.soft_weights(lg, noise, p, tau, O.W_SOFT)
        return float((dW * ws).sum())

    gl_true, gp = O.soft_backward(x, gy, logits, noise, pal, tau, scale_by_inv_tau=True)
    gl_ref, gp_ref = O.soft_backward(x, gy, logits, noise, pal, tau)
    assert np.allclose(gl_ref * (1.0 / tau), gl_true) and np.allclose(gp, gp_ref)
    h = 1e-6
    for (n, k, c) in [(0, 0, 0), (1, 17, 3), (0, 255, 2), (1, 100, 1)]:
        l1 = logits.copy()
        l1[n, k, c] += h
        l0 = logits.copy()
        l0[n, k, c] -= h
        fd = (loss(l1, pal) - loss(l0, pal)) / (2 * h)
        assert abs(fd - gl_true[n, k, c]) < 1e-6 * max(1.0, abs(fd))
    for (n, c) in [(0, 0), (1, 3)]:
        p1 = pal.copy()
        p1[n, 0, c] += h
        fd = (loss(logits, p1) - loss(logits, pal)) / h
        assert abs(fd - gp[n, 0, c]) < 1e-5 * max(1.0, abs(fd))


def test_soft_backward_equal_palette_kills_logit_grad():
    logits, noise, pal, tau = _soft_problem(seed=12, N=2, K=256)
    x = np.random.default_rng(1).standard_normal((3, 256))
    gy = np.random.default_rng(2).standard_normal((3, 2))
    gl, _ = O.soft_backward(x, gy, logits, noise, np.full_like(pal, 0.3), tau)
    assert np.allclose(gl, 0.0, atol=1e-12)


# ---- LoRA, RMSNorm, SwiGLU vs torch library routines -------------------------------------
def test_lora_forward_and_grads_vs_torch_autograd():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 64, dtype=torch.float64, generator=g)
    A = torch.randn(16, 64, dtype=torch.float64, generator=g, requires_grad=True)
    B = torch.randn(32, 16, dtype=torch.float64, generator=g, requires_grad=True)
    y = 2.0 * (x @ A.T) @ B.T
    assert np.allclose(O.lora_forward(x.numpy(), A.detach().numpy(), B.detach().numpy(), 2.0),
                       y.detach().numpy())
    gy = torch.randn(5, 32, dtype=torch.float64, generator=g)
    y.backward(gy)
    ga, gb = O.lora_weight_grads(x.numpy(), gy.numpy(), A.detach().numpy(), B.detach().numpy(),
                                 2.0)
    assert np.allclose(ga, A.grad.numpy()) and np.allclose(gb, B.grad.numpy())


def test_rmsnorm_matches_hf_formula():
    torch.manual_seed(0)
    x = torch.randn(16, 256).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(256)).to(torch.bfloat16)
    eps = 1e-6
    # HF Qwen3RMSNorm.forward (modeling_qwen3.py:57-64), written with torch ops
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    y_hf = w * h.to(torch.bfloat16)
    y, r = O.rmsnorm_fwd(O.bf16_to_f32(x.view(torch.int16).numpy().view(np.uint16)),
                         O.bf16_to_f32(w.view(torch.int16).numpy().view(np.uint16)), eps)
    diff = np.abs(y - y_hf.float().numpy())
    ulp = np.abs(y_hf.float().numpy()) * 2.0 ** -7 + 1e-30
    assert np.all(diff <= ulp) and np.mean(diff == 0) > 0.99
    # backward vs autograd in fp64
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    gy = torch.randn(16, 256, dtype=torch.float64)
    hd = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    (wd * hd).backward(gy)
    gx, gw = O.rmsnorm_bwd(x.double().numpy(), w.double().numpy(), gy.numpy(), eps)
    assert np.allclose(gx, xd.grad.numpy(), rtol=1e-9, atol=1e-12)
    # HF multiplies w by h.to(bf16): dL/dw = sum_rows gy * bf16(h)
    gw_hf = (gy * h.to(torch.bfloat16).double()).sum(0)
    assert np.allclose(gw, gw_hf.numpy(), rtol=1e-6, atol=1e-6)


def test_swiglu_matches_torch():
    torch.manual_seed(1)
    g = (3 * torch.randn(4096)).to(torch.bfloat16)
    u = torch.randn(4096).to(torch.bfloat16)
    h_t = torch.nn.functional.silu(g) * u
    h = O.swiglu_fwd(g.float().numpy(), u.float().numpy())
    diff = np.abs(h - h_t.float().numpy())
    assert np.all(diff <= np.abs(h_t.float().numpy()) * 2.0 ** -7) and np.mean(diff == 0) > 0.99
    gd = g.double().requires_grad_(True)
    ud = u.double().requires_grad_(True)
    gh = torch.randn(4096, dtype=torch.float64)
    (torch.nn.functional.silu(gd) * ud).backward(gh)
    og, ou = O.swiglu_bwd(g.double().numpy(), u.double().numpy(), gh.numpy())
    assert np.allclose(og, gd.grad.numpy(), rtol=1e-9) and np.allclose(ou, ud.grad.numpy())


# ---- layer optimizer: clip + AdamW + clamp vs torch ------------------------------------------
def test_adamw_step_matches_torch_clip_adamw_clamp():
    import torch
    rng = np.random.default_rng(11)
    shapes = [(7, 5), (300,), (2, 3, 4)]
    groups = [0, 1, 1]
    lrs = [1e-2, 1e-4, 3e-4]
    clamps = [(-0.05, 0.05), (-np.inf, np.inf), (-np.inf, np.inf)]
    masters = [rng.standard_normal(s) * 0.03 for s in shapes]
    tparams = [torch.tensor(m, dtype=torch.float64, requires_grad=True) for m in masters]
    opt = torch.optim.AdamW([{"params": [tparams[i]], "lr": lrs[i]} for i in range(3)],
                            betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0)
    ms = [np.zeros(s) for s in shapes]
    vs = [np.zeros(s) for s in shapes]
    for step in range(1, 4):
        grads = [rng.standard_normal(s) * (3.0 if step == 2 else 0.01) for s in shapes]
        for t, g in zip(tparams, grads):
            t.grad = torch.tensor(g)
        n0 = torch.nn.utils.clip_grad_norm_([tparams[0]], 1.0)
        n1 = torch.nn.utils.clip_grad_norm_(tparams[1:], 0.3)
        opt.step()
        with torch.no_grad():
            tparams[0].clamp_(-0.05, 0.05)
        norms = O.adamw_step(masters, grads, ms, vs, lrs, groups, (1.0, 0.3), clamps, step)
        assert np.isclose(norms[0], float(n0)) and np.isclose(norms[1], float(n1))
        for m, t in zip(masters, tparams):
            assert np.allclose(m, t.detach().numpy(), rtol=1e-10, atol=1e-12)


def test_gemv_decode_layout_through_the_dequantiser_slot_order():
    """Decode-layout words read through the GEMV dequantiser's field -> slot pairing (v_perm
    selectors 0x05010400 / 0x07030602 on the bytes of (w >> 2j) & 0x03030303: slot 2j <- field
    2j, 2j+1 <- field 8+2j, 8+2j <- field 16+2j, 9+2j <- field 24+2j) give back every row's
    indices in natural k order; padded rows past N are zero. A wrong field map, row or lane
    order fails here."""
    rng = np.random.default_rng(5)
    N, K = 200, 512
    idx = rng.integers(0, 4, (N, K))
    items, stages = (N + 127) // 128, K // 256
    words = O.gemv_decode_layout(idx)
    assert words.size == items * 128 * K // 16
    words = words.reshape(items, stages, 4, 2, 4, 16, 4)  # item, stage, w, b, q, r, t
    slot_field = [0] * 16
    for j in range(4):
        slot_field[2 * j], slot_field[2 * j + 1] = 2 * j, 8 + 2 * j
        slot_field[8 + 2 * j], slot_field[9 + 2 * j] = 16 + 2 * j, 24 + 2 * j
    dec = np.stack([(words >> np.uint32(f)) & 3 for f in slot_field], -1)
    back = dec.transpose(0, 2, 3, 5, 1, 4, 6, 7).reshape(items * 128, K)
    assert np.array_equal(back[:N], idx)
    assert not back[N:].any()


def test_gemv_palette_luts_reassemble_torch_bf16():
    """Byte c of the low word and byte c of the high word of each row's tables reassemble
    entry c as torch rounds it to bf16; padded rows are zero."""
    rng = np.random.default_rng(6)
    pal = (rng.standard_normal((130, 3, 4)) * 0.02).astype(np.float32)
    luts = O.gemv_palette_luts(pal).reshape(2, 3, 128, 2).transpose(0, 2, 1, 3).reshape(256, 3, 2)
    c = np.arange(4, dtype=np.uint32) * 8
    lo = (luts[..., 0:1] >> c) & 0xFF
    hi = (luts[..., 1:2] >> c) & 0xFF
    got = (lo | (hi << 8)).astype(np.uint16)
    want = torch.from_numpy(pal).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[:130], want)
    assert not got[130:].any()


def test_gemv_planes_layout_through_the_plane_masks():
    """Planes-layout words read the way the bit-plane GEMV reads them give back every row's
    indices in natural k order: with t = q >> 1, MFMA half 0 takes b0 = q & 0x11111111,
    b1 = q & 0x22222222, b0 b1 = q & t & 0x11111111 and half 1 b0 = q & 0x44444444,
    b1 = t & 0x44444444, b0 b1 = q & t & 0x44444444 from the lane's four words j = 0..3 as FP4
    nibbles e = 8j + i of k = 128 h + 32 g + e (the B operand's lane layout). Padded rows are
    zero. A wrong nibble, word, lane or row order fails here."""
    rng = np.random.default_rng(8)
    N, K = 200, 512
    idx = rng.integers(0, 4, (N, K))
    items, stages = (N + 127) // 128, K // 256
    words = O.gemv_planes_layout(idx)
    assert words.size == items * 128 * K // 16
    words = words.reshape(items, stages, 4, 2, 4, 16, 4)  # item, stage, w, b, g, r, j
    back = np.zeros((items, 4, 2, 16, stages, 256), np.int64)  # item, w, b, r, stage, k
    for h, (m0, m1, bit0, bit1) in enumerate(((0x11111111, 0x22222222, 0, 1),
                                               (0x44444444, 0x44444444, 2, 2))):
        for j in range(4):
            q = words[..., j]
            t = q >> np.uint32(1)
            p0 = q & np.uint32(m0)
            p1 = (t if h else q) & np.uint32(m1)
            p3 = q & t & np.uint32(m0)
            for i in range(8):
                b0 = (p0 >> np.uint32(4 * i + bit0)) & 1
                b1 = (p1 >> np.uint32(4 * i + bit1)) & 1
                assert np.array_equal((p3 >> np.uint32(4 * i + bit0)) & 1, b0 & b1)
                for g in range(4):  # nibble e = 8j + i of lane group g: k = 128h + 32g + e
                    back[:, :, :, :, :, 128 * h + 32 * g + 8 * j + i] = \
                        (b0 + 2 * b1)[:, :, :, :, g, :].transpose(0, 2, 3, 4, 1)
    back = back.reshape(items * 128, stages * 256)
    assert np.array_equal(back[:N], idx)
    assert not back[N:].any()


def test_gemv_planes_decomposition_reproduces_the_dequantised_weight():
    """p0 + (p1 - p0) b0 + (p2 - p0) b1 + (p3 - p2 - p1 + p0) b0 b1 is the palette entry of
    index b0 + 2 b1 exactly, for bf16 palette entries evaluated in fp32 (the bit-plane GEMV's
    coefficients)."""
    rng = np.random.default_rng(9)
    pal = O.bf16_round(rng.standard_normal((500, 4)).astype(np.float32) * 0.03)
    idx = rng.integers(0, 4, 500)
    b0, b1 = idx & 1, idx >> 1
    p = pal.astype(np.float32)
    c1, c2 = p[:, 1] - p[:, 0], p[:, 2] - p[:, 0]
    c3 = (p[:, 3] - p[:, 2]) - c1
    w = p[:, 0] + c1 * b0 + c2 * b1 + c3 * (b0 & b1)
    assert np.array_equal(w.astype(np.float32), pal[np.arange(500), idx])
