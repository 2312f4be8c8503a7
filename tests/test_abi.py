"""CPU checks of the C ABI and the host logic (no compute call reaches a GPU)."""
import ctypes as C
import os
import re

import numpy as np
import pytest
import torch

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "palettize_hip.h")


@pytest.fixture(scope="module")
def lib():
    from palettize_hip import _lib
    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    return _lib.lib()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(plz_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    from palettize_hip import _lib
    names = header_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.plz_abi_version() == 18


def test_shape_errors_are_reported_without_touching_the_gpu(lib):
    rc = lib.plz_dequant(None, None, None, 8, 100, None)
    assert rc == 1 and b"multiple of 256" in lib.plz_last_error()
    rc = lib.plz_lut_linear_fwd(None, None, None, None, None, None, 12, None, None, 0, 4, 8, 256, None)
    assert rc == 1 and b"rank" in lib.plz_last_error()
    rc = lib.plz_lut_linear_fwd(None, None, None, None, None, None, 0, None, None, 0, 4, 8, 256, None)
    assert rc == 1 and b"null" in lib.plz_last_error()
    rc = lib.plz_lut_gemv(None, None, None, None, 17, 8, 256, None)
    assert rc == 1 and b"[1, 16]" in lib.plz_last_error()
    rc = lib.plz_linear_fwd_dense_residual(None, None, None, None, None, 0, None, None, None, 0,
                                           8, 8, 8, None)
    assert rc == 1 and b"residual" in lib.plz_last_error()
    rc = lib.plz_linear_bwd_x_dense_swiglu(None, None, None, None, 0, None, None, None, 0, 8, 8,
                                           8, None)
    assert rc == 1 and b"gate_up" in lib.plz_last_error()
    rc = lib.plz_soft_build_w(None, 0, None, None, 0.0, 0, None, None, None, 8, 256, None)
    assert rc == 1 and b"tau" in lib.plz_last_error()
    rc = lib.plz_rmsnorm_fwd(None, None, None, None, 4, 5000, 1e-6, None)
    assert rc == 1
    rc = lib.plz_lut_linear_bwd_palette_lora(None, None, None, None, None, 12, 1.0, None, None,
                                             None, 0, None, 0, 64, 256, 256, None)
    assert rc == 1 and b"rank" in lib.plz_last_error()
    rc = lib.plz_lut_linear_bwd_palette_lora(None, None, None, None, None, 16, 1.0, None, None,
                                             None, 0, None, 0, 64, 256, 256, None)
    assert rc == 1 and b"null" in lib.plz_last_error()
    rc = lib.plz_soft_bwd_lora(None, None, None, 0, None, 0, 0, None, None, 0.5, 0, None, None,
                               12, 1.0, None, None, None, None, 0, None, None, 0, 64, 256, 256,
                               None)
    assert rc == 1 and b"rank" in lib.plz_last_error()
    rc = lib.plz_soft_bwd_lora(None, None, None, 0, None, 0, 0, None, None, 0.5, 0, None, None,
                               16, 1.0, None, None, None, None, 0, None, None, 0, 64, 256, 256,
                               None)
    assert rc == 1 and b"null" in lib.plz_last_error()


def test_tail_split_workspace_queries(lib):
    # 640 output tiles on 256 CUs: a last wave of 128 tiles, split two ways when the reduction
    # is long enough to pay for the partials; whole waves and short reductions need none.
    # The LUT GEMMs from 4096 rows: a bf16 copy of W ahead of the tail partials.
    assert lib.plz_linear_fwd_dense_workspace(16384, 2560, 9728) == 128 * 2 * 256 * 256 * 4
    ws = lib.plz_lut_linear_fwd_workspace(16384, 2560, 9728)
    assert ws == 2560 * 9728 * 2 + 128 * 2 * 256 * 256 * 4
    assert lib.plz_lut_linear_bwd_x_workspace(16384, 9728, 2560) == (9728 * 2560 * 2
                                                                    + 128 * 2 * 256 * 256 * 4)
    assert lib.plz_lut_linear_bwd_x_workspace(4096, 1024, 2560) == 1024 * 2560 * 2
    assert lib.plz_lut_linear_bwd_x_workspace(4095, 1024, 2560) == \
        lib.plz_linear_bwd_x_dense_workspace(4095, 1024, 2560)
    assert lib.plz_lut_linear_fwd_workspace(16384, 4096, 2560) == 4096 * 2560 * 2  # 1024 tiles
    assert lib.plz_lut_linear_fwd_workspace(2048, 4096, 2560) == \
        lib.plz_linear_fwd_dense_workspace(2048, 4096, 2560)
    assert lib.plz_linear_fwd_dense_workspace(16384, 1024, 2560) == 0  # 256 tiles
    assert lib.plz_linear_bwd_x_dense_workspace(16384, 1024, 2560) == 0  # 16 stages
    assert lib.plz_lut_linear_fwd_workspace(0, 2560, 9728) == 0


def test_workspace_queries_and_missing_workspace(lib):
    ws = lib.plz_lut_linear_bwd_palette_workspace(16384, 1024, 2560)
    assert ws > 0 and ws % (1024 * 20 * 16) == 0
    assert lib.plz_lut_linear_bwd_palette_workspace(0, 1024, 2560) == 0
    # soft backward: palette partials, plus fp32 dW rows per reduction split where it splits
    # (gate at M = 16384: 2 splits; k_proj: 6; a short reduction: none)
    pal = 9728 * 20 * 16
    assert lib.plz_soft_bwd_workspace(16384, 9728, 2560) == pal + 2 * 9728 * 2560 * 4
    assert lib.plz_soft_bwd_workspace(16384, 1024, 2560) == 1024 * 20 * 16 + 6 * 1024 * 2560 * 4
    assert lib.plz_soft_bwd_workspace(192, 9728, 2560) == pal
    # with the LoRA weight gradients (rank 16): their partials [z][tiles_i][r][K] and
    # [z][tiles_j][r][N] behind the soft workspace, each start 256-byte aligned
    a256 = lambda b: (b + 255) // 256 * 256
    soft = lib.plz_soft_bwd_workspace(16384, 9728, 2560)
    assert lib.plz_soft_bwd_lora_workspace(16384, 9728, 2560, 16) == (
        a256(soft) + a256(2 * 38 * 16 * 2560 * 4) + a256(2 * 10 * 16 * 9728 * 4))
    assert lib.plz_soft_bwd_lora_workspace(16384, 9728, 2560, 0) == soft
    fake = C.c_void_p(16)  # never dereferenced: the size check fails first
    rc = lib.plz_lut_linear_bwd_palette(fake, fake, fake, fake, None, 0, 16384, 1024, 2560, None)
    assert rc == 4 and b"workspace" in lib.plz_last_error()


def test_ops_refuse_cpu_tensors():
    from palettize_hip import ops
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.pack_indices(torch.zeros(4, 16, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.lut_linear_fwd(torch.zeros(2, 256, dtype=torch.bfloat16),
                           torch.zeros(8, 16, dtype=torch.int32),
                           torch.zeros(8, 1, 4))


def test_dropin_layout_maps_match_oracle():
    from palettize_hip import fused_lut_linear_cuda as FL
    g = torch.Generator().manual_seed(0)
    N, K, GS = 512, 640, 256
    pal = torch.randn(N // GS, 4, generator=g).to(torch.bfloat16)
    nat = FL.palette_from_reference(pal, N, K, GS)
    assert nat.shape == (N, 768 // 256, 4)
    want = O.expand_reference_palette(pal.float().numpy(), N, 768, GS)
    assert np.array_equal(nat.numpy(), want)
    grad = torch.randn(N, 3, 4, generator=g)
    red = FL.palette_grad_to_reference(grad, GS)
    assert torch.allclose(red, grad.view(2, 256, 3, 4).sum((1, 2)))
    lg = torch.randn(4, K, 8, generator=g).to(torch.float16)
    nk4 = FL.logits_from_reference(lg, K)
    assert nk4.shape == (8, 768, 4)
    assert torch.equal(nk4[:, :K, :], lg.permute(2, 1, 0))
    assert torch.count_nonzero(nk4[:, K:, :]) == 0


def test_attention_argument_errors(lib):
    """Shape, support and workspace checks of the attention entry points fail before any GPU
    work (pointer 16 stands for an aligned device pointer and is never dereferenced)."""
    f = C.c_void_p(16)
    rc = lib.plz_attn_fwd(f, f, f, f, f, 1, 128, 4, 3, 128, 0.1, None)
    assert rc == 1 and b"multiple of kv_heads" in lib.plz_last_error()
    rc = lib.plz_attn_fwd(f, f, f, f, f, 1, 128, 4, 2, 64, 0.1, None)
    assert rc == 3 and b"head_dim" in lib.plz_last_error()
    rc = lib.plz_attn_fwd(f, f, f, f, f, 1, 100, 4, 2, 128, 0.1, None)
    assert rc == 1 and b"multiple of 128" in lib.plz_last_error()
    rc = lib.plz_attn_fwd(None, f, f, f, f, 1, 128, 4, 2, 128, 0.1, None)
    assert rc == 1 and b"null" in lib.plz_last_error()
    rc = lib.plz_attn_fwd(f, f, f, f, f, 1, 128, 4, 2, 128, -1.0, None)
    assert rc == 1 and b"scale" in lib.plz_last_error()
    assert lib.plz_attn_fwd(None, None, None, None, None, 0, 128, 4, 2, 128, 0.1, None) == 0
    assert lib.plz_attn_bwd_workspace(2, 256, 8) == 2 * 2 * 8 * 256 * 4  # D and -lse log2 e
    assert lib.plz_attn_bwd_workspace(0, 256, 8) == 0
    rc = lib.plz_attn_bwd(f, f, f, f, f, f, f, f, f, None, 0, 2, 256, 8, 2, 128, 0.1, None)
    assert rc == 4 and b"workspace" in lib.plz_last_error()
    rc = lib.plz_attn_bwd(f, f, f, f, f, f, f, f, f, f, 2 * 8 * 256 * 4 - 16, 2, 256, 8, 2, 128,
                          0.1, None)
    assert rc == 4
    rc = lib.plz_attn_bwd(f, C.c_void_p(24), f, f, f, f, f, f, f, f, 1 << 20, 2, 256, 8, 2, 128,
                          0.1, None)
    assert rc == 1 and b"aligned" in lib.plz_last_error()


def test_gemv_decode_layout_argument_errors(lib):
    assert lib.plz_gemv_packed_items_bytes(300, 768) == 384 * 768 // 4
    assert lib.plz_gemv_packed_items_bytes(0, 768) == 0
    rc = lib.plz_gemv_pack_indices(None, None, 8, 100, None)
    assert rc == 1 and b"multiple of 256" in lib.plz_last_error()
    assert lib.plz_gemv_pack_indices(None, None, 0, 256, None) == 0
    rc = lib.plz_lut_gemv_decode(None, None, None, None, 1, 8, 256, None)
    assert rc == 1 and b"null" in lib.plz_last_error()
    rc = lib.plz_lut_gemv_decode(None, None, None, None, 0, 8, 256, None)
    assert rc == 1 and b"[1, 16]" in lib.plz_last_error()
    rc = lib.plz_lut_gemv_grouped(None, 1, 1, 1, 7, None)
    assert rc == 1 and b"layout" in lib.plz_last_error()


def test_gemv_plan_rejects_descriptors_without_the_layouts_arrays(lib):
    """A plan for the decode layout over a descriptor that holds only the native arrays (or the
    reverse) fails at plan time instead of launching a GEMV that would read zeros. Pointers are
    never dereferenced by the plan."""
    from palettize_hip import _lib
    f = 4096  # stands for an aligned device address
    native = _lib.GemvDesc(f, f, f, f, 256, 512, 0, 0, None, None)
    decode = _lib.GemvDesc(f, None, None, f, 256, 512, 0, 0, f, f)
    empty = _lib.GemvDesc(f, None, None, f, 0, 512, 0, 0, None, None)
    for layout, ok, bad in ((_lib.PLZ_GEMV_NATIVE, native, decode),
                            (_lib.PLZ_GEMV_DECODE, decode, native)):
        descs = (_lib.GemvDesc * 2)(ok, empty)
        assert lib.plz_gemv_plan(descs, 2, 4, layout) == 2
        descs = (_lib.GemvDesc * 3)(ok, bad, empty)
        assert lib.plz_gemv_plan(descs, 3, 4, layout) == -1
        assert b"descriptor 1" in lib.plz_last_error()
    descs = (_lib.GemvDesc * 1)(native)
    assert lib.plz_gemv_plan(descs, 1, 4, 9) == -1 and b"layout" in lib.plz_last_error()


@pytest.fixture
def host_ops(monkeypatch):
    """ops with the device check and the library stubbed out: argument checks run on CPU
    tensors, and any call that would reach the library fails the test."""
    from palettize_hip import ops

    def no_call(name, *a):
        raise AssertionError(f"{name} reached the library")

    monkeypatch.setattr(ops, "_on_gpu", lambda t: True)
    monkeypatch.setattr(ops, "call", no_call)
    monkeypatch.setattr(ops, "query", lambda *a: 0)
    return ops


def test_bias_length_is_checked_before_the_call(host_ops):
    ops = host_ops
    bf = torch.bfloat16
    x = torch.zeros(4, 256, dtype=bf)
    packed = torch.zeros(24, 16, dtype=torch.int32)
    pal = torch.zeros(24, 1, 4)
    with pytest.raises(ValueError, match="bias has 16 elements"):
        ops.lut_linear_fwd(x, packed, pal, torch.zeros(16, dtype=bf))
    with pytest.raises(ValueError, match="bias has 25 elements"):
        ops.linear_fwd_dense(x, torch.zeros(24, 256, dtype=bf), torch.zeros(25, dtype=bf))
    with pytest.raises(TypeError):
        ops.lut_linear_fwd(x, packed, pal, torch.zeros(24, dtype=torch.float32))
    with pytest.raises(ValueError, match="lora_gt / lora_a"):
        ops.linear_bwd_x_dense(torch.zeros(4, 24, dtype=bf), torch.zeros(24, 256, dtype=bf),
                               torch.zeros(4, 16, dtype=bf), torch.zeros(16, 128, dtype=bf))
    with pytest.raises(ValueError, match="together"):
        ops.linear_bwd_x_dense(torch.zeros(4, 24, dtype=bf), torch.zeros(24, 256, dtype=bf),
                               torch.zeros(4, 16, dtype=bf))


def test_rmsnorm_weight_and_rstd_are_checked_before_the_call(host_ops):
    ops = host_ops
    bf = torch.bfloat16
    x = torch.zeros(6, 320, dtype=bf)
    with pytest.raises(ValueError, match="weight has 300"):
        ops.rmsnorm_fwd(x, torch.zeros(300, dtype=bf), 1e-6)
    with pytest.raises(TypeError):
        ops.rmsnorm_fwd(x, torch.zeros(320), 1e-6)
    with pytest.raises(ValueError, match="weight has 1"):
        ops.rmsnorm_bwd(x, torch.zeros(1, dtype=bf), torch.zeros(6), x)
    with pytest.raises(ValueError, match="rstd"):
        ops.rmsnorm_bwd(x, torch.zeros(320, dtype=bf), torch.zeros(5), x)
    with pytest.raises(TypeError):
        ops.rmsnorm_bwd(x, torch.zeros(320, dtype=bf), torch.zeros(6, dtype=bf), x)


def test_fused_norm_entry_points_check_arguments_before_launching(lib, host_ops):
    """The fused per-head norm + RoPE and residual add + RMSNorm entries: bad head_dim / cols
    and null operands are refused on the host; empty inputs return without a launch; the
    Python wrappers check shapes before the call."""
    rc = lib.plz_head_norm_rope_fwd(None, None, None, None, None, None, 4, 4, 2, 64, 1e-6, None)
    assert rc == 1 and b"128" in lib.plz_last_error()
    rc = lib.plz_head_norm_rope_bwd(None, None, None, None, None, None, None, 4, 4, 2, 128, None)
    assert rc == 1 and b"non-null" in lib.plz_last_error()
    assert lib.plz_head_norm_rope_fwd(None, None, None, None, None, None, 0, 4, 2, 128, 1e-6,
                                      None) == 0
    rc = lib.plz_add_rmsnorm_fwd(None, None, None, None, None, None, 4, 12, 1e-6, None)
    assert rc == 1 and b"multiple of 8" in lib.plz_last_error()
    rc = lib.plz_rmsnorm_bwd_add(None, None, None, None, None, None, 4, 256, None)
    assert rc == 1 and b"non-null" in lib.plz_last_error()
    assert lib.plz_add_rmsnorm_fwd(None, None, None, None, None, None, 0, 256, 1e-6, None) == 0
    ops = host_ops
    bf = torch.bfloat16
    x = torch.zeros(6, 320, dtype=bf)
    with pytest.raises(ValueError, match="shape mismatch"):
        ops.add_rmsnorm_fwd(x, torch.zeros(6, 312, dtype=bf), torch.zeros(320, dtype=bf), 1e-6)
    with pytest.raises(ValueError, match="weight has 300"):
        ops.add_rmsnorm_fwd(x, x, torch.zeros(300, dtype=bf), 1e-6)
    with pytest.raises(ValueError, match="do not match"):
        ops.rmsnorm_bwd_add(x, torch.zeros(320, dtype=bf), torch.zeros(6), x,
                            torch.zeros(6, 8, dtype=bf))
    q = torch.zeros(1, 16, 2, 128, dtype=bf)
    cos = torch.ones(16, 128)
    with pytest.raises(ValueError, match="cos must be"):
        ops.head_norm_rope_fwd(q, torch.zeros(128, dtype=bf), torch.ones(8, 128), cos, 1e-6)
    with pytest.raises(ValueError, match="weight has 64"):
        ops.head_norm_rope_fwd(q, torch.zeros(64, dtype=bf), cos, cos, 1e-6)


def test_layer_step_has_no_cpu_path():
    """The layer-step pieces refuse CPU tensors instead of computing in torch on the CPU."""
    from palettize_hip import layer
    x = torch.zeros(1, 128, 2, 128, dtype=torch.bfloat16)
    cos = torch.ones(128, 128)
    with pytest.raises(RuntimeError, match="no CPU path"):
        layer.apply_rope(x, cos, cos)
    with pytest.raises(RuntimeError, match="no CPU path"):
        layer.attention(x, x, x, 2, 2)
    with pytest.raises(RuntimeError, match="no CPU path"):
        layer.compute_loss(torch.zeros(2, 3, 8, dtype=torch.bfloat16),
                           torch.zeros(2, 3, 8, dtype=torch.bfloat16))
    lin = layer.SoftPalettizedLinear(256, 16, rank=8)
    with pytest.raises(RuntimeError, match="no CPU path"):
        lin(torch.zeros(4, 256, dtype=torch.bfloat16))
    from palettize_hip import qwen_model
    import torch.nn as nn
    m = qwen_model.PalettizedLinear(nn.Linear(256, 16, bias=False),
                                    torch.zeros(256, 16, dtype=torch.long), 1, 4, 256, False)
    with pytest.raises(RuntimeError, match="no CPU path"):
        m(torch.zeros(2, 256, dtype=torch.bfloat16))


def test_build_w_plan_accepts_philox_descriptors(lib):
    """A batched build-W descriptor without a noise tensor (in-kernel Philox noise with its own
    key) plans like one with a tensor; a missing logits pointer still fails. Pointers are never
    dereferenced by the plan."""
    from palettize_hip import _lib
    f = 4096
    assert C.sizeof(_lib.BuildWDesc) == 5 * 8 + 2 * 8 + 2 * 4 + 8 + 8 + 8 + 8
    d = (_lib.BuildWDesc * 3)(
        _lib.BuildWDesc(f, f, f, f, None, 64, 512, 0, 0, 0, 0),
        _lib.BuildWDesc(f, None, f, f, None, 8, 256, 1, 0, 0, 7),
        _lib.BuildWDesc(f, None, f, f, None, 0, 256, 0, 0, 0, 9))
    assert lib.plz_build_w_plan(d, 3) == 64 * 256 // 256 + 8 * 128 // 256
    assert d[1].block_begin == 64 and d[2].block_begin == 68
    bad = (_lib.BuildWDesc * 1)(_lib.BuildWDesc(None, None, f, f, None, 8, 256, 0, 0, 0, 1))
    assert lib.plz_build_w_plan(bad, 1) < 0


def test_swiglu_cat_gemm_checks_arguments_before_launching(lib):
    """plz_linear_fwd_dense_swiglu_cat: F not a multiple of 128, a bad rank and null or
    misaligned operands are refused on the host; an empty problem returns without a launch."""
    f = 4096
    rc = lib.plz_linear_fwd_dense_swiglu_cat(f, f, None, None, 0, None, f, 64, 192, 256, None)
    assert rc == 1 and b"F of 128" in lib.plz_last_error()
    rc = lib.plz_linear_fwd_dense_swiglu_cat(f, f, f, f, 12, None, f, 64, 128, 256, None)
    assert rc == 1 and b"rank" in lib.plz_last_error()
    rc = lib.plz_linear_fwd_dense_swiglu_cat(f, None, None, None, 0, None, f, 64, 128, 256, None)
    assert rc == 1 and b"non-null" in lib.plz_last_error()
    rc = lib.plz_linear_fwd_dense_swiglu_cat(f, f, None, None, 0, f + 2, f, 64, 128, 256, None)
    assert rc == 1 and b"aligned" in lib.plz_last_error()
    assert lib.plz_linear_fwd_dense_swiglu_cat(None, None, None, None, 0, None, None, 0, 128, 256,
                                               None) == 0


def test_adamw_build_plan_checks_the_pairs(lib):
    """plz_adamw_plan_build: the descriptors with a build must come last, each build must
    rebuild its own bf16 [N, K, 4] parameter; the split block is the first built block.
    Pointers are never dereferenced by the plan."""
    from palettize_hip import _lib
    P, G, W = 4096, 8192, 12288

    def adam(param, n):
        return _lib.AdamWDesc(param, G, G, G, G, n, _lib.PLZ_DT_BF16, 0, 1e-3, -1.0, 1.0, 0.0, 0)

    def build(param, N, K):
        return _lib.BuildWDesc(param, None, G, W, None, N, K, _lib.PLZ_DT_BF16, 0, 0, 7, 0)

    none = _lib.BuildWDesc()
    split = C.c_int64(-1)
    d = (_lib.AdamWDesc * 3)(adam(P, 1000), adam(P + 65536, 8 * 256 * 4), adam(P + 131072, 4 * 512 * 4))
    b = (_lib.BuildWDesc * 3)(none, build(P + 65536, 8, 256), build(P + 131072, 4, 512))
    total = lib.plz_adamw_plan_build(d, b, 3, C.byref(split))
    assert total == 1 + 1 + 1 and split.value == 1
    # a build before a descriptor without one
    b2 = (_lib.BuildWDesc * 3)(build(P, 1, 256), none, none)
    d2 = (_lib.AdamWDesc * 3)(adam(P, 1024), adam(P + 65536, 64), adam(P + 131072, 64))
    assert lib.plz_adamw_plan_build(d2, b2, 3, C.byref(split)) < 0
    assert b"must come last" in lib.plz_last_error()
    # a build of another tensor, and a size that does not match N*K*4
    for bad in (build(P + 4096, 8, 256), build(P + 65536, 8, 512)):
        d3 = (_lib.AdamWDesc * 1)(adam(P + 65536, 8 * 256 * 4))
        b3 = (_lib.BuildWDesc * 1)(bad)
        assert lib.plz_adamw_plan_build(d3, b3, 1, C.byref(split)) < 0
        assert b"own bf16" in lib.plz_last_error()
    # no builds at all: the split is the end
    d4 = (_lib.AdamWDesc * 1)(adam(P, 1000))
    b4 = (_lib.BuildWDesc * 1)(none)
    assert lib.plz_adamw_plan_build(d4, b4, 1, C.byref(split)) == 1 and split.value == 1
