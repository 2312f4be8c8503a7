"""GPU tests of the drop-in modules PalettizedLinear and QwenLoRA (qwen_model.py:65-304).

They follow the reference's own module tests (scripts/test_palettized_v2.py): forward and
grad_x against the naive gather + matmul of test_palettized_v2.py:19-33 in both index
orientations, grad_palette against autograd of that formula and a finite difference
(test_palettized_v2.py:111-159), here in fp64 on the CPU. They also cover the train/eval
dispatch (qwen_model.py:147-196), extract_hard_indices (:198-209), QwenLoRA's alpha/r scaling
and LoftQ init (:236-258, :291-304), and the packed-index cache of the functional interface.
"""
import pytest
import torch
import torch.nn as nn

from helpers import assert_close, f32

pytestmark = pytest.mark.gpu
QM = pytest.importorskip("palettize_hip.qwen_model")
FL = pytest.importorskip("palettize_hip.fused_lut_linear_cuda")


def naive_forward(x, palette, indices, group_size, pre_transposed, bias=None):
    """test_palettized_v2.py:19-33 in fp64: W = flat_palette[(c // GS) * 4 + idx] over the
    stored (rows, cols) indices, y = x @ W, or x @ W.T when pre_transposed."""
    si, so = indices.shape
    flat_idx = (torch.arange(so) // group_size)[None, :].expand(si, so) * 4 + indices.long()
    W = palette.double().reshape(-1)[flat_idx]
    y = x.double() @ (W.T if pre_transposed else W)
    if bias is not None:
        y = y + bias.double()
    return y


def _module(in_dim, out_dim, gs, pre_transposed, seed, bias=False, soft=False, n_groups=None):
    g = torch.Generator().manual_seed(seed)
    lin = nn.Linear(in_dim, out_dim, bias=bias)
    if bias:
        with torch.no_grad():
            lin.bias.copy_(torch.randn(out_dim, generator=g) * 0.1)
    shape = (out_dim, in_dim) if pre_transposed else (in_dim, out_dim)
    indices = torch.randint(0, 4, shape, generator=g)
    if n_groups is None:  # groups run along the stored indices' second dimension
        n_groups = -(-(in_dim if pre_transposed else out_dim) // gs)
    palette = torch.randn(n_groups, 4, generator=g) * 0.1
    m = QM.PalettizedLinear(lin, indices, n_groups, 4, gs, pre_transposed=pre_transposed,
                            initial_palette=palette, use_soft_indices=soft)
    return m


# (in, out, group_size, n_groups): the reference test's shape (groups of 16; with
# pre_transposed the groups run along the 64 inputs, so 4 of its 8 palettes are used), a
# non-multiple-of-256 K, and Qwen-sized square and rectangular weights with groups of 256
CASES = [(64, 128, 16, 8), (320, 136, 8, None), (2560, 2560, 256, None), (512, 1024, 256, None),
         (1024, 512, 128, None)]


@pytest.mark.parametrize("pre_transposed", [False, True], ids=["in-out", "pre-transposed"])
@pytest.mark.parametrize("in_dim,out_dim,gs,ng", CASES)
def test_forward_and_grads_match_naive_gather(dev, pre_transposed, in_dim, out_dim, gs, ng):
    m = _module(in_dim, out_dim, gs, pre_transposed, seed=in_dim + out_dim, bias=in_dim == 320,
                n_groups=ng).to(dev)
    m.eval()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 8, in_dim, generator=g).to(torch.bfloat16)
    gy = torch.randn(2, 8, out_dim, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = m(xd)
    assert y.shape == (2, 8, out_dim) and y.dtype == torch.bfloat16
    y.backward(gy.to(dev))
    pal = m.palette.detach().cpu().double().requires_grad_(True)
    xr = x.reshape(-1, in_dim).double().requires_grad_(True)
    bias = None if m.bias is None else m.bias.cpu()
    want = naive_forward(xr, pal, m.indices.cpu(), gs, pre_transposed, bias)
    want.backward(gy.reshape(-1, out_dim).double())
    assert_close(f32(y).reshape(-1, out_dim), want.detach().numpy(), what="y")
    assert_close(f32(xd.grad).reshape(-1, in_dim), xr.grad.numpy(), what="grad_x")
    assert m.palette.grad.dtype == torch.bfloat16 and m.palette.grad.shape == m.palette.shape
    used = -(-(in_dim if pre_transposed else out_dim) // gs)
    assert_close(f32(m.palette.grad)[:used], pal.grad.numpy()[:used], what="grad_palette")
    assert torch.count_nonzero(m.palette.grad[used:]) == 0  # palettes no row or column uses
    # the formula's own pin: it is linear in each palette entry, so a central difference of
    # the scalar <gy, y> is exact
    with torch.no_grad():
        yy = lambda p: float((naive_forward(x.reshape(-1, in_dim), p, m.indices.cpu(), gs,
                                            pre_transposed, bias)
                              * gy.reshape(-1, out_dim).double()).sum())
        e = torch.zeros_like(pal)
        e[0, 1] = 1e-3
        fd = (yy(pal.detach() + e) - yy(pal.detach() - e)) / 2e-3
        assert abs(fd - float(pal.grad[0, 1])) <= 1e-9 * max(1.0, abs(fd))


def test_train_eval_dispatch_and_extract_hard_indices(dev):
    """With soft indices a module trains through the Gumbel-softmax path (logits get a
    gradient) and evaluates through the hard path; its +-10 one-hot logits make both select the
    stored indices, so the two forwards agree. extract_hard_indices freezes argmax(logits):
    afterwards the hard path uses the new indices (not the packed copy of the old ones)."""
    in_dim, out_dim, gs = 512, 256, 256
    m = _module(in_dim, out_dim, gs, False, seed=3, soft=True).to(dev)
    assert m.index_logits.shape == (4, in_dim, out_dim)
    assert m.index_logits.dtype == torch.float16
    onehot = torch.nn.functional.one_hot(m.indices, 4).permute(2, 0, 1).bool()
    assert torch.equal(m.index_logits == 10.0, onehot)
    assert torch.equal(m.index_logits == -10.0, ~onehot)
    x = torch.randn(64, in_dim, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    x = x.to(dev)
    m.eval()
    y_eval = m(x)
    assert m.index_logits.grad is None
    m.train()
    y_train = m(x)
    y_train.float().sum().backward()
    assert m.index_logits.grad is not None and m.index_logits.grad.shape == m.index_logits.shape
    want = naive_forward(x.cpu(), m.palette.detach().cpu(), m.indices.cpu(), gs, False)
    assert_close(f32(y_eval), want.numpy(), what="eval (hard)")
    assert_close(f32(y_train), want.numpy(), what="train (soft, one-hot logits)")
    # move the argmax of a block of weights, then freeze
    with torch.no_grad():
        m.index_logits[:, :, :16] = -10.0
        m.index_logits[2, :, :16] = 10.0
    m.extract_hard_indices()
    assert m.index_logits is None and not m.use_soft_indices
    new_idx = m.indices.cpu()
    assert bool((new_idx[:, :16] == 2).all())
    assert torch.equal(m.indices_int8.cpu(), new_idx.to(torch.int8))
    m.train()  # no logits any more: the hard path even in training mode
    y2 = m(x)
    want2 = naive_forward(x.cpu(), m.palette.detach().cpu(), new_idx, gs, False)
    assert_close(f32(y2), want2.numpy(), what="after extract_hard_indices")


def test_functional_pack_cache_never_serves_a_freed_or_modified_tensor(dev):
    """fused_lut_linear packs each index tensor once; a different tensor placed at a freed one's
    address, or an in-place write to the indices, must not reuse the old packed copy."""
    K, N, GS = 512, 256, 256
    g = torch.Generator().manual_seed(9)
    x = torch.randn(32, K, generator=g).to(torch.bfloat16).to(dev)
    pal = (torch.randn(N // GS, 4, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    outs = []
    for trial in range(3):
        idx = torch.randint(0, 4, (K, N), generator=g).to(torch.int8).to(dev)
        ptr = idx.data_ptr()
        y = FL.fused_lut_linear(x, pal, idx)
        want = naive_forward(x.cpu(), pal.cpu(), idx.cpu(), GS, False)
        assert_close(f32(y), want.numpy(), what=f"trial {trial}")
        outs.append((ptr, y))
        del idx
    idx = torch.randint(0, 4, (K, N), generator=g).to(torch.int8).to(dev)
    y_before = FL.fused_lut_linear(x, pal, idx)
    idx.copy_(torch.randint(0, 4, (K, N), generator=g).to(torch.int8))
    y_after = FL.fused_lut_linear(x, pal, idx)
    want = naive_forward(x.cpu(), pal.cpu(), idx.cpu(), GS, False)
    assert_close(f32(y_after), want.numpy(), what="after in-place write")
    assert not torch.equal(y_before, y_after)


@pytest.mark.parametrize("pre_transposed", [False, True], ids=["in-out", "pre-transposed"])
def test_qwen_lora_loftq_init_scaling_forward_backward(dev, pre_transposed):
    """LoftQ: B A^T * alpha/r is the rank-r truncated SVD of (W_orig - W_palettized) in the
    (out, in) orientation for either index orientation; forward adds (alpha/r) (x A) B^T to the
    base output, and A, B and x get the gradients of that expression."""
    in_dim, out_dim, gs, rank, alpha = 512, 256, 256, 16, 32.0
    g = torch.Generator().manual_seed(21)
    base = _module(in_dim, out_dim, gs, pre_transposed, seed=22)
    w_orig = torch.randn(out_dim, in_dim, generator=g) * 0.05
    lora = QM.QwenLoRA(base, rank=rank, alpha=alpha, init="loftq", original_weight=w_orig)
    assert lora.scaling == alpha / rank
    assert lora.lora_A.shape == (in_dim, rank) and lora.lora_B.shape == (out_dim, rank)
    assert lora.lora_A.dtype == torch.bfloat16
    # residual in fp64 from the naive gather, as (out, in)
    w_pal = naive_forward(torch.eye(in_dim), base.palette.detach(), base.indices, gs,
                          pre_transposed).T          # x = I gives W^T (in, out) -> (out, in)
    U, S, Vh = torch.linalg.svd(w_orig.double() - w_pal, full_matrices=False)
    best = (U[:, :rank] * S[:rank]) @ Vh[:rank]
    got = lora.lora_B.detach().double() @ lora.lora_A.detach().double().T * lora.scaling
    assert_close(got.numpy(), best.numpy(), max_rel=2e-2, min_cos=0.9995, what="LoftQ B A^T")
    lora = lora.to(dev).eval()
    x = torch.randn(3, 5, in_dim, generator=g).to(torch.bfloat16)
    gy = torch.randn(3, 5, out_dim, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = lora(xd)
    y.backward(gy.to(dev))
    A = lora.lora_A.detach().cpu().double().requires_grad_(True)
    B = lora.lora_B.detach().cpu().double().requires_grad_(True)
    xr = x.reshape(-1, in_dim).double().requires_grad_(True)
    want = naive_forward(xr, base.palette.detach().cpu(), base.indices.cpu(), gs, pre_transposed)
    want = want + (xr @ A) @ B.T * lora.scaling
    want.backward(gy.reshape(-1, out_dim).double())
    assert_close(f32(y).reshape(-1, out_dim), want.detach().numpy(), what="y")
    assert_close(f32(xd.grad).reshape(-1, in_dim), xr.grad.numpy(), what="grad_x")
    assert_close(f32(lora.lora_A.grad), A.grad.numpy(), what="grad_A")
    assert_close(f32(lora.lora_B.grad), B.grad.numpy(), what="grad_B")


def test_qwen_lora_random_init_adds_nothing(dev):
    """init='random': A ~ N(0, 0.01), B = 0 (qwen_model.py:262-264), so the adapter's output
    equals the base output bit for bit until B moves."""
    base = _module(512, 256, 256, False, seed=5)
    torch.manual_seed(0)
    lora = QM.QwenLoRA(base, rank=16, alpha=32, init="random").to(dev)
    assert torch.count_nonzero(lora.lora_B) == 0
    assert 0.005 < float(lora.lora_A.detach().float().std()) < 0.02
    x = torch.randn(2, 7, 512).to(torch.bfloat16).to(dev)
    assert torch.equal(lora(x), base.to(dev)(x))


def test_pre_transposed_lora_a_shape_from_palettized_files(dev):
    """The reference's one pre-transposed use: a palettized LoRA A, stored (rank, in_dim) with
    groups of 256 along in_dim (qwen_model.py:360-414). Rank 32, in 2560, M = 512."""
    rank, in_dim = 32, 2560
    m = _module(in_dim, rank, 256, True, seed=31, n_groups=in_dim // 256).to(dev)
    x = torch.randn(512, in_dim, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = m(xd)
    gy = torch.randn(512, rank, generator=torch.Generator().manual_seed(33)).to(torch.bfloat16)
    y.backward(gy.to(dev))
    pal = m.palette.detach().cpu().double().requires_grad_(True)
    xr = x.double().requires_grad_(True)
    want = naive_forward(xr, pal, m.indices.cpu(), 256, True)
    want.backward(gy.double())
    assert_close(f32(y), want.detach().numpy(), what="y")
    assert_close(f32(xd.grad), xr.grad.numpy(), what="grad_x")
    assert_close(f32(m.palette.grad), pal.grad.numpy(), what="grad_palette")
