"""The entry point that allocates nothing, plz_lut_linear_bwd_palette_noalloc, against the
workspace entry point plz_lut_linear_bwd_palette it varies, through the C ABI: two calls in a
row, the second with a smaller input (its scratch keeps the first call's contents), bit-equal
wherever the workspace variant's split count fits the scratch; plus the oracle and the size
limit."""
import pytest
import torch

import oracle as O
from helpers import assert_close, f32, make_weight, randn_bf16

pytestmark = pytest.mark.gpu
ops = pytest.importorskip("palettize_hip.ops")
SCRATCH = 32 << 20


def _case(M, N, K, seed, dev):
    idx, _ = make_weight(N, K, seed=seed)
    x = randn_bf16(M, K, seed=seed + 1)
    gy = randn_bf16(M, N, seed=seed + 2)
    return idx, x, gy, ops.pack_indices(idx.to(dev)), x.to(dev), gy.to(dev)


@pytest.mark.parametrize("shapes", [
    [(16384, 9728, 2560), (2048, 1024, 2560)],    # gate at config 3, then k_proj at M = 2048
    [(4096, 2560, 4096), (77, 1032, 768)],
])
def test_noalloc_matches_workspace_entry_point(dev, shapes):
    for call_no, (M, N, K) in enumerate(shapes):
        print(f"noalloc call {call_no}: M={M} N={N} K={K}", flush=True)
        idx, x, gy, p, xd, gyd = _case(M, N, K, 40 + call_no, dev)
        want = ops.lut_linear_bwd_palette(xd, gyd, p)
        out = torch.full((N, K // 256, 4), float("nan"), device=dev)
        got = ops.lut_linear_bwd_palette_noalloc(xd, gyd, p, out=out)
        assert got is out
        torch.cuda.synchronize()
        if ops.query("plz_lut_linear_bwd_palette_workspace", M, N, K) <= SCRATCH:
            assert torch.equal(got, want), f"call {call_no}: differs from the workspace variant"
        else:
            assert_close(f32(got), f32(want), max_rel=1e-5, min_cos=0.999999)
        rows = torch.tensor([0, N // 3, N - 1])
        ref = O.grad_palette(f32(x), f32(gy[:, rows]), idx[rows].numpy())
        assert_close(f32(got[rows.to(dev)]), ref, max_rel=1e-3, min_cos=0.99999,
                     what=f"call {call_no} vs oracle")


def test_noalloc_rejects_weights_beyond_the_scratch(dev):
    from palettize_hip import _lib
    lib = _lib.lib()
    # null pointers: the size check fires first; were it ever moved after the null-pointer
    # check, the call would still return PLZ_EINVAL without launching anything
    N, K = 16384, 16640   # N * K / 8 bytes of partials per split > 32 MiB
    rc = lib.plz_lut_linear_bwd_palette_noalloc(None, None, None, None, 64, N, K, None)
    assert rc == 1 and b"scratch" in lib.plz_last_error()
