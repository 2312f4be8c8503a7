"""GPU parity of the on-disk format converters against the oracle, on the real-file fixture
and on random inputs; end to end from the fixture bytes to a forward pass."""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from helpers import assert_close, f32, gen, randn_bf16

pytestmark = pytest.mark.gpu
F = pytest.importorskip("palettize_hip.formats")
from palettize_hip import ops  # noqa: E402

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def fixture():
    meta = json.load(open(os.path.join(GOLD, "palettized_k_proj_meta.json")))
    z = np.load(os.path.join(GOLD, "palettized_k_proj_slice.npz"))
    return meta, z["idx2_slice"].tobytes(), z["lut_scalar"].tobytes()


def test_idx2_to_packed_on_real_bytes(dev, fixture):
    meta, idx, _ = fixture
    N, K = meta["entry"]["dense_shape"][0], meta["k_rows"]
    packed = F.idx2_to_packed(idx, N, K, dev)
    assert np.array_equal(packed.cpu().numpy(), O.idx2_to_native(idx, N, K))
    assert F.packed_to_idx2(packed) == idx


@pytest.mark.parametrize("N,K", [(4, 16), (8, 256), (264, 512), (1024, 2560)])
def test_idx2_round_trips(dev, N, K):
    rng = np.random.default_rng(N + K)
    kn = rng.integers(0, 4, (K, N), dtype=np.uint8)
    data = O.pack_idx2(kn)
    packed = F.idx2_to_packed(data, N, K, dev)
    assert np.array_equal(packed.cpu().numpy(), O.pack_native(np.ascontiguousarray(kn.T)))
    assert F.packed_to_idx2(packed) == data


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_logits_argmax_export(dev, dtype):
    K, N = 64, 40
    lg = torch.randn(4, K, N, generator=gen(7)).to(dtype)
    lg[1, :8] = lg[2, :8] = 4.0            # ties: the first maximal plane (1) wins
    lg[:, 8:10] = 1.0                       # all equal: plane 0
    data = F.logits_argmax_idx2(lg.to(dev))
    want = O.logits_argmax(lg.float().numpy())
    assert data == O.pack_idx2(want)
    assert np.all(want[:8] == 1) and np.all(want[8:10] == 0)


def test_lut_to_palette(dev, fixture):
    meta, _, lut = fixture
    N, K = meta["entry"]["dense_shape"]
    lut16 = torch.frombuffer(bytearray(lut), dtype=torch.float16).reshape(-1, 4)
    pal = F.lut_to_palette(lut16.to(dev), N, K)
    want = O.expand_reference_palette(lut16.float().numpy(), N, K)
    assert np.array_equal(pal.cpu().numpy(), want)


def test_fixture_end_to_end_forward_and_decode(dev, fixture):
    """Real file bytes -> device layouts -> forward and decode GEMV, against the reference's
    own gather W[k, n] = palette[n // 256][idx[k, n]] (qwen_model.py:97-102)."""
    meta, idx, lut = fixture
    N, K = meta["entry"]["dense_shape"][0], meta["k_rows"]
    lut16 = torch.frombuffer(bytearray(lut), dtype=torch.float16).reshape(-1, 4)
    packed = F.idx2_to_packed(idx, N, K, dev)
    pal = F.lut_to_palette(lut16.to(dev), N, K)
    kn = O.unpack_idx2(idx, N * K).reshape(K, N)
    W_kn = O.reference_weight(kn, lut16.float().numpy())      # (K, N)
    for M in (1, 16):
        x = randn_bf16(M, K, seed=M)
        want = f32(x).astype(np.float64) @ W_kn
        y = ops.lut_gemv(x.to(dev), packed, pal)
        assert_close(f32(y), want, what=f"gemv M={M}")
    x = randn_bf16(64, K, seed=3)
    y = ops.lut_linear_fwd(x.to(dev), packed, pal)
    assert_close(f32(y), f32(x).astype(np.float64) @ W_kn, what="forward")


def test_save_and_load_tensor_files(dev, tmp_path, fixture):
    meta, idx, lut = fixture
    N, K = meta["entry"]["dense_shape"][0], meta["k_rows"]
    lut16 = torch.frombuffer(bytearray(lut), dtype=torch.float16).reshape(-1, 4)
    packed = F.idx2_to_packed(idx, N, K, dev)
    e = F.save_tensor(str(tmp_path), "blk.k_proj.weight", lut16, packed=packed)
    F.write_metadata_json(str(tmp_path / "metadata.json"), {"blk.k_proj.weight": e})
    assert open(tmp_path / e["index_file"], "rb").read() == idx
    got = F.load_tensor(str(tmp_path), "blk.k_proj.weight", dev)
    assert torch.equal(got["packed"], packed)
    assert torch.equal(got["lut"].cpu(), lut16)
    kn = F.load_indices(str(tmp_path / e["index_file"]), N, K, dev)
    assert np.array_equal(kn.cpu().numpy(), O.unpack_idx2(idx, N * K).reshape(K, N))
