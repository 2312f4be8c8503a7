"""On-disk format (.idx2 / .lut_scalar / metadata.json): fixtures cut from the reference's own
palettized files, the oracle's conversions, and the host-side reader (no GPU)."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
REF_DIR = "/root/reference/palettized/superblock_0"


@pytest.fixture(scope="module")
def fixture():
    meta = json.load(open(os.path.join(GOLD, "palettized_k_proj_meta.json")))
    z = np.load(os.path.join(GOLD, "palettized_k_proj_slice.npz"))
    return meta, z["idx2_slice"].tobytes(), z["lut_scalar"].tobytes()


def test_fixture_metadata_schema(fixture):
    meta, idx, lut = fixture
    top, e = meta["top"], meta["entry"]
    assert top["bitwidth"] == 2 and top["group_size"] == 256
    assert top["nibble_order"] == "LSB_FIRST" and top["indices_layout"] == "D0D1"
    N, K = e["dense_shape"]
    assert (N, K) == (1024, 2560) and e["groups"] == N // 256
    assert e["packed_len_bytes"] == N * K // 4
    assert len(idx) == meta["k_rows"] * N // 4
    # the lut fixture is the whole file: its digest is the reference's
    assert hashlib.sha256(lut).hexdigest() == e["sha256_lut"]
    from palettize_hip.formats import sanitize_name
    assert sanitize_name(meta["name"]) + ".idx2" == e["index_file"]
    assert sanitize_name(meta["name"]) + ".lut_scalar" == e["lut_file"]


def test_fixture_palettes_are_sorted_kmeans_centres(fixture):
    _, _, lut = fixture
    pal = np.frombuffer(lut, dtype=np.float16).astype(np.float32).reshape(-1, 4)
    assert pal.shape == (4, 4)
    assert np.all(np.diff(pal, axis=1) > 0)  # palettize_pytorch.py:79-85 sorts the centres


def test_fixture_indices_decode_like_coreml_bits(fixture):
    meta, idx, _ = fixture
    N = meta["entry"]["dense_shape"][0]
    kn = O.unpack_idx2(idx, len(idx) * 4).reshape(-1, N)
    bits = np.unpackbits(np.frombuffer(idx, np.uint8).reshape(-1, 1), bitorder="little", axis=-1)
    apple = (bits[:, 0::2] | (bits[:, 1::2] << 1)).reshape(-1, N)
    assert np.array_equal(kn, apple)
    assert set(np.unique(kn)) == {0, 1, 2, 3}


def test_oracle_idx2_native_round_trip(fixture):
    meta, idx, _ = fixture
    N = meta["entry"]["dense_shape"][0]
    K = meta["k_rows"]
    packed = O.idx2_to_native(idx, N, K)
    assert packed.shape == (N, K // 16)
    kn = O.unpack_idx2(idx, N * K).reshape(K, N)
    assert np.array_equal(O.unpack_native(packed), kn.T)
    assert O.native_to_idx2(packed) == idx


def test_oracle_logits_argmax_first_max_wins():
    lg = np.zeros((4, 2, 4), np.float32)
    lg[:, 0, 0] = [1, 3, 3, 2]   # tie between planes 1 and 2 -> 1
    lg[:, 0, 1] = [5, 5, 5, 5]   # all equal -> 0
    lg[:, 0, 2] = [0, 0, 0, 1]
    assert list(O.logits_argmax(lg)[0, :3]) == [1, 0, 3]


@pytest.mark.skipif(not os.path.isdir(REF_DIR), reason="reference checkout not present")
def test_reference_files_match_metadata_and_fixture(fixture):
    from palettize_hip.formats import read_metadata, verify_tensor
    meta, idx, lut = fixture
    m = read_metadata(REF_DIR)
    e = m["tensors"][meta["name"]]
    verify_tensor(REF_DIR, e)
    data = open(os.path.join(REF_DIR, e["index_file"]), "rb").read()
    assert data[: len(idx)] == idx


def test_metadata_writer_schema(tmp_path):
    from palettize_hip import formats as F
    idx = O.pack_idx2(np.arange(256 * 8) % 4)
    lut = np.arange(4, dtype=np.float16).tobytes()
    e = F.tensor_entry("model.layers.9.mlp.up_proj.weight", 8, 256, idx, lut)
    assert e["index_file"] == "model_layers_9_mlp_up_proj_weight.idx2"
    assert e["groups"] == 1 and e["packed_len_bytes"] == len(idx)
    assert e["sha256_idx"] == hashlib.sha256(idx).hexdigest()
    F.write_metadata_json(str(tmp_path / "metadata.json"), {"w": e})
    back = F.read_metadata(str(tmp_path))
    assert back["tensors"]["w"] == e and back["bitwidth"] == 2 and back["default_group_size"] == 256
