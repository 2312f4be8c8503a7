"""Reading and writing the palettized on-disk format, with the device-side conversions.

The format is the reference's (CoreML palettizer schema):

* ``<name>.idx2``: the (K, N) index matrix (W^T for a weight of dense shape [N, K]) flattened
  row-major, 4 two-bit indices per byte, LSB first (palettize_core.py:31-47, read back by
  palettize_core.py:159-172).
* ``<name>.lut_scalar``: fp16 palettes (G, 4), G = N / 256, one per 256 output rows
  (palettize_pytorch.py:150-159).
* ``metadata.json``: per-tensor shapes, files and sha256 digests (palettize_core.py:120-145,
  palettize_pytorch.py:162-181); file names from ``sanitize_name`` (palettize_pytorch.py:20-22).

The byte layouts are converted on the device by the library (``plz_idx2_to_packed``,
``plz_packed_to_idx2``, ``plz_logits_argmax_idx2``, ``plz_lut_to_palette``); this module only
moves bytes between files and device memory and checks digests.
"""
from __future__ import annotations

import hashlib
import json
import os

import torch

from ._lib import PLZ_DT_BF16, PLZ_DT_FP16, call

BITWIDTH = 2
GROUP_SIZE = 256
PALETTE_SIZE = 1 << BITWIDTH


def sanitize_name(name: str) -> str:
    """Tensor name -> file stem (palettize_pytorch.py:20-22)."""
    return name.replace(".", "_").replace("/", "_").replace("[", "").replace("]", "")


def sha256_bytes(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _device(device) -> torch.device:
    d = torch.device(device)
    if d.type != "cuda":
        raise ValueError("the format converters run on the GPU; pass a cuda device")
    return d


# ---- reading -------------------------------------------------------------------------------
def read_metadata(directory: str) -> dict:
    with open(os.path.join(directory, "metadata.json")) as f:
        return json.load(f)


def verify_tensor(directory: str, entry: dict) -> None:
    """Sizes and sha256 digests of one metadata entry's .idx2 and .lut_scalar files."""
    N, K = entry["dense_shape"]
    with open(os.path.join(directory, entry["index_file"]), "rb") as f:
        idx = f.read()
    with open(os.path.join(directory, entry["lut_file"]), "rb") as f:
        lut = f.read()
    if len(idx) != (N * K + 3) // 4 or len(idx) != entry["packed_len_bytes"]:
        raise ValueError(f"{entry['index_file']}: {len(idx)} bytes for a {N}x{K} tensor")
    if len(lut) != entry["groups"] * PALETTE_SIZE * 2:
        raise ValueError(f"{entry['lut_file']}: {len(lut)} bytes for {entry['groups']} groups")
    if sha256_bytes(idx) != entry["sha256_idx"]:
        raise ValueError(f"{entry['index_file']}: sha256 mismatch")
    if sha256_bytes(lut) != entry["sha256_lut"]:
        raise ValueError(f"{entry['lut_file']}: sha256 mismatch")


def idx2_to_packed(data, N: int, K: int, device="cuda") -> torch.Tensor:
    """.idx2 bytes (bytes or a uint8 tensor) -> native packed int32 [N, K/16] on the device."""
    dev = _device(device)
    if isinstance(data, (bytes, bytearray, memoryview)):
        raw = torch.frombuffer(bytearray(data), dtype=torch.uint8)
    else:
        raw = data
    if raw.numel() < N * K // 4:
        raise ValueError(f"{raw.numel()} index bytes for a {N}x{K} tensor")
    raw = raw[: N * K // 4].to(dev)
    packed = torch.empty((N, K // 16), dtype=torch.int32, device=dev)
    call("plz_idx2_to_packed", raw.data_ptr(), packed.data_ptr(), N, K, _stream(dev))
    return packed


def lut_to_palette(lut_fp16: torch.Tensor, N: int, K: int, group_size: int = GROUP_SIZE):
    """fp16 palettes (G, 4) (device) -> native fp32 palette [N, K/256, 4]."""
    lut = lut_fp16.to(torch.float16).contiguous()
    pal = torch.empty((N, K // 256, 4), dtype=torch.float32, device=lut.device)
    call("plz_lut_to_palette", lut.data_ptr(), pal.data_ptr(), N, K, group_size,
         _stream(lut.device))
    return pal


def read_lut_scalar(path: str, device="cuda") -> torch.Tensor:
    """.lut_scalar -> fp16 (G, 4) on the device (palettize_core.py:175-178 reads the same
    values as fp32)."""
    with open(path, "rb") as f:
        data = f.read()
    lut = torch.frombuffer(bytearray(data), dtype=torch.float16).reshape(-1, PALETTE_SIZE)
    return lut.to(_device(device))


def load_indices(idx_path: str, out_dim: int, in_dim: int, device="cuda") -> torch.Tensor:
    """The reference's (in_dim, out_dim) = (K, N) uint8 index matrix (palettize_core.py:167-172),
    decoded on the device."""
    from . import ops
    with open(idx_path, "rb") as f:
        data = f.read()
    packed = idx2_to_packed(data, out_dim, in_dim, device)
    return ops.unpack_indices(packed).t().contiguous()


def load_tensor(directory: str, name: str, device="cuda", verify: bool = True) -> dict:
    """One palettized linear of a metadata.json directory: native packed indices [N, K/16],
    native fp32 palette [N, K/256, 4], the reference palette (G, 4) fp16 and the entry."""
    meta = read_metadata(directory)
    entry = meta["tensors"][name]
    if verify:
        verify_tensor(directory, entry)
    N, K = entry["dense_shape"]
    gs = entry.get("group_size", meta.get("group_size", GROUP_SIZE))
    with open(os.path.join(directory, entry["index_file"]), "rb") as f:
        packed = idx2_to_packed(f.read(), N, K, device)
    lut = read_lut_scalar(os.path.join(directory, entry["lut_file"]), device)
    return dict(packed=packed, palette=lut_to_palette(lut, N, K, gs), lut=lut, entry=entry)


# ---- writing -------------------------------------------------------------------------------
def packed_to_idx2(packed: torch.Tensor) -> bytes:
    """Native packed int32 [N, K/16] (device) -> .idx2 bytes."""
    N, K = packed.shape[0], packed.shape[1] * 16
    out = torch.empty(N * K // 4, dtype=torch.uint8, device=packed.device)
    call("plz_packed_to_idx2", packed.contiguous().data_ptr(), out.data_ptr(), N, K,
         _stream(packed.device))
    return out.cpu().numpy().tobytes()


def logits_argmax_idx2(logits: torch.Tensor) -> bytes:
    """Index logits (4, K, N) fp16/bf16 (device) -> .idx2 bytes of their argmax over the 4
    planes, first maximum winning (train_qwen.py:826-835)."""
    if logits.dim() != 3 or logits.shape[0] != PALETTE_SIZE:
        raise ValueError("logits must be (4, K, N)")
    if logits.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("logits must be fp16 or bf16")
    _, K, N = logits.shape
    lg = logits.contiguous()
    out = torch.empty(K * N // 4, dtype=torch.uint8, device=lg.device)
    call("plz_logits_argmax_idx2", lg.data_ptr(),
         PLZ_DT_FP16 if lg.dtype == torch.float16 else PLZ_DT_BF16,
         out.data_ptr(), N, K, _stream(lg.device))
    return out.cpu().numpy().tobytes()


def lut_scalar_bytes(lut: torch.Tensor) -> bytes:
    """(G, 4) palettes -> .lut_scalar bytes, fp16 (palettize_pytorch.py:150-159)."""
    return lut.detach().reshape(-1).to(torch.float16).cpu().numpy().tobytes()


def tensor_entry(name: str, N: int, K: int, idx2: bytes, lut: bytes, **extra) -> dict:
    """A metadata.json tensor entry with the reference's fields (palettize_core.py:120-140)."""
    san = sanitize_name(name)
    entry = {
        "var": name,
        "dense_shape": [N, K],
        "indices_shape": [N, K],
        "bitwidth": BITWIDTH,
        "groups": len(lut) // (PALETTE_SIZE * 2),
        "group_axis": 1,
        "group_size": GROUP_SIZE,
        "nibble_order": "LSB_FIRST",
        "indices_layout": "D0D1",
        "consumer_transpose_y": False,
        "index_file": f"{san}.idx2",
        "lut_file": f"{san}.lut_scalar",
        "sha256_idx": sha256_bytes(idx2),
        "sha256_lut": sha256_bytes(lut),
        "packed_len_bytes": len(idx2),
        "idx_payload_offset_used": 0,
        "lut_payload_offset_used": 0,
    }
    entry.update(extra)
    return entry


def save_tensor(directory: str, name: str, lut: torch.Tensor, packed: torch.Tensor = None,
                logits: torch.Tensor = None, **extra) -> dict:
    """Write <name>.idx2 (from native packed indices, or from the argmax of index logits) and
    <name>.lut_scalar; returns the metadata entry (train_qwen.py:812-844 save_state)."""
    if (packed is None) == (logits is None):
        raise ValueError("give exactly one of packed and logits")
    os.makedirs(directory, exist_ok=True)
    if packed is not None:
        N, K = packed.shape[0], packed.shape[1] * 16
        idx2 = packed_to_idx2(packed)
    else:
        _, K, N = logits.shape
        idx2 = logits_argmax_idx2(logits)
    lut_b = lut_scalar_bytes(lut)
    entry = tensor_entry(name, N, K, idx2, lut_b, **extra)
    with open(os.path.join(directory, entry["index_file"]), "wb") as f:
        f.write(idx2)
    with open(os.path.join(directory, entry["lut_file"]), "wb") as f:
        f.write(lut_b)
    return entry


def write_metadata_json(path: str, entries: dict, teacher_id: str = "qwen35-4b") -> None:
    """metadata.json with the reference's top-level fields (palettize_core.py:143-156,
    palettize_pytorch.py:162-181)."""
    meta = {"tensors": dict(entries), "default_group_size": GROUP_SIZE,
            "teacher_id": teacher_id, "bitwidth": BITWIDTH}
    with open(path, "w") as f:
        json.dump(meta, f, indent=2)
