"""Writes the on-disk-format fixtures from the reference's own palettized files.

Run in a checkout that has the reference next to it (REF, default /root/reference):
    python tests/golden/make_golden.py
It copies data only: a 256-row slice of one real .idx2 file (the first 256 k-rows of the
(K, N) index matrix), the complete .lut_scalar and metadata entry of that tensor, and the
top-level metadata fields. Expected decodings are not stored; the tests derive them with the
oracle, whose unpacking is pinned by the reference's known-answer bytes.
"""
import json
import os
import sys

import numpy as np

REF = os.environ.get("REF", "/root/reference")
SRC = os.path.join(REF, "palettized", "superblock_0")
NAME = "model.layers.3.self_attn.k_proj.weight"
K_ROWS = 256


def main():
    meta = json.load(open(os.path.join(SRC, "metadata.json")))
    entry = meta["tensors"][NAME]
    N, K = entry["dense_shape"]
    idx = open(os.path.join(SRC, entry["index_file"]), "rb").read()
    lut = open(os.path.join(SRC, entry["lut_file"]), "rb").read()
    out = os.path.dirname(os.path.abspath(__file__))
    np.savez_compressed(
        os.path.join(out, "palettized_k_proj_slice.npz"),
        idx2_slice=np.frombuffer(idx[: K_ROWS * N // 4], dtype=np.uint8),
        lut_scalar=np.frombuffer(lut, dtype=np.uint8))
    top = {k: v for k, v in meta.items() if k != "tensors"}
    with open(os.path.join(out, "palettized_k_proj_meta.json"), "w") as f:
        json.dump({"top": top, "name": NAME, "entry": entry, "k_rows": K_ROWS}, f, indent=2)
    print("wrote fixtures for", NAME, N, K, file=sys.stderr)


if __name__ == "__main__":
    main()
