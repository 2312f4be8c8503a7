"""CPU: a debug host build (asserts on) of the MFMA GEMM's work-item index math, checked over
many shapes and CU counts for every launch the entry points make (tests/native/
gemm_item_check.hip includes the same header the kernels use)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_gemm_item_map_covers_every_tile_split_and_part_once(tmp_path):
    exe = tmp_path / "gemm_item_check"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17",
           "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "qwen-palettize_amd", "csrc"),
           os.path.join(ROOT, "tests", "native", "gemm_item_check.hip"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert "checks passed" in r.stdout
