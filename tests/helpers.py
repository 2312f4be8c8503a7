"""Shared input generators and metrics for the parity tests."""
import numpy as np
import torch

# Parity bar for floating-point outputs: max-rel-err and cosine
# against an fp32-or-better accumulated reference. The oracle computes in fp64.
MAX_REL = 1e-2
MIN_COS = 0.9999


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))


def assert_close(a, b, max_rel=MAX_REL, min_cos=MIN_COS, what=""):
    r, c = rel_err(a, b), cosine(a, b)
    assert r <= max_rel and c >= min_cos, f"{what}: max-rel-err {r:.3e} cosine {c:.8f}"


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def make_weight(N, K, seed=0, std=0.02):
    """Uniform 2-bit indices [N, K] (uint8) and sorted fp32 palettes [N, K/256, 4] ~N(0, std)."""
    g = gen(seed)
    idx = torch.randint(0, 4, (N, K), generator=g, dtype=torch.uint8)
    pal = torch.sort(torch.randn(N, K // 256, 4, generator=g) * std, dim=-1).values
    return idx, pal.contiguous()


def randn_bf16(*shape, seed=0, std=1.0):
    return (torch.randn(*shape, generator=gen(seed)) * std).to(torch.bfloat16)
