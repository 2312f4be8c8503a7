"""GPU parity of the fused optimizer step (plz_adamw_step) against the oracle's fp64
clip + AdamW + clamp, over several steps, mixed bf16/fp32 parameters and both clip groups."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import f32

pytestmark = pytest.mark.gpu
optim = pytest.importorskip("palettize_hip.optim")


def test_fused_adamw_matches_oracle(dev):
    rng = np.random.default_rng(5)
    specs = [((4, 2048 * 3 + 5), torch.bfloat16, 0), ((33,), torch.bfloat16, 0),
             ((9, 7), torch.float32, 1), ((2049,), torch.bfloat16, 1), ((0,), torch.float32, 1)]
    lrs = {0: 1e-2, 1: 3e-4}
    params = [torch.tensor(rng.standard_normal(s) * 0.02, dtype=dt, device=dev).requires_grad_(True)
              for s, dt, _ in specs]
    groups = [{"params": [p for p, (_, _, g) in zip(params, specs) if g == G], "lr": lrs[G],
               "clip_group": G} for G in (0, 1)]
    opt = optim.FusedAdamW(groups)
    order = [i for G in (0, 1) for i, (_, _, g) in enumerate(specs) if g == G]
    masters = [params[i].detach().double().cpu().numpy() for i in order]
    ms = [np.zeros_like(m) for m in masters]
    vs = [np.zeros_like(m) for m in masters]
    cg = [specs[i][2] for i in order]
    for step in range(1, 5):
        tau = 1.0 / step
        opt.set_clamp(0, -0.05 * tau, 0.05 * tau)
        grads = []
        for j, i in enumerate(order):
            g = torch.tensor(rng.standard_normal(specs[i][0]) * (2.0 if step == 3 else 0.01),
                             dtype=specs[i][1])
            params[i].grad = g.to(dev)
            grads.append(g.double().numpy())
        norms = opt.step(max_norms=(1.0, 0.3))
        clamps = [(-0.05 * tau, 0.05 * tau) if c == 0 else (-np.inf, np.inf) for c in cg]
        want_norms = O.adamw_step(masters, grads, ms, vs, [lrs[c] for c in cg], cg, (1.0, 0.3),
                                  clamps, step)
        assert np.allclose(f32(norms), want_norms, rtol=1e-5)
        for j, i in enumerate(order):
            got = f32(params[i])
            want = masters[j]
            if specs[i][1] == torch.bfloat16:  # bf16 param = round(master): one bf16 ulp
                assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-9), (i, step)
            else:
                assert np.allclose(got, want, rtol=1e-5, atol=1e-8), (i, step)
            if specs[i][1] == torch.bfloat16:
                m32 = next(e[1] for e in opt.entries if e[0] is params[i])
                assert np.allclose(f32(m32), want, rtol=1e-5, atol=1e-8), (i, step)


def test_fused_adamw_takes_the_producers_squared_sums(dev):
    """grad_sq: the clip norm of a parameter read from one fp32 sum per 512 gradient elements
    (what the soft backward writes) instead of from the gradient: the same norms (summation
    order aside) and, with the clip active, the same update to fp32 rounding; sums that do not
    cover the parameter are refused."""
    rng = np.random.default_rng(7)
    shape = (12, 256, 4)  # 12288 elements: one full block of 8192 and a partial one
    base = torch.tensor(rng.standard_normal(shape) * 0.02, dtype=torch.bfloat16)
    grad = torch.tensor(rng.standard_normal(shape) * 0.5, dtype=torch.bfloat16)
    other = torch.tensor(rng.standard_normal((300,)) * 0.02, dtype=torch.float32)
    results = []
    for use_sq in (False, True):
        p = base.clone().to(dev).requires_grad_(True)
        q = other.clone().to(dev).requires_grad_(True)
        opt = optim.FusedAdamW([{"params": [p], "lr": 1e-2, "clip_group": 0},
                                {"params": [q], "lr": 1e-3, "clip_group": 1}])
        p.grad = grad.to(dev)
        q.grad = torch.ones(300, device=dev)
        sq = None
        if use_sq:
            sq = {id(p): (p.grad.float() ** 2).reshape(-1, 512).sum(1).contiguous()}
        norms = opt.step(max_norms=(1.0, 0.3), grad_sq=sq)
        results.append((f32(norms), f32(p), f32(q)))
    (n0, p0, q0), (n1, p1, q1) = results
    assert np.allclose(n0, n1, rtol=1e-5) and n0[0] > 1.0  # the clip is active
    assert np.allclose(p0, p1, rtol=2.0 ** -7, atol=1e-6) and np.array_equal(q0, q1)
    p = base.clone().to(dev).requires_grad_(True)
    opt = optim.FusedAdamW([{"params": [p], "lr": 1e-2, "clip_group": 0}])
    p.grad = grad.to(dev)
    with pytest.raises(ValueError, match="512"):
        opt.step(grad_sq={id(p): torch.zeros(5, device=dev)})
