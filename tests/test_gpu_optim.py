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
