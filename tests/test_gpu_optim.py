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


@pytest.mark.parametrize("N,K", [(3, 256), (40, 768), (9, 2560)])
def test_step_build_matches_a_separate_build(dev, N, K):
    """FusedAdamW.step(build=NextBuild(...)): the soft weight and P written by the update pass,
    for logits whose element count is or is not a multiple of the update's 8192-element blocks,
    with a palette updated in the same step and a non-zero noise counter base, equal the batched
    build of the updated logits (plz_soft_build_w_batched_philox) bit for bit; the parameters
    equal those of the same step without the build."""
    ops = pytest.importorskip("palettize_hip.ops")
    from palettize_hip import _lib
    rng = np.random.default_rng(N * K)
    logits0 = torch.tensor(rng.standard_normal((N, K, 4)) * 2, dtype=torch.bfloat16)
    pal0 = torch.tensor(np.sort(rng.standard_normal((N, K // 256, 4)) * 0.02, -1),
                        dtype=torch.float32)
    glog = torch.tensor(rng.standard_normal((N, K, 4)), dtype=torch.bfloat16)
    gpal = torch.tensor(rng.standard_normal((N, K // 256, 4)) * 0.1, dtype=torch.float32)
    seed, counter, offset, tau = 77, 5 * K, 123456, 0.75
    outs = []
    for with_build in (False, True):
        lg = logits0.clone().to(dev).requires_grad_(True)
        pal = pal0.clone().to(dev).requires_grad_(True)
        opt = optim.FusedAdamW([{"params": [pal], "lr": 1e-2, "clip_group": 1},
                                {"params": [lg], "lr": 0.5, "clip_group": 0,
                                 "clamp": (-3.0, 3.0)}])
        lg.grad, pal.grad = glog.to(dev), gpal.to(dev)
        w = torch.zeros(N, K, dtype=torch.bfloat16, device=dev)
        pr = torch.zeros(N, K, 4, dtype=torch.float16, device=dev)
        nb = (optim.NextBuild([(lg, pal, w, seed, counter, pr)], offset, tau) if with_build
              else None)
        opt.step(max_norms=(1.0, 0.3), build=nb)
        if with_build:
            assert nb.built == {id(lg)}
        outs.append((lg.detach().clone(), pal.detach().clone(), w, pr))
    (lg_a, pal_a, _, _), (lg_b, pal_b, w_b, pr_b) = outs
    assert torch.equal(lg_a.view(torch.int16), lg_b.view(torch.int16)) and torch.equal(pal_a, pal_b)
    grp = ops.SoftBuildGroup([(lg_b, ops.PhiloxNoise(seed, 0), pal_b)], _lib.PLZ_W_HARD_NOISY,
                             want_probs=True)
    (w_ref, _), = grp.run(tau, offset + counter)
    assert torch.equal(w_b.view(torch.int16), w_ref.view(torch.int16))
    assert torch.equal(pr_b.view(torch.int16), grp.probs[0].view(torch.int16))
