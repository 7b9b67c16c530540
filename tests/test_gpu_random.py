"""Seeded random configurations of the full path against the CPU oracle.

Each case draws T (log-uniform 1-3000), E_local, H, I, the local expert offset, how hard
and how many tokens lean towards the local experts, which tokens carry 30-120x hidden
amplitude, and whether shared-expert rows are fused in.  Bars as in the other parity tests:
routing ids / weights and the permutation bit-exact, and every output element within
atol 1e-2 / rtol 2e-2.  An element that misses the bar against the fp32 oracle is
re-evaluated for its single token with fp64 accumulation (the fp32 oracle's own
accumulation order moves outputs that cancel from ~1e4 to ~1e-2 by ~1e-2); the bar then
applies against that value.
"""
import math
import random

import numpy as np
import pytest
import torch

import moe_oracle as O
import moe_fp8
from moe_fp8 import workloads as W

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
ATOL, RTOL = 1e-2, 2e-2
N_CASES = 40


def draw(case):
    rng = random.Random(9000 + case)
    return dict(
        T=max(1, int(math.exp(rng.uniform(0.0, math.log(3000.0))))),
        E=rng.choice([1, 4, 8, 16, 32, 32, 64]),
        H=128 * rng.choice([2, 3, 4, 6, 8, 16]),
        I=128 * rng.choice([1, 2, 3, 4, 8]),
        offset=rng.choice([0, 0, 32 * rng.randrange(8), rng.randrange(-8, 260)]),
        lean=rng.choice([0.0, 1.5, 3.0]),
        lean_frac=rng.choice([0.25, 0.5, 1.0]),
        stride=rng.choice([0, 0, 3, 7, 31]),
        shared=rng.random() < 0.25,
    )


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_configuration(case):
    p = draw(case)
    print(f"[random {case}] {p}", flush=True)
    T, E, H, I, off = p["T"], p["E"], p["H"], p["I"], p["offset"]
    weights = W.make_weights(E, H, I, device="cpu", seed=300 + case)
    args = W.make_inputs(W.Workload(f"rand{case}", T, 5000 + case), device="cpu", E_local=E, H=H, I=I,
                         weights=weights, local_expert_offset=off)
    logits = args[0].clone()
    lo, hi = max(off, 0), min(off + E, 256)
    if hi > lo and p["lean"]:
        logits[: int(T * p["lean_frac"]), lo:hi] += p["lean"]
    hss = args[3].clone()
    if p["stride"]:
        amp = torch.ones(T)
        amp[:: p["stride"]] = torch.linspace(30.0, 120.0, len(amp[:: p["stride"]]))
        hss *= amp[None, :]
    args = (logits,) + args[1:3] + (hss,) + args[4:]
    shared = torch.randn(T, H, generator=torch.Generator().manual_seed(case)) * 0.5 if p["shared"] else None

    dbg = {}
    dev_args = tuple(a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args)
    out = moe_fp8.run(*dev_args, debug=dbg, shared_output=None if shared is None else shared.to(DEV))
    torch.cuda.synchronize()

    ridx, rw, _, _ = O.route(logits.float().numpy(), args[1].float().numpy(), W.RSF)
    _, offsets, ptok, _ = O.permute(ridx, rw, E, off)
    assert np.array_equal(dbg["topk_ids"].cpu().numpy(), ridx)
    assert np.array_equal(dbg["topk_weights"].cpu().numpy().view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(dbg["expert_offsets"].cpu().numpy(), offsets)
    assert np.array_equal(dbg["permuted_tokens"].cpu().numpy()[: offsets[-1]], ptok)

    ref32, _ = O.moe_forward(*args)
    if shared is not None:
        ref32 = ref32 + shared
    got = out.float().cpu()
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H)
    miss = (got - ref32).abs() > ATOL + RTOL * ref32.abs()
    for t, h in torch.nonzero(miss).tolist():
        one = (logits[t:t + 1], args[1], args[2][t:t + 1], hss[:, t:t + 1].contiguous()) + tuple(args[4:])
        o64, _ = O.moe_forward(*one, accumulate=torch.float64)
        exact = float(o64[0, h]) + (float(shared[t, h]) if shared is not None else 0.0)
        print(f"  t={t} h={h}: fp32 oracle {float(ref32[t, h]):.5f}, fp64 {exact:.5f}, HIP {float(got[t, h]):.5f}",
              flush=True)
        assert abs(float(got[t, h]) - exact) <= ATOL + RTOL * abs(exact), (case, t, h)
