"""The named synthetic workloads route as documented (CPU, oracle routing)."""
import numpy as np
import pytest

import moe_oracle as O
from moe_fp8 import workloads as W


def local_work(name):
    wl = W.workloads()[name]
    logits, bias, _, _ = W.make_activations(wl, device="cpu", H=128)
    idx, _, _, _ = O.route(logits.numpy(), bias.float().numpy(), W.RSF)
    loc = idx[idx < W.E_LOCAL_FULL]
    return int(loc.size), len(set(loc.tolist()))


@pytest.mark.parametrize("name,P,A", [("decode_t1", 0, 0), ("decode_t4", 0, 0),
                                      ("decode_t1_local", 1, 1), ("decode_t4_local", 2, 2)])
def test_small_decode_workloads(name, P, A):
    """decode_t1 / decode_t4 (seeds 101 / 104) route no token to local experts 0-31; the _local
    variants take the first later seed 100+T+k with local work."""
    assert local_work(name) == (P, A)


def test_local_seeds_are_the_first_with_local_work():
    for T, seed in ((1, 102), (4, 105)):
        for s in range(100 + T + 1, seed):
            logits, bias, _, _ = W.make_activations(W.Workload("x", T, s), device="cpu", H=128)
            idx, _, _, _ = O.route(logits.numpy(), bias.float().numpy(), W.RSF)
            assert not np.any(idx < W.E_LOCAL_FULL), s
        assert W.workloads()[f"decode_t{T}_local"].seed == seed
