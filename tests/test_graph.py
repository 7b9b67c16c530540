"""The operator captured in a HIP graph (torch.cuda.CUDAGraph), as a serving loop captures its decode
step: every replay must give the eager call's output bit for bit.

The call holds no memset and no host synchronisation: its counters and flags are cleared by its own
kernels, so a replay starts from the same state as an eager call.  Each case replays the graph
several times with eager work and synchronisations between the replays, and once more after new
inputs were written into the captured input buffers (a replay reads whatever they hold).
"""
import pytest
import torch

from moe_fp8 import _abi
from moe_fp8 import workloads as W
from moe_fp8.main import Runner

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def inputs(T, E_local, H, I, seed):
    wl = W.Workload(f"graph_t{T}", T, seed)
    logits, bias, hs, hss = W.make_activations(wl, device="cpu", H=H)
    return [logits.to(DEV), bias.to(DEV), hs.to(DEV), hss.to(DEV)]


# (T, E_local, H, I, path): the decode, grouped 16*MT-row and 128-row paths, and the headline
# decode size at full width
CASES = [(48, 16, 512, 256, _abi.PATH_SMALL_T), (100, 16, 512, 256, _abi.PATH_GROUPED),
         (400, 16, 512, 256, _abi.PATH_ROWS128), (16, 32, 7168, 2048, _abi.PATH_SMALL_T)]


@pytest.mark.parametrize("T,E_local,H,I,path", CASES)
def test_graph_replays_match_eager(T, E_local, H, I, path):
    print(f"[graph] T={T} E_local={E_local} H={H} I={I}", flush=True)
    lib = _abi.load()
    assert lib.moefp8_path(T, E_local, H, I) == path
    act = inputs(T, E_local, H, I, 8100 + T)
    weights = W.make_weights(E_local, H, I, device=DEV, seed=81)
    runner = Runner(*act, *weights, 0, W.RSF)
    runner()
    torch.cuda.synchronize()
    eager = runner.out.clone()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        runner()
    torch.cuda.synchronize()
    for rep in range(3):
        runner.out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(runner.out.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
        runner()                       # eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(runner.out.view(torch.int16), eager.view(torch.int16)), f"eager after replay {rep}"

    # new routing logits and hidden states in the captured buffers: the replay follows them
    fresh = inputs(T, E_local, H, I, 8200 + T)
    for dst, src in zip(act, fresh):
        dst.copy_(src)
    runner()
    torch.cuda.synchronize()
    eager2 = runner.out.clone()
    assert not torch.equal(eager2.view(torch.int16), eager.view(torch.int16))
    runner.out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(runner.out.view(torch.int16), eager2.view(torch.int16)), "replay on new inputs"
