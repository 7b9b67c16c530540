"""The no-allocation entry point (moefp8_run_noalloc, static 64 MiB scratch per device) against
moefp8_run on the same inputs, through the C ABI: bit-identical outputs and routing on two calls
in a row, the second one smaller (T = 150 on the 128-row path, then T = 16 on the small-T path),
and again after the first size, so stale scratch contents from a larger call are never read; and
captured in a HIP graph, every replay equal to moefp8_run.  At
H = 7168, I = 2048 the scratch holds every T <= 226."""
import ctypes

import pytest
import torch

from moe_fp8 import _abi
from moe_fp8 import main as M
from moe_fp8 import workloads as W

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def weights():
    w = W.make_weights(device=DEV, seed=606)
    torch.cuda.synchronize()
    return w


def _call(weights, T, seed, noalloc):
    wl = W.Workload(f"na{T}", T, seed)
    act = W.make_activations(wl, device=DEV)
    logits = act[0].clone()
    logits[: T // 2, :32] += 1.0                 # local work on half of the tokens
    dbg = {}
    lib, args, out, ws, ws_bytes, keep = M._prepare(logits, *act[1:], *weights, 0, W.RSF, debug=dbg)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    if noalloc:
        rc = lib.moefp8_run_noalloc(ctypes.byref(args), stream)
    else:
        rc = lib.moefp8_run(ctypes.byref(args), ws.data_ptr(), ws_bytes, stream)
    _abi.check(lib, rc)
    torch.cuda.synchronize()
    return out, dbg


@pytest.mark.parametrize("sizes", [((150, 41), (16, 42), (150, 41))])
def test_noalloc_matches_run(weights, sizes):
    for T, seed in sizes:
        print(f"[noalloc] T={T} seed={seed}", flush=True)
        ref, dref = _call(weights, T, seed, noalloc=False)
        got, dgot = _call(weights, T, seed, noalloc=True)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"T={T}: output differs"
        for k in ("topk_ids", "topk_weights", "expert_offsets"):
            assert torch.equal(dgot[k], dref[k]), f"T={T}: {k} differs"
        P = int(dref["expert_offsets"][-1])
        assert torch.equal(dgot["permuted_tokens"][:P], dref["permuted_tokens"][:P])
        assert P > 0 and float(ref.float().abs().max()) > 0.0


def test_noalloc_rejects_large_sizes(weights):
    wl = W.Workload("na_big", 2048, 7)
    act = W.make_activations(wl, device=DEV)
    lib, args, out, ws, ws_bytes, keep = M._prepare(*act, *weights, 0, W.RSF)
    rc = lib.moefp8_run_noalloc(ctypes.byref(args), torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == -8


def test_noalloc_under_graph_capture(weights):
    """The callers the entry point is for: captured in a HIP graph (no allocation during capture),
    every replay gives moefp8_run's output bit for bit, with eager calls on the same static
    scratch between the replays."""
    T = 16
    print(f"[noalloc] graph capture T={T}", flush=True)
    ref, _ = _call(weights, T, 43, noalloc=False)
    wl = W.Workload(f"na{T}", T, 43)
    act = W.make_activations(wl, device=DEV)
    logits = act[0].clone()
    logits[: T // 2, :32] += 1.0
    lib, args, out, ws, ws_bytes, keep = M._prepare(logits, *act[1:], *weights, 0, W.RSF)
    _abi.check(lib, lib.moefp8_run_noalloc(ctypes.byref(args), torch.cuda.current_stream(DEV).cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.moefp8_run_noalloc(ctypes.byref(args), torch.cuda.current_stream(DEV).cuda_stream)
    _abi.check(lib, rc)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        _call(weights, 150, 41, noalloc=True)     # an eager call of another size on the same scratch
