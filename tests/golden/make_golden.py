"""Write the golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

The reference ships no golden vectors for this operator (its parity harness
draws inputs at run time, tools/moe_parity.py:72, 121), so the fixtures here are
computed by an implementation written independently of oracle/moe_oracle.py:

* routing: torch.topk restatement of solutions/moe_fp8/main.py:139-165 on the
  canonical sigmoid (fp64 evaluation rounded to fp32); top-k ties cannot occur
  in these draws (checked below), so torch.topk's unspecified tie order does not
  matter; the normaliser is summed in ascending expert id order in fp32;
* output: a dense fp64 formulation -- every local expert applied to every
  token, weighted by the dense [T, 256] routing weights -- instead of the
  reference's per-expert gather / index_add_ loop (main.py:216-243).

Inputs are tiny (reduced H / I; routing at the real 256 experts) so the fixture
files stay small.  Each .npz holds the inputs and the expected outputs.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
BLOCK = 128


def sigmoid_canonical(x: torch.Tensor) -> torch.Tensor:
    return torch.sigmoid(x.double()).float()


def route_topk(logits: torch.Tensor, bias: torch.Tensor, rsf: float):
    T = logits.shape[0]
    s = sigmoid_canonical(logits)
    sb = s + bias.float()
    grp = sb.view(T, 8, 32)
    top2 = torch.topk(grp, k=2, dim=2).values
    gscore = top2[:, :, 0] + top2[:, :, 1]
    gs_sorted = torch.sort(gscore, dim=1, descending=True).values
    assert not torch.any(gs_sorted[:, 3] == gs_sorted[:, 4]), "group-score tie at the top-4 boundary"
    gidx = torch.topk(gscore, k=4, dim=1).indices
    gmask = torch.zeros(T, 8).scatter_(1, gidx, 1.0).repeat_interleave(32, dim=1)
    pruned = sb.masked_fill(gmask == 0, torch.finfo(torch.float32).min)
    ps = torch.sort(pruned, dim=1, descending=True).values
    assert not torch.any(ps[:, 7] == ps[:, 8]), "expert tie at the top-8 boundary"
    ids = torch.topk(pruned, k=8, dim=1).indices.sort(dim=1).values
    s_sel = torch.gather(s, 1, ids)
    acc = s_sel[:, 0].clone()
    for j in range(1, 8):
        acc = acc + s_sel[:, j]
    w = (s_sel / (acc + 1e-20)[:, None]) * float(np.float32(rsf))
    return ids.to(torch.int32), w.float()


def dense_forward_fp64(logits, bias, hs_codes, hss, w13c, s13, w2c, s2, offset, rsf):
    T = logits.shape[0]
    ids, w = route_topk(logits, bias, rsf)
    dense = torch.zeros(T, 256, dtype=torch.float64)
    dense.scatter_(1, ids.long(), w.double())
    f8 = torch.float8_e4m3fn
    A = hs_codes.view(f8).double() * hss.double().t().repeat_interleave(BLOCK, dim=1)
    E_local = w13c.shape[0]
    I = w13c.shape[1] // 2
    out = torch.zeros(T, A.shape[1], dtype=torch.float64)
    for le in range(E_local):
        ge = offset + le
        if not 0 <= ge < 256:
            continue
        W13 = w13c[le].view(f8).double() * s13[le].double().repeat_interleave(BLOCK, 0).repeat_interleave(BLOCK, 1)
        W2 = w2c[le].view(f8).double() * s2[le].double().repeat_interleave(BLOCK, 0).repeat_interleave(BLOCK, 1)
        G1 = A @ W13.t()
        C = torch.nn.functional.silu(G1[:, I:]) * G1[:, :I]
        out += dense[:, ge:ge + 1] * (C @ W2.t())
    return ids, w, out


def quant_rows(x):
    T, H = x.shape
    xb = x.view(T, H // BLOCK, BLOCK)
    amax = xb.abs().amax(2)
    sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (xb / sc[..., None]).to(torch.float8_e4m3fn).view(T, H)
    return q.view(torch.uint8), sc.t().contiguous()


def quant_blocks(w):
    R, C = w.shape
    wb = w.view(R // BLOCK, BLOCK, C // BLOCK, BLOCK)
    amax = wb.abs().amax(dim=(1, 3))
    sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wb / sc[:, None, :, None]).to(torch.float8_e4m3fn).view(R, C)
    return q.view(torch.uint8), sc


def make_case(name, seed, T, E_local, H, I, offset, rsf, local_boost):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, 256, generator=g)
    lo, hi = max(offset, 0), min(offset + E_local, 256)
    if hi > lo:
        logits[: T // 2, lo:hi] += local_boost          # half the tokens lean towards local experts
    bias = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16)
    hs, hss = quant_rows(torch.randn(T, H, generator=g))
    # weight std scaled so the reduced shapes keep the full operator's activation sizes
    # (0.02 * sqrt(7168) for G1, 0.02 * sqrt(2048) for GEMM2's gain)
    std13, std2 = 0.02 * (7168 / H) ** 0.5, 0.02 * (2048 / I) ** 0.5
    w13 = [quant_blocks(torch.randn(2 * I, H, generator=g) * std13) for _ in range(E_local)]
    w2 = [quant_blocks(torch.randn(H, I, generator=g) * std2) for _ in range(E_local)]
    w13c = torch.stack([q for q, _ in w13]); s13 = torch.stack([s for _, s in w13])
    w2c = torch.stack([q for q, _ in w2]); s2 = torch.stack([s for _, s in w2])
    ids, w, out = dense_forward_fp64(logits, bias, hs, hss, w13c, s13, w2c, s2, offset, rsf)
    np.savez_compressed(
        HERE / f"{name}.npz",
        logits=logits.numpy(), bias_bf16_bits=bias.view(torch.int16).numpy(), hidden=hs.numpy(),
        hidden_scale=hss.numpy(), w13=w13c.numpy(), s13=s13.numpy(), w2=w2c.numpy(), s2=s2.numpy(),
        offset=np.int32(offset), rsf=np.float32(rsf), topk_ids=ids.numpy(), topk_w=w.numpy(),
        out_fp64=out.numpy())
    print(f"{name}: T={T} E_local={E_local} H={H} I={I} offset={offset}")


def make_routing_case(name, seed, T, rsf):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, 256, generator=g)
    bias = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16)
    ids, w = route_topk(logits, bias, rsf)
    np.savez_compressed(HERE / f"{name}.npz", logits=logits.numpy(), bias_bf16_bits=bias.view(torch.int16).numpy(),
                        rsf=np.float32(rsf), topk_ids=ids.numpy(), topk_w=w.numpy())
    print(f"{name}: routing T={T}")


def main():
    make_routing_case("route_t300_s1", 1, 300, 2.5)
    make_routing_case("route_t64_s2_rsf1", 2, 64, 1.0)
    make_case("moe_t24_e4_h256_i128_off0", 3, 24, 4, 256, 128, 0, 2.5, 2.0)
    make_case("moe_t40_e6_h384_i256_off252", 4, 40, 6, 384, 256, 252, 2.5, 2.0)
    return 0


if __name__ == "__main__":
    sys.exit(main())
