"""Seeded synthetic inputs for the fp8 block-scale MoE operator.

The generators follow the contest's input contract (``solutions/moe_fp8/main.py:173-187``,
``tools/moe_parity.py:124-132``): fp32 routing logits ``[T, 256]``, bf16 routing
bias ``[256]``, e4m3fn hidden states ``[T, H]`` with fp32 per-token 1x128 scales
stored transposed ``[H/128, T]``, e4m3fn gate/up weights ``[E, 2I, H]`` and down
weights ``[E, H, I]`` with fp32 128x128 block scales ``[E, 2I/128, H/128]`` and
``[E, H/128, I/128]``.  Quantisation is ``scale = amax / 448`` per block (amax 0
-> scale 1) and ``q = e4m3(x / scale)`` with round-to-nearest-even.

Named workloads (T tokens, 32 local experts at offset 0, H=7168, I=2048,
routed scaling 2.5):

* ``plumbing``  T=16, seed 0.
* ``decode``    T in {1, 4, 16, 64}, seed 100+T.  At T = 1 and 4 these seeds route no token to
  local experts 0-31 (routing plus the zero output only), so
* ``decode_t1_local`` / ``decode_t4_local`` take the first seed 100+T+k (k >= 1) whose routing
  gives local work: seed 102 (1 pair, 1 active expert) and seed 105 (2 pairs, 2 experts).
* ``prefill``   T=1024, seed 1024.
* ``large``     T=8192, seed 8192; per-token hidden amplitude exp(z), z~N(0,1).
* ``skewed``    T=5000, seed 5000; Zipf(s=1.2) expert popularity over a seeded
  permutation of the 256 experts, added as centred log-probabilities to the
  logits.

Weights use their own seed (``WEIGHT_SEED``) so one weight set serves every
workload of a process.  Draw order: logits, bias, hidden, then (separately)
W13 expert by expert, W2 expert by expert.
"""
from __future__ import annotations

import dataclasses
import math

import torch

H_FULL = 7168
I_FULL = 2048
E_LOCAL_FULL = 32
E_GLOBAL = 256
BLOCK = 128
WEIGHT_SEED = 4242
RSF = 2.5


@dataclasses.dataclass
class Workload:
    name: str
    T: int
    seed: int
    hidden_dist: str = "normal"      # "normal" | "lognormal"
    routing: str = "normal"          # "normal" | "zipf"


def workloads():
    """The named synthetic workloads, keyed by label."""
    w = {"plumbing_t16": Workload("plumbing_t16", 16, 0)}
    for T in (1, 4, 16, 64):
        w[f"decode_t{T}"] = Workload(f"decode_t{T}", T, 100 + T)
    w["decode_t1_local"] = Workload("decode_t1_local", 1, 102)
    w["decode_t4_local"] = Workload("decode_t4_local", 4, 105)
    w["prefill_t1024"] = Workload("prefill_t1024", 1024, 1024)
    w["large_t8192"] = Workload("large_t8192", 8192, 8192, hidden_dist="lognormal")
    w["skewed_t5000"] = Workload("skewed_t5000", 5000, 5000, routing="zipf")
    return w


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def quantize_rows_1x128(x: torch.Tensor):
    """[T, H] float -> (e4m3fn [T, H], fp32 scale [H/128, T])."""
    T, H = x.shape
    xb = x.float().view(T, H // BLOCK, BLOCK)
    amax = xb.abs().amax(dim=2)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (xb / scale.unsqueeze(-1)).to(torch.float8_e4m3fn).view(T, H)
    return q, scale.t().contiguous()


def quantize_blocks_128x128(w: torch.Tensor):
    """[R, C] float -> (e4m3fn [R, C], fp32 scale [R/128, C/128])."""
    R, C = w.shape
    wb = w.float().view(R // BLOCK, BLOCK, C // BLOCK, BLOCK)
    amax = wb.abs().amax(dim=(1, 3))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wb / scale[:, None, :, None]).to(torch.float8_e4m3fn).view(R, C)
    return q, scale.contiguous()


def zipf_logit_bias(n_experts: int, s: float, perm: torch.Tensor) -> torch.Tensor:
    """Centred log-popularity: expert perm[r] gets log p_r, p_r ~ (r+1)^-s."""
    r = torch.arange(1, n_experts + 1, dtype=torch.float64)
    logp = -s * torch.log(r)
    logp = logp - torch.logsumexp(logp, 0)
    logp = logp - logp.mean()
    out = torch.empty(n_experts, dtype=torch.float64)
    out[perm] = logp
    return out.float()


def make_activations(wl: Workload, device="cpu", H=H_FULL):
    """Routing logits, routing bias and quantised hidden states for one workload.

    Always drawn with the CPU generator (then moved to ``device``), so a workload
    has the same values -- and the same routing -- on every device."""
    g = _gen("cpu", wl.seed)
    T = wl.T
    logits = torch.randn(T, E_GLOBAL, generator=g, dtype=torch.float32)
    bias = (torch.randn(E_GLOBAL, generator=g) * 0.1).to(torch.bfloat16)
    hidden = torch.randn(T, H, generator=g, dtype=torch.float32)
    if wl.hidden_dist == "lognormal":
        z = torch.randn(T, 1, generator=g, dtype=torch.float32)
        hidden = hidden * torch.exp(z)
    if wl.routing == "zipf":
        gp = torch.Generator(device="cpu")
        gp.manual_seed(wl.seed + 1)
        perm = torch.randperm(E_GLOBAL, generator=gp)
        logits = logits + zipf_logit_bias(E_GLOBAL, 1.2, perm)
    hs, hss = quantize_rows_1x128(hidden)
    del hidden
    return tuple(x.to(device) for x in (logits, bias, hs, hss))


def reduced_std(H, I):
    """Weight std for reduced test shapes that keeps the full operator's activation
    magnitudes: 0.02 at H=7168 / I=2048, scaled by sqrt(7168/H) and sqrt(2048/I)."""
    return 0.02 * (H_FULL / H) ** 0.5, 0.02 * (I_FULL / I) ** 0.5


def make_weights(E_local=E_LOCAL_FULL, H=H_FULL, I=I_FULL, device="cpu", seed=WEIGHT_SEED, std=None):
    """N(0, std) gate/up and down weights, quantised per 128x128 block, expert by expert.
    ``std`` is a (gate/up, down) pair; the default is ``reduced_std(H, I)`` (0.02 at full size)."""
    std13, std2 = std if std is not None else reduced_std(H, I)
    g = _gen(device, seed)
    w13 = torch.empty(E_local, 2 * I, H, dtype=torch.float8_e4m3fn, device=device)
    s13 = torch.empty(E_local, 2 * I // BLOCK, H // BLOCK, dtype=torch.float32, device=device)
    w2 = torch.empty(E_local, H, I, dtype=torch.float8_e4m3fn, device=device)
    s2 = torch.empty(E_local, H // BLOCK, I // BLOCK, dtype=torch.float32, device=device)
    for e in range(E_local):
        q, s = quantize_blocks_128x128(torch.randn(2 * I, H, generator=g, device=device) * std13)
        w13[e].copy_(q)
        s13[e].copy_(s)
    for e in range(E_local):
        q, s = quantize_blocks_128x128(torch.randn(H, I, generator=g, device=device) * std2)
        w2[e].copy_(q)
        s2[e].copy_(s)
    return w13, s13, w2, s2


def make_inputs(wl: Workload, device="cpu", E_local=E_LOCAL_FULL, H=H_FULL, I=I_FULL,
                weights=None, local_expert_offset=0, rsf=RSF):
    """Full argument tuple for ``run(...)`` in the reference's positional order."""
    logits, bias, hs, hss = make_activations(wl, device=device, H=H)
    if weights is None:
        weights = make_weights(E_local, H, I, device=device)
    w13, s13, w2, s2 = weights
    return (logits, bias, hs, hss, w13, s13, w2, s2, local_expert_offset, rsf)
