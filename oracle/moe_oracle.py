"""CPU oracle for the DeepSeek-V3 fp8 block-scale MoE operator.

TEST INFRASTRUCTURE ONLY.  This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``moe_fp8.run``) never calls it and fails loudly
when the HIP library is missing.

It restates, on the host in numpy + torch-CPU fp32, the algorithm of the
reference solution ``solutions/moe_fp8/main.py`` of jhinpan/rocm-flashinfer-contest:

* ``decode_e4m3`` / ``E4M3_TABLE``   -- OCP e4m3fn decode used by ``main.py:117``
  and ``main.py:136`` (``.to(torch.float32)`` of float8_e4m3fn).
* ``dequant_hidden``                 -- ``main.py:129-136`` (kept fp32, as the
  contest reference does, not the solution's bf16).
* ``dequant_block``                  -- ``main.py:110-118`` (fp32 result).
* ``route``                          -- ``main.py:139-165`` in canonical form
  (see below).
* ``permute``                        -- selection + ordering of ``main.py:216-226``.
* ``swiglu``                         -- ``main.py:168-170`` (gate = second half).
* ``moe_forward``                    -- ``run`` at ``main.py:173-243`` with fp32
  throughout (GEMM1, SwiGLU, GEMM2, ``index_add_`` combine, bf16 round).
* ``quantize_hidden``                -- the step before the operator: the per-token
  1x128 e4m3 quantization whose output ``main.py:129-136`` dequantizes (the reference
  repository ships no quantizer; the convention is DeepSeek-V3's: scale = amax / 448,
  1 for an all-zero block, q = e4m3fn(x / scale) rounded to nearest even).

Canonical routing arithmetic.  ``torch.topk(sorted=False)`` leaves tie order
and output order unspecified and ``weights.sum(dim=1)`` has an ISA-dependent
association order (``main.py:152,154,160,164``).  The oracle pins them:

* ``s = fp32(1 / (1 + exp(-x)))`` evaluated in fp64, then rounded once to fp32;
* ``sb = fp32(s + fp32(bias))``;
* group score = ``fp32(top1 + top2)`` of ``sb`` inside each group of 32;
* groups and experts are ranked by (value descending, index ascending), so
  the lowest index wins a tie;
* the selected ids are returned in ascending id order, and the normaliser is
  the sequential fp32 sum of ``s`` over them in that order;
* ``w = fp32(fp32(s / fp32(sum + 1e-20)) * fp32(rsf))``.

Pinning status (each item is checked in ``tests/test_oracle.py``):
  decode_e4m3     exhaustive 256-code table vs the closed form and torch's cast;
  route           torch.topk restatement of ``main.py:139-165`` (id sets, weights
                  to 1e-6), brute force over all 70 group subsets, forced-logit
                  cases after ``tools/moe_parity.py:91-98``, invariants, golden
                  fixtures from an independent fp64 implementation;
  permute         brute-force nonzero() per expert (``main.py:222-225``);
  swiglu          closed form + negative check against the interleaved order
                  (``tools/moe_parity.py:108-115``);
  moe_forward     dense fp64 formulation (every expert on every token, masked by
                  the dense routing weights) on reduced shapes, and golden
                  fixtures produced by that formulation;
  quantize_hidden codes vs a brute-force nearest-value encoder over the 256-code
                  table with ties to the even code (so torch's cast is checked,
                  not trusted), scales vs the closed form, round trip of every
                  finite code, the block maximum landing on +-448.
  torch's own sigmoid ulp / sum association / topk tie bits are not pinned
  (the contest's torch reference is not available offline); the canonical
  form above replaces them.
"""
from __future__ import annotations

import math

import numpy as np
import torch

# Operator constants (``main.py:22-29``).
BLOCK = 128
E_GLOBAL = 256
TOP_K = 8
N_GROUP = 8
TOPK_GROUP = 4
GROUP_SIZE = E_GLOBAL // N_GROUP

_F32 = np.float32


def _e4m3_value(code: int) -> float:
    """Closed-form OCP e4m3fn decode: 1 sign, 4 exponent (bias 7), 3 mantissa
    bits; exponent field 0 is subnormal; S.1111.111 is NaN; there is no inf."""
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return float("nan")
    if exp == 0:
        return sign * (man / 8.0) * 2.0 ** (-6)
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


E4M3_TABLE = np.array([_e4m3_value(c) for c in range(256)], dtype=_F32)


def decode_e4m3(codes) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (table lookup)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def _as_codes_t(x) -> torch.Tensor:
    """Accept a float8_e4m3fn tensor, a uint8 tensor or a uint8 ndarray; return uint8 CPU tensor."""
    if isinstance(x, np.ndarray):
        return torch.from_numpy(np.ascontiguousarray(x, dtype=np.uint8))
    x = x.detach().cpu()
    if x.dtype == torch.float8_e4m3fn:
        return x.view(torch.uint8)
    assert x.dtype == torch.uint8, x.dtype
    return x


def _decode_t(codes_u8: torch.Tensor) -> torch.Tensor:
    """Bulk decode through torch's own float8_e4m3fn cast (what main.py:117, 136 use);
    equal to E4M3_TABLE on all 256 codes (tests/test_oracle.py)."""
    return codes_u8.view(torch.float8_e4m3fn).float()


def dequant_hidden(hidden_codes, hidden_scale) -> torch.Tensor:
    """``main.py:129-136`` in fp32: A[t, h] = e4m3(hs[t, h]) * scale[h // 128, t]."""
    q = _decode_t(_as_codes_t(hidden_codes))                       # [T, H]
    sc = torch.as_tensor(np.asarray(hidden_scale, dtype=_F32) if isinstance(hidden_scale, np.ndarray)
                         else hidden_scale.detach().cpu().float())  # [H/128, T]
    T, H = q.shape
    assert sc.shape == (H // BLOCK, T), (sc.shape, H, T)
    return (q.view(T, H // BLOCK, BLOCK) * sc.t().unsqueeze(-1)).reshape(T, H)


def quantize_hidden(x):
    """Per-token 1x128 quantization of ``x [T, H]`` (any float dtype, finite):
    returns ``(codes uint8 [T, H], scale fp32 [H/128, T])`` with, per token and
    128 columns, ``scale = fp32(amax / 448)`` (1 for an all-zero block) and
    ``codes = e4m3fn(fp32(x / scale))`` rounded to nearest even -- the pair that
    ``dequant_hidden`` (``main.py:129-136``) turns back into activations."""
    x32 = torch.as_tensor(x).detach().cpu().float()
    T, H = x32.shape
    xb = x32.view(T, H // BLOCK, BLOCK)
    amax = xb.abs().amax(dim=2)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    codes = (xb / scale.unsqueeze(-1)).to(torch.float8_e4m3fn).view(torch.uint8).reshape(T, H)
    return codes.numpy(), scale.t().contiguous().numpy()


def encode_e4m3_bruteforce(v) -> np.ndarray:
    """Reference encoder for the tests: for each finite fp32 value with |v| <= 464,
    the non-negative e4m3fn code whose value is nearest to |v| (ties to the even
    mantissa, i.e. round to nearest even), with the sign bit of v -- straight from
    the 256-code table."""
    v = np.asarray(v, dtype=np.float64).reshape(-1)
    mags = np.arange(0x7F, dtype=np.int64)            # codes 0x00..0x7E (0x7F is NaN)
    vals = E4M3_TABLE[mags].astype(np.float64)
    out = np.empty(v.shape, dtype=np.uint8)
    for i, x in enumerate(v):
        d = np.abs(vals - abs(x))
        cand = mags[d == d.min()]
        if len(cand) > 1:
            cand = cand[(cand & 1) == 0]
        out[i] = int(cand[0]) | (0x80 if math.copysign(1.0, x) < 0 else 0)
    return out


def dequant_block(w_codes, scale) -> torch.Tensor:
    """``main.py:110-118`` in fp32: W[r, c] = e4m3(w[r, c]) * scale[r // 128, c // 128]."""
    q = _decode_t(_as_codes_t(w_codes))
    sc = scale if isinstance(scale, torch.Tensor) else torch.from_numpy(np.asarray(scale, _F32))
    sc = sc.detach().cpu().float()
    R, C = q.shape
    return (q.view(R // BLOCK, BLOCK, C // BLOCK, BLOCK) * sc[:, None, :, None]).reshape(R, C)


# --------------------------------------------------------------------------- routing

def sigmoid_f32(x) -> np.ndarray:
    """fp32 sigmoid evaluated in fp64 and rounded once (canonical form)."""
    xd = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-xd))).astype(_F32)


def route(logits, bias, routed_scaling_factor):
    """Canonical restatement of ``_route`` (``main.py:139-165``).

    Returns ``(idx [T, 8] int32 ascending, w [T, 8] float32, s [T,256] f32,
    sb [T,256] f32)``.  ``w[t, j]`` is the reference's dense ``weights[t, idx[t, j]]``.
    """
    lg = np.asarray(logits, dtype=_F32)
    T, E = lg.shape
    assert E == E_GLOBAL
    b = np.asarray(bias, dtype=_F32).reshape(E_GLOBAL)
    s = sigmoid_f32(lg)
    sb = (s + b).astype(_F32)                                     # main.py:148

    # per-group top-2 sum (main.py:151-153); the values, not their order, matter
    g = np.sort(sb.reshape(T, N_GROUP, GROUP_SIZE), axis=2)
    gscore = (g[:, :, -1] + g[:, :, -2]).astype(_F32)             # [T, 8]

    # top-4 groups by (score desc, group asc) (main.py:154-156)
    gi = np.arange(N_GROUP)
    beats = (gscore[:, None, :] > gscore[:, :, None]) | (
        (gscore[:, None, :] == gscore[:, :, None]) & (gi[None, None, :] < gi[None, :, None]))
    grank = beats.sum(axis=2)                                     # [T, 8]
    keep = grank < TOPK_GROUP
    emask = np.repeat(keep, GROUP_SIZE, axis=1)                   # [T, 256]

    # top-8 experts among kept groups by (sb desc, id asc) (main.py:158-160)
    key = np.where(emask, -sb.astype(np.float64), np.inf)
    order = np.argsort(key, axis=1, kind="stable")[:, :TOP_K]
    idx = np.sort(order, axis=1).astype(np.int32)                 # ascending ids

    # normalised weights from the unbiased s (main.py:162-164)
    s_sel = np.take_along_axis(s, idx.astype(np.int64), axis=1)   # [T, 8]
    acc = s_sel[:, 0].copy()
    for j in range(1, TOP_K):
        acc = (acc + s_sel[:, j]).astype(_F32)
    denom = (acc + _F32(1e-20)).astype(_F32)
    w = ((s_sel / denom[:, None]).astype(_F32) * _F32(routed_scaling_factor)).astype(_F32)
    return idx, w, s, sb


def dense_weights(idx, w, T) -> np.ndarray:
    """Scatter the compact [T, 8] weights back to the reference's dense [T, 256] form."""
    out = np.zeros((T, E_GLOBAL), dtype=_F32)
    np.put_along_axis(out, np.asarray(idx, dtype=np.int64), np.asarray(w, dtype=_F32), axis=1)
    return out


# --------------------------------------------------------------------------- permutation

def permute(idx, w, E_local: int, local_expert_offset: int):
    """Selection + ordering of ``main.py:216-226``: for local expert le = 0..E_local-1
    (global id ge = offset + le, skipped outside [0, 256)), the tokens that picked
    ge in ascending token order.

    Returns ``counts [E_local] int32, offsets [E_local+1] int32, perm_token [P] int32,
    perm_w [P] float32`` (perm_w[p] = routing weight of that (token, expert) pair).
    """
    idx = np.asarray(idx, dtype=np.int64)
    w = np.asarray(w, dtype=_F32)
    T = idx.shape[0]
    le = idx - int(local_expert_offset)                            # [T, 8]
    valid = (le >= 0) & (le < E_local) & (idx >= 0) & (idx < E_GLOBAL)
    tok = np.broadcast_to(np.arange(T)[:, None], idx.shape)
    le_v, tok_v, w_v = le[valid], tok[valid], w[valid]
    order = np.lexsort((tok_v, le_v))                              # expert major, token minor
    counts = np.bincount(le_v, minlength=E_local).astype(np.int32)[:E_local]
    offsets = np.zeros(E_local + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return counts, offsets, tok_v[order].astype(np.int32), w_v[order].astype(_F32)


# --------------------------------------------------------------------------- expert FFN

def swiglu(G1: torch.Tensor) -> torch.Tensor:
    """``main.py:168-170``: C = silu(G1[:, I:]) * G1[:, :I] in G1's dtype, fp32 as in the
    reference (gate = second half)."""
    I = G1.shape[1] // 2
    return torch.nn.functional.silu(G1[:, I:]) * G1[:, :I]


def moe_forward(routing_logits, routing_bias, hidden_states, hidden_states_scale,
                gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
                local_expert_offset, routed_scaling_factor, dequant_all_upfront=False,
                return_intermediates=False, accumulate=torch.float32):
    """fp32 restatement of ``run`` (``main.py:173-243``).

    Every tensor argument may be a torch tensor (any device) or an ndarray; fp8
    tensors may be float8_e4m3fn or raw uint8.  Returns the fp32 output before the
    final bf16 rounding and the bf16 output (``main.py:243``).  With
    ``dequant_all_upfront`` it dequantises all local experts to fp32 before the
    loop, as the contest's torch reference does (``main.py:7-8``); the result is
    identical, only the cost differs.

    ``accumulate=torch.float64`` keeps the fp32 dequantisation (``main.py:117,136``)
    and runs GEMM1, SwiGLU, GEMM2 and the combine in fp64: an arbiter for outputs
    whose pairs cancel (rows of ~1e4 summing to ~1e-2), where fp32 accumulation
    order alone moves the result by ~1e-2.
    """
    def f32(x):
        if isinstance(x, torch.Tensor):
            return x.detach().cpu().float().numpy()
        return np.asarray(x, dtype=_F32)

    if isinstance(local_expert_offset, torch.Tensor):
        local_expert_offset = int(local_expert_offset.item())
    if isinstance(routed_scaling_factor, torch.Tensor):
        routed_scaling_factor = float(routed_scaling_factor.item())
    local_start = int(local_expert_offset)

    logits = f32(routing_logits)
    T = logits.shape[0]
    w13c = _as_codes_t(gemm1_weights)
    w2c = _as_codes_t(gemm2_weights)
    E_local, two_I, H = w13c.shape
    I = two_I // 2
    s13 = torch.from_numpy(f32(gemm1_weights_scale))
    s2 = torch.from_numpy(f32(gemm2_weights_scale))

    A = dequant_hidden(hidden_states, hidden_states_scale).to(accumulate)   # [T, H]
    idx, w, _, _ = route(logits, f32(routing_bias), routed_scaling_factor)
    dense_w = torch.from_numpy(dense_weights(idx, w, T))

    if dequant_all_upfront:
        W13_all = [dequant_block(w13c[e], s13[e]) for e in range(E_local)]
        W2_all = [dequant_block(w2c[e], s2[e]) for e in range(E_local)]

    out = torch.zeros((T, H), dtype=accumulate)
    sel = torch.from_numpy(idx.astype(np.int64))
    inter = {}
    for le in range(E_local):                                      # main.py:218
        ge = local_start + le
        if ge < 0 or ge >= E_GLOBAL:                               # main.py:219-221
            continue
        tok = torch.nonzero((sel == ge).any(dim=1), as_tuple=False).squeeze(1)
        if tok.numel() == 0:                                       # main.py:223
            continue
        A_e = A.index_select(0, tok)
        W13 = (W13_all[le] if dequant_all_upfront else dequant_block(w13c[le], s13[le])).to(accumulate)
        G1 = A_e @ W13.t()                                         # main.py:232
        C = swiglu(G1)                                             # main.py:233
        W2 = (W2_all[le] if dequant_all_upfront else dequant_block(w2c[le], s2[le])).to(accumulate)
        O = C @ W2.t()                                             # main.py:238
        w_tok = dense_w.index_select(0, tok)[:, ge]                # main.py:240
        out.index_add_(0, tok, O * w_tok.to(accumulate).unsqueeze(1))   # main.py:241
        if return_intermediates:
            inter[le] = dict(tokens=tok.numpy().astype(np.int32), G1=G1, C=C, O=O)
    out_bf16 = out.to(torch.bfloat16)                              # main.py:243
    if return_intermediates:
        return out, out_bf16, dict(idx=idx, w=w, experts=inter, A=A)
    return out, out_bf16


def roofline_work(idx, E_local: int, local_expert_offset: int, T: int, H: int = 7168, I: int = 2048):
    """Algorithmic HBM bytes and fp8 flops of one call, counted from the routing.

    bytes = A * (W13 + W2 + their scales) + T * (hidden + hidden scales + logits + bf16 out)
            + bias;  flops = P * (2*H*2I + 2*I*H), A = active local experts, P = local pairs.
    """
    counts, _, _, _ = permute(idx, np.zeros_like(idx, dtype=_F32), E_local, local_expert_offset)
    n_active = int((counts > 0).sum())
    P = int(counts.sum())
    per_expert = 2 * I * H + H * I + (2 * I // BLOCK) * (H // BLOCK) * 4 + (H // BLOCK) * (I // BLOCK) * 4
    per_token = H + (H // BLOCK) * 4 + E_GLOBAL * 4 + H * 2
    nbytes = n_active * per_expert + T * per_token + E_GLOBAL * 2
    flops = P * (2 * H * 2 * I + 2 * I * H)
    return dict(active_experts=n_active, pairs=P, bytes=nbytes, flops=flops)
