"""Official-workload tooling for the contest definition
``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``: a reader for
flashinfer-trace definition JSON and workload JSONL (tensors from safetensors files)
and the contest's matched-ratio scorer.

The dataset is not available offline and flashinfer-bench is not installed here, so both
follow the reference's call sites rather than that library:

* a workload names the operator's inputs; each input is ``{"type": "safetensors", "path",
  "tensor_key"}`` (path relative to the dataset root), ``{"type": "scalar", "value"}`` or
  ``{"type": "random"}``, and ``axes["seq_len"]`` is T -- the shape that
  ``tools/local_verify.py:100-106`` and ``tools/moe_parity.py:170-175`` hand to
  ``load_safetensors`` / ``gen_inputs``;
* an output element matches when ``|out - ref| <= atol + rtol * |ref|``; a workload passes
  when the matched ratio reaches the required one (atol 1.0, rtol 0.3, ratio 0.9 for this
  definition, ``tools/run_benchmarks.py:146-147``, ``tools/moe_parity.py:162-164``).

Random inputs are drawn with this repository's own generator conventions (``workloads.py``),
not flashinfer-bench's, so they are comparable only with themselves.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from . import workloads as W

DEFINITION = "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
ARG_ORDER = ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale", "gemm1_weights",
             "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale", "local_expert_offset",
             "routed_scaling_factor")
ATOL, RTOL, REQUIRED_MATCHED_RATIO = 1.0, 0.3, 0.9


def load_definition(path) -> dict:
    """A definition JSON (``name``, ``axes``, ``inputs``, ``outputs``, ...)."""
    d = json.loads(Path(path).read_text())
    if d.get("name") != DEFINITION:
        raise ValueError(f"{path}: definition {d.get('name')!r} is not {DEFINITION}")
    return d


def load_workloads(path, definition: str = DEFINITION) -> list[dict]:
    """Workloads of one definition from a JSONL file: each line is either a trace record
    ``{"definition": ..., "workload": {...}}`` or a bare workload ``{"uuid", "axes", "inputs"}``."""
    out = []
    for line in Path(path).read_text().splitlines():
        if not line.strip():
            continue
        rec = json.loads(line)
        if "workload" in rec:
            if rec.get("definition", definition) != definition:
                continue
            rec = rec["workload"]
        out.append(rec)
    return out


def _random_inputs(T: int, seed: int, E_local: int, H: int, I: int) -> dict:
    wl = W.Workload(f"random_t{T}", T, seed)
    logits, bias, hidden, hscale = W.make_activations(wl, device="cpu", H=H)
    w13, s13, w2, s2 = W.make_weights(E_local=E_local, H=H, I=I, seed=seed + 1)
    return {"routing_logits": logits, "routing_bias": bias, "hidden_states": hidden, "hidden_states_scale": hscale,
            "gemm1_weights": w13, "gemm1_weights_scale": s13, "gemm2_weights": w2, "gemm2_weights_scale": s2,
            "local_expert_offset": 0, "routed_scaling_factor": W.RSF}


def materialize(workload: dict, root=".", device="cuda", seed: int = 0, E_local: int = W.E_LOCAL_FULL,
                H: int = W.H_FULL, I: int = W.I_FULL) -> tuple:
    """The ``run`` arguments of a workload, in ``main.py:173-184`` order, tensors on ``device``."""
    from safetensors.torch import load_file

    T = int(workload["axes"]["seq_len"])
    inputs = workload.get("inputs", {})
    files: dict = {}
    rand = None
    args = []
    for name in ARG_ORDER:
        spec = inputs.get(name, {"type": "random"})
        kind = spec.get("type")
        if kind == "safetensors":
            p = Path(root) / spec["path"]
            if p not in files:
                files[p] = load_file(str(p))
            v = files[p][spec.get("tensor_key", name)]
        elif kind == "scalar":
            v = spec["value"]
        elif kind == "random":
            if rand is None:
                rand = _random_inputs(T, seed, E_local, H, I)
            v = rand[name]
        else:
            raise ValueError(f"input {name}: unknown type {kind!r}")
        args.append(v.to(device) if isinstance(v, torch.Tensor) else v)
    return tuple(args)


def error_stats(out: torch.Tensor, ref: torch.Tensor, atol: float = ATOL, rtol: float = RTOL,
                required_matched_ratio: float = REQUIRED_MATCHED_RATIO) -> dict:
    """Matched-ratio score of ``out`` against ``ref`` (both compared in fp32)."""
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    if o.shape != r.shape:
        raise ValueError(f"shape {tuple(o.shape)} != {tuple(r.shape)}")
    err = (o - r).abs()
    n = err.numel()
    matched = int((err <= atol + rtol * r.abs()).sum()) if n else 0
    ratio = matched / n if n else 1.0
    rel = err / r.abs().clamp_min(1e-12)
    return {"max_abs": float(err.max()) if n else 0.0, "max_rel": float(rel.max()) if n else 0.0,
            "matched_ratio": ratio, "passed": ratio >= required_matched_ratio}
