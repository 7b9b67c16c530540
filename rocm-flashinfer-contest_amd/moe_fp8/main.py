"""MI355X-native ``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``.

Drop-in for the reference solution ``solutions/moe_fp8/main.py`` (entry point
``main.py::run``, ``solution.json:5-15``): same positional signature, same
argument meaning, returns a fresh bf16 ``[T, H]`` tensor and never mutates its
inputs.  All arithmetic runs in the gfx950 HIP library behind the C ABI of
``include/moefp8.h``; this module only checks arguments, allocates the output
and the workspace with the torch allocator and passes raw pointers and the
current HIP stream.  If the library is missing it raises: there is no
fallback path.

Operator (``main.py:139-243``): DeepSeek-V3 no-aux routing (sigmoid, bias,
top-2-sum group score, top-4 of 8 groups, top-8 of 256 experts, weights from
the unbiased sigmoid normalised and scaled by ``routed_scaling_factor``);
for each local expert ``le`` (global id ``local_expert_offset + le``) the
tokens that picked it; GEMM1 with the 128x128 block-scaled e4m3 gate/up
weights and the 1x128 block-scaled e4m3 hidden states; SwiGLU with the gate in
the second half; GEMM2 with the block-scaled down weights; routing-weighted sum
over experts in ascending order; bf16 output.
"""
from __future__ import annotations

import collections
import ctypes

import torch

try:
    from . import _abi
except ImportError:  # loaded as a standalone file, as flashinfer-bench's PythonBuilder does
    import importlib.util
    from pathlib import Path

    _spec = importlib.util.spec_from_file_location("moe_fp8_abi", Path(__file__).with_name("_abi.py"))
    _abi = importlib.util.module_from_spec(_spec)
    _spec.loader.exec_module(_abi)

# Operator constants (main.py:22-29).
H = 7168
I = 2048
BLOCK = 128
E_GLOBAL = 256
TOP_K = 8
N_GROUP = 8
TOPK_GROUP = 4

_DT = {torch.float32: _abi.DTYPE_F32, torch.bfloat16: _abi.DTYPE_BF16, torch.float16: _abi.DTYPE_F16}

# Workspace bytes per (T, E_local, H, I), and reusable workspaces per (device, stream) for calls
# whose workspace is at most _WS_KEEP_MAX bytes (the small-T decode sizes of a serving loop): calls
# on one stream run in stream order, so they can share one buffer.  At most _WS_KEEP_PER_DEVICE
# of them are held per device, the least recently used one dropped first (a server that makes a
# stream per request does not grow device memory, and a reused stream handle only finds a buffer
# that its stream order already protects).  Larger workspaces come from the torch allocator on
# every call (it caches them itself) and are not held between calls.
_WS_BYTES = {}
_WS_KEEP = collections.OrderedDict()
_WS_KEEP_MAX = 64 << 20
_WS_KEEP_PER_DEVICE = 4


def _workspace(lib, device, stream, T, E_local, Hd, Id):
    key = (T, E_local, Hd, Id)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        nbytes = _WS_BYTES[key] = _abi.workspace_size(lib, T, E_local, Hd, Id)
    if nbytes > _WS_KEEP_MAX:
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device), nbytes
    skey = (device.index, stream)
    ws = _WS_KEEP.pop(skey, None)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
    _WS_KEEP[skey] = ws                       # most recently used last
    same_dev = [k for k in _WS_KEEP if k[0] == device.index]
    for k in same_dev[:max(0, len(same_dev) - _WS_KEEP_PER_DEVICE)]:
        del _WS_KEEP[k]
    return ws, nbytes


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _routing_input(x, name, device):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.device != device:
        raise ValueError(f"{name} is on {x.device}, expected {device}")
    if x.dtype not in _DT:
        raise TypeError(f"{name}: unsupported dtype {x.dtype} (float32, bfloat16 or float16)")
    x = x.contiguous()
    # the routing kernel loads 4 elements at a time (8-byte loads): fp32 rows must start on 16
    # bytes, 16-bit ones on 8; a view at another storage offset is copied
    if x.data_ptr() % (16 if x.dtype == torch.float32 else 8) != 0:
        x = x.clone()
    return x


def _fp8_input(x, name, device):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.device != device:
        raise ValueError(f"{name} is on {x.device}, expected {device}")
    if x.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"{name}: expected float8_e4m3fn, got {x.dtype}")
    return x.contiguous()


def _scale_input(x, name, device, shape):
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.device != device:
        raise ValueError(f"{name} is on {x.device}, expected {device}")
    if tuple(x.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(x.shape)} != expected {tuple(shape)}")
    if x.dtype != torch.float32:
        raise TypeError(f"{name}: expected float32, got {x.dtype}")
    return x.contiguous()


def _scalar(x, kind):
    if isinstance(x, torch.Tensor):   # main.py:188-193 (host sync, as in the reference)
        return kind(x.item())
    return kind(x)


def _prepare(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
             gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
             routed_scaling_factor, debug=None, shared_output=None, output_dtype=torch.bfloat16,
             reuse_workspace=False):
    """Check the arguments, allocate output + workspace, fill the C argument struct.  With
    ``reuse_workspace`` a small workspace is shared by the calls on the current stream."""
    lib = _abi.load()
    if not isinstance(hidden_states, torch.Tensor) or hidden_states.device.type != "cuda":
        raise ValueError("hidden_states must be a device (cuda/HIP) tensor")
    device = hidden_states.device
    T = int(routing_logits.shape[0])
    E_local, two_I, Hd = (int(v) for v in gemm1_weights.shape)
    Id = two_I // 2
    logits = _routing_input(routing_logits, "routing_logits", device)
    bias = _routing_input(routing_bias, "routing_bias", device).reshape(-1)
    if tuple(logits.shape) != (T, E_GLOBAL) or bias.numel() != E_GLOBAL:
        raise ValueError(f"routing_logits must be [T, {E_GLOBAL}] and routing_bias [{E_GLOBAL}]")
    hs = _fp8_input(hidden_states, "hidden_states", device)
    if tuple(hs.shape) != (T, Hd):
        raise ValueError(f"hidden_states: shape {tuple(hs.shape)} != ({T}, {Hd})")
    w13 = _fp8_input(gemm1_weights, "gemm1_weights", device)
    w2 = _fp8_input(gemm2_weights, "gemm2_weights", device)
    if tuple(w2.shape) != (E_local, Hd, Id):
        raise ValueError(f"gemm2_weights: shape {tuple(w2.shape)} != ({E_local}, {Hd}, {Id})")
    hss = _scale_input(hidden_states_scale, "hidden_states_scale", device, (Hd // BLOCK, T))
    s13 = _scale_input(gemm1_weights_scale, "gemm1_weights_scale", device, (E_local, two_I // BLOCK, Hd // BLOCK))
    s2 = _scale_input(gemm2_weights_scale, "gemm2_weights_scale", device, (E_local, Hd // BLOCK, Id // BLOCK))
    offset = _scalar(local_expert_offset, int)
    rsf = _scalar(routed_scaling_factor, float)

    if output_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"output_dtype: expected torch.bfloat16 or torch.float32, got {output_dtype}")
    out = torch.empty((T, Hd), dtype=output_dtype, device=device)
    if reuse_workspace and T > 0:
        ws, ws_bytes = _workspace(lib, device, torch.cuda.current_stream(device).cuda_stream, T, E_local, Hd, Id)
    else:
        ws_bytes = _abi.workspace_size(lib, T, E_local, Hd, Id)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)

    args = _abi.MoeFp8Args()
    args.routing_logits = logits.data_ptr()
    args.routing_bias = bias.data_ptr()
    args.hidden_states = hs.data_ptr()
    args.hidden_states_scale = hss.data_ptr()
    args.gemm1_weights = w13.data_ptr()
    args.gemm1_weights_scale = s13.data_ptr()
    args.gemm2_weights = w2.data_ptr()
    args.gemm2_weights_scale = s2.data_ptr()
    args.num_tokens = T
    args.num_local_experts = E_local
    args.hidden_size = Hd
    args.intermediate_size = Id
    args.local_expert_offset = max(min(offset, 1 << 30), -(1 << 30))
    args.routed_scaling_factor = rsf
    args.logits_dtype = _DT[logits.dtype]
    args.bias_dtype = _DT[bias.dtype]
    args.output = out.data_ptr()
    args.output_f32 = 1 if output_dtype == torch.float32 else 0
    if debug is not None:
        P = T * min(TOP_K, E_local)
        debug["topk_ids"] = torch.empty((T, TOP_K), dtype=torch.int32, device=device)
        debug["topk_weights"] = torch.empty((T, TOP_K), dtype=torch.float32, device=device)
        debug["expert_offsets"] = torch.empty(E_local + 1, dtype=torch.int32, device=device)
        debug["permuted_tokens"] = torch.empty(P, dtype=torch.int32, device=device)
        args.topk_ids = debug["topk_ids"].data_ptr()
        args.topk_weights = debug["topk_weights"].data_ptr()
        args.expert_offsets = debug["expert_offsets"].data_ptr()
        args.permuted_tokens = debug["permuted_tokens"].data_ptr()
    shared = None
    if shared_output is not None:
        if not isinstance(shared_output, torch.Tensor) or shared_output.device != device:
            raise ValueError(f"shared_output must be a tensor on {device}")
        if tuple(shared_output.shape) != (T, Hd):
            raise ValueError(f"shared_output: shape {tuple(shared_output.shape)} != ({T}, {Hd})")
        if shared_output.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"shared_output: expected float32 or bfloat16, got {shared_output.dtype}")
        shared = shared_output.contiguous()
        args.shared_output = shared.data_ptr()
        args.shared_dtype = _DT[shared.dtype]
    keep = (logits, bias, hs, hss, w13, s13, w2, s2, shared)      # keep contiguous copies alive
    return lib, args, out, ws, ws_bytes, keep


def run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
        gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
        routed_scaling_factor, *, shared_output=None, output_dtype=torch.bfloat16, debug=None):
    """Same contract as ``solutions/moe_fp8/main.py:173-243``.

    ``shared_output`` (optional, keyword only; no counterpart in the reference): a [T, H]
    float32 or bfloat16 device tensor, e.g. DeepSeek-V3's shared-expert output, added to each
    token's routed sum in fp32 before the single bf16 rounding (the add fused into the
    combine instead of a separate pass over the output).

    ``output_dtype`` (keyword only): ``torch.bfloat16`` (the reference's) or ``torch.float32``,
    the same per-token sum before its bf16 rounding, for callers that add further partial sums
    (e.g. expert-parallel ranks) and round once; no counterpart in the reference.

    ``debug`` (optional dict) receives the device tensors ``topk_ids`` [T, 8]
    int32 (ascending global ids), ``topk_weights`` [T, 8] fp32,
    ``expert_offsets`` [E_local + 1] int32 and ``permuted_tokens`` int32 for the
    parity tests.
    """
    lib, args, out, ws, ws_bytes, _keep = _prepare(
        routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
        gemm2_weights, gemm2_weights_scale, local_expert_offset, routed_scaling_factor, debug, shared_output,
        output_dtype, reuse_workspace=True)
    if args.num_tokens == 0:
        return out
    device = out.device
    if torch.cuda.current_device() == device.index:
        stream = torch.cuda.current_stream(device).cuda_stream
        _abi.check(lib, lib.moefp8_run(ctypes.byref(args), ws.data_ptr(), ws_bytes, stream))
    else:
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device).cuda_stream
            _abi.check(lib, lib.moefp8_run(ctypes.byref(args), ws.data_ptr(), ws_bytes, stream))
    return out


class Runner:
    """``run`` with its arguments bound once: output and workspace are allocated at
    construction and every call only crosses the C ABI (for timing loops and
    serving loops that reuse the same buffers).  Each call overwrites ``out``."""

    def __init__(self, *run_args, debug=None, shared_output=None, output_dtype=torch.bfloat16):
        (self.lib, self.args, self.out, self.workspace, self.ws_bytes,
         self._keep) = _prepare(*run_args, debug=debug, shared_output=shared_output, output_dtype=output_dtype)
        self.device = self.out.device

    def __call__(self, stage_events=None, stream=None):
        if self.args.num_tokens == 0:
            return self.out
        self.args.stage_events = stage_events
        s = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
        _abi.check(self.lib, self.lib.moefp8_run(ctypes.byref(self.args), self.workspace.data_ptr(),
                                                 self.ws_bytes, s))
        self.args.stage_events = None
        return self.out


def route(routing_logits, routing_bias, routed_scaling_factor):
    """Routing alone (``main.py:139-165``): returns ``(topk_ids [T, 8] int32``
    in ascending id order, ``topk_weights [T, 8] fp32)``; ``topk_weights[t, j]``
    equals the reference's dense ``weights[t, topk_ids[t, j]]``."""
    lib = _abi.load()
    device = routing_logits.device
    if device.type != "cuda":
        raise ValueError("routing_logits must be a device (cuda/HIP) tensor")
    logits = _routing_input(routing_logits, "routing_logits", device)
    bias = _routing_input(routing_bias, "routing_bias", device).reshape(-1)
    T = int(logits.shape[0])
    if tuple(logits.shape) != (T, E_GLOBAL) or bias.numel() != E_GLOBAL:
        raise ValueError(f"routing_logits must be [T, {E_GLOBAL}] and routing_bias [{E_GLOBAL}]")
    ids = torch.empty((T, TOP_K), dtype=torch.int32, device=device)
    w = torch.empty((T, TOP_K), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.device(device):
        _abi.check(lib, lib.moefp8_route(logits.data_ptr(), _DT[logits.dtype], bias.data_ptr(), _DT[bias.dtype], T,
                                         _scalar(routed_scaling_factor, float), ids.data_ptr(), w.data_ptr(),
                                         stream))
    return ids, w


def quantize_hidden(x):
    """Per-token 1x128 quantization of activations ``x [T, H]`` (bf16 or fp32, device
    tensor, H a multiple of 128): returns ``(hidden_states e4m3fn [T, H],
    hidden_states_scale fp32 [H/128, T])``, the pair ``run`` consumes and
    ``main.py:129-136`` dequantizes, with scale = amax / 448 per token and 128 columns
    (1 for an all-zero block) and q = e4m3(x / scale) rounded to nearest even."""
    lib = _abi.load()
    device = x.device
    if device.type != "cuda":
        raise ValueError("x must be a device (cuda/HIP) tensor")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bfloat16 or float32, got {x.dtype}")
    if x.dim() != 2 or x.shape[1] % BLOCK != 0:
        raise ValueError(f"x must be [T, H] with H a multiple of {BLOCK}, got {tuple(x.shape)}")
    x = x.contiguous()
    T, Hd = int(x.shape[0]), int(x.shape[1])
    q = torch.empty((T, Hd), dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty((Hd // BLOCK, T), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.device(device):
        _abi.check(lib, lib.moefp8_quantize_hidden(x.data_ptr(), _DT[x.dtype], T, Hd, q.data_ptr(), scale.data_ptr(),
                                                   stream))
    return q, scale
