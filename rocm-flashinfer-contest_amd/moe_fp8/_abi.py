"""ctypes binding of the C ABI declared in ``include/moefp8.h``.

This is the Python side of the drop-in boundary: plain pointers, sizes and a
HIP stream handle cross it; no torch types do.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_NAME = "libmoefp8.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

ABI_VERSION = 7

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

STATUS = {
    0: "MOEFP8_OK",
    -1: "MOEFP8_ERR_NULL_POINTER",
    -2: "MOEFP8_ERR_SHAPE",
    -3: "MOEFP8_ERR_DTYPE",
    -4: "MOEFP8_ERR_ALIGNMENT",
    -5: "MOEFP8_ERR_WORKSPACE",
    -6: "MOEFP8_ERR_LAUNCH",
    -7: "MOEFP8_ERR_DEVICE",
    -8: "MOEFP8_ERR_SCRATCH_LIMIT",
}

# Every extern "C" symbol of include/moefp8.h.
EXPORTS = ("moefp8_abi_version", "moefp8_strerror", "moefp8_workspace_size", "moefp8_path", "moefp8_output_passes",
           "moefp8_run", "moefp8_run_noalloc", "moefp8_route", "moefp8_quantize_hidden")

# MOEFP8_NOALLOC_SCRATCH_BYTES: static scratch of moefp8_run_noalloc
NOALLOC_SCRATCH_BYTES = 64 << 20

# moefp8_path results
PATH_SMALL_T = 0
PATH_GROUPED = 1
PATH_ROWS128 = 2


class MoeFp8Args(ctypes.Structure):
    """Mirror of ``struct moefp8_args``."""
    _fields_ = [
        ("routing_logits", ctypes.c_void_p),
        ("routing_bias", ctypes.c_void_p),
        ("hidden_states", ctypes.c_void_p),
        ("hidden_states_scale", ctypes.c_void_p),
        ("gemm1_weights", ctypes.c_void_p),
        ("gemm1_weights_scale", ctypes.c_void_p),
        ("gemm2_weights", ctypes.c_void_p),
        ("gemm2_weights_scale", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int64),
        ("num_local_experts", ctypes.c_int32),
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("local_expert_offset", ctypes.c_int32),
        ("routed_scaling_factor", ctypes.c_float),
        ("logits_dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32),
        ("output", ctypes.c_void_p),
        ("topk_ids", ctypes.c_void_p),
        ("topk_weights", ctypes.c_void_p),
        ("expert_offsets", ctypes.c_void_p),
        ("permuted_tokens", ctypes.c_void_p),
        ("stage_events", ctypes.c_void_p),
        ("shared_output", ctypes.c_void_p),
        ("shared_dtype", ctypes.c_int32),
        ("output_f32", ctypes.c_int32),
    ]


NUM_STAGE_EVENTS = 9
# the last two stages run GEMM2 and the combine again for the second half of the output columns
# when the per-pair output rows do not fit the workspace in one pass (empty otherwise)
STAGES = ("route", "permute", "gemm1", "activation", "gemm2", "combine", "gemm2_b", "combine_b")


class MoeFp8Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


_LIB = None


def load(path: os.PathLike | None = None):
    """Load the HIP library (cached).  Raises if it has not been built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build the gfx950 HIP library first (python -m moe_fp8.build, "
            "or __graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(str(p))
    lib.moefp8_abi_version.restype = ctypes.c_int
    lib.moefp8_abi_version.argtypes = []
    lib.moefp8_strerror.restype = ctypes.c_char_p
    lib.moefp8_strerror.argtypes = [ctypes.c_int]
    lib.moefp8_workspace_size.restype = ctypes.c_int
    lib.moefp8_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.POINTER(ctypes.c_size_t)]
    lib.moefp8_path.restype = ctypes.c_int
    lib.moefp8_path.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    lib.moefp8_output_passes.restype = ctypes.c_int
    lib.moefp8_output_passes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_int64]
    lib.moefp8_run.restype = ctypes.c_int
    lib.moefp8_run.argtypes = [ctypes.POINTER(MoeFp8Args), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.moefp8_run_noalloc.restype = ctypes.c_int
    lib.moefp8_run_noalloc.argtypes = [ctypes.POINTER(MoeFp8Args), ctypes.c_void_p]
    lib.moefp8_route.restype = ctypes.c_int
    lib.moefp8_route.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                 ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.moefp8_quantize_hidden.restype = ctypes.c_int
    lib.moefp8_quantize_hidden.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    if lib.moefp8_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {lib.moefp8_abi_version()} != {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def check(lib, status: int):
    if status != 0:
        raise MoeFp8Error(status, lib.moefp8_strerror(status).decode())


def workspace_size(lib, T: int, E_local: int, H: int, I: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib, lib.moefp8_workspace_size(T, E_local, H, I, ctypes.byref(out)))
    return int(out.value)
