"""C-ABI library: builds for gfx950, loads, exports every declared symbol, and rejects
bad arguments on the host before any GPU work.  CPU only (no kernel is launched)."""
import ctypes
import re
from pathlib import Path

import pytest

from moe_fp8 import _abi
from moe_fp8 import build as mbuild

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moefp8.h"


@pytest.fixture(scope="module")
def lib():
    if not _abi.LIB_PATH.exists():
        mbuild.build()
    return _abi.load()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(moefp8_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_bound_exports():
    assert declared_functions() == sorted(_abi.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_library_is_built_for_gfx950_only():
    data = _abi.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in data


def test_ctypes_struct_mirrors_the_header():
    """Field names and order of struct moefp8_args in the header == the ctypes mirror."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct moefp8_args \{(.*?)\} moefp8_args;", text, flags=re.S).group(1)
    names = re.findall(r"(\w+)\s*;", body)
    assert names == [f for f, _ in _abi.MoeFp8Args._fields_]


def test_abi_version_and_strerror(lib):
    assert lib.moefp8_abi_version() == _abi.ABI_VERSION
    for code in _abi.STATUS:
        assert lib.moefp8_strerror(code)
    assert lib.moefp8_strerror(0) == b"ok"
    assert lib.moefp8_strerror(12345) == b"unknown status"


def test_workspace_size(lib):
    full = _abi.workspace_size(lib, 8192, 32, 7168, 2048)
    small = _abi.workspace_size(lib, 16, 32, 7168, 2048)
    assert small < full
    pmax = 8192 * 8
    # fp32 per-pair GEMM2 rows for half the pairs' worth of all columns above 1 GiB of them: one
    # pass over the columns while the call's pairs fit, two (half the columns each) beyond
    passes = lib.moefp8_output_passes
    assert full >= pmax * 3584 * 4
    assert full <= 1.5e9
    assert passes(8192, 32, 7168, 2048, 8587) == 1              # the benchmark's routing
    assert passes(8192, 32, 7168, 2048, pmax // 2) == 1
    assert passes(8192, 32, 7168, 2048, pmax // 2 + 1) == 2
    assert passes(8192, 32, 7168, 2048, pmax) == 2
    assert passes(4681, 32, 7168, 2048, 8 * 4681) == 1          # 4681 * 8 * 7168 * 4 B < 1 GiB: all rows
    assert passes(4682, 32, 7168, 2048, 8 * 4682) == 2
    assert passes(4682, 32, 384, 2048, 8 * 4682) == 1           # not the 128-row path (H % 256)
    assert passes(64, 32, 7168, 2048, 512) == 1
    assert passes(-1, 32, 7168, 2048, 0) == -2
    assert passes(16, 32, 7168, 2048, -1) == -2
    assert _abi.workspace_size(lib, 0, 32, 7168, 2048) > 0
    out = ctypes.c_size_t()
    assert lib.moefp8_workspace_size(16, 32, 7000, 2048, ctypes.byref(out)) == -2   # H not a multiple of 128
    assert lib.moefp8_workspace_size(16, 0, 7168, 2048, ctypes.byref(out)) == -2
    assert lib.moefp8_workspace_size(16, 257, 7168, 2048, ctypes.byref(out)) == -2
    assert lib.moefp8_workspace_size(-1, 32, 7168, 2048, ctypes.byref(out)) == -2
    assert lib.moefp8_workspace_size(16, 32, 7168, 2048, None) == -1


def _args(**kw):
    a = _abi.MoeFp8Args()
    a.num_tokens, a.num_local_experts, a.hidden_size, a.intermediate_size = 16, 32, 7168, 2048
    a.routed_scaling_factor = 2.5
    for i, f in enumerate(("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
                           "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale",
                           "output")):
        setattr(a, f, 0x100000 * (i + 1))     # fake, aligned, never dereferenced: validation fails first
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_run_rejects_bad_arguments_before_any_launch(lib):
    ws = 0x7000000
    run = lambda a, n=1 << 40, w=ws: lib.moefp8_run(ctypes.byref(a), w, n, None)
    assert lib.moefp8_run(None, ws, 0, None) == -1
    assert run(_args(hidden_size=100)) == -2
    assert run(_args(intermediate_size=0)) == -2
    assert run(_args(num_local_experts=0)) == -2
    assert run(_args(num_tokens=-5)) == -2
    assert run(_args(logits_dtype=7)) == -3
    assert run(_args(bias_dtype=-1)) == -3
    assert run(_args(routing_logits=None)) == -1
    assert run(_args(output=None)) == -1
    assert run(_args(gemm2_weights_scale=None)) == -1
    assert run(_args(hidden_states=0x100001)) == -4
    assert run(_args(routing_logits=0x100002)) == -4              # fp32 logits need 16-byte rows
    assert run(_args(routing_logits=0x100008)) == -4
    # 16-bit routing inputs are read with 8-byte loads: 8-byte alignment
    assert run(_args(routing_bias=0x200002, bias_dtype=1)) == -4            # 2-byte offset bf16 bias
    assert run(_args(routing_bias=0x200004, bias_dtype=2)) == -4            # 4-byte offset f16 bias
    assert run(_args(routing_logits=0x100002, logits_dtype=1)) == -4        # bf16 logits
    assert run(_args(gemm1_weights_scale=0x100002)) == -4
    assert run(_args(shared_output=0x100000 * 12, shared_dtype=2)) == -3   # shared rows: fp32 or bf16
    assert run(_args(shared_output=0x100008, shared_dtype=1)) == -4
    assert run(_args(output_f32=2)) == -3                                     # output: bf16 (0) or fp32 (1)
    assert run(_args(), n=1024) == -5                              # workspace too small
    assert run(_args(), w=0) == -5
    assert run(_args(num_tokens=0)) == 0                           # nothing to do, nothing launched


def test_route_rejects_bad_arguments(lib):
    f = lib.moefp8_route
    assert f(0x1000, 0, 0x2000, 1, -1, 2.5, 0x3000, 0x4000, None) == -2
    assert f(0x1000, 9, 0x2000, 1, 4, 2.5, 0x3000, 0x4000, None) == -3
    assert f(None, 0, 0x2000, 1, 4, 2.5, 0x3000, 0x4000, None) == -1
    assert f(0x1000, 0, 0x2000, 1, 0, 2.5, 0x3000, 0x4000, None) == 0
    assert f(0x1000, 0, 0x2002, 1, 4, 2.5, 0x3000, 0x4000, None) == -4   # bf16 bias: 8-byte aligned
    assert f(0x1008, 0, 0x2000, 1, 4, 2.5, 0x3000, 0x4000, None) == -4   # fp32 logits: 16-byte aligned


def test_quantize_rejects_bad_arguments(lib):
    f = lib.moefp8_quantize_hidden
    assert f(0x1000, 1, -1, 7168, 0x2000, 0x3000, None) == -2
    assert f(0x1000, 1, (1 << 24) + 1, 128, 0x2000, 0x3000, None) == -2
    assert f(0x1000, 1, 16, 100, 0x2000, 0x3000, None) == -2
    assert f(0x1000, 2, 16, 7168, 0x2000, 0x3000, None) == -3
    assert f(0x1000, 1, 0, 7168, 0x2000, 0x3000, None) == 0
    assert f(None, 1, 16, 7168, 0x2000, 0x3000, None) == -1
    assert f(0x1008, 1, 16, 7168, 0x2000, 0x3000, None) == -4             # x: 16-byte aligned


def test_python_entry_point_fails_loudly_without_device_tensors(lib):
    import torch
    import moe_fp8
    with pytest.raises(ValueError):
        moe_fp8.run(torch.zeros(4, 256), torch.zeros(256), torch.zeros(4, 256, dtype=torch.uint8),
                    torch.ones(2, 4), torch.zeros(1, 256, 256, dtype=torch.uint8), torch.ones(1, 2, 2),
                    torch.zeros(1, 256, 128, dtype=torch.uint8), torch.ones(1, 2, 1), 0, 2.5)


def test_missing_library_raises(tmp_path):
    with pytest.raises(FileNotFoundError):
        _abi.load(tmp_path / "libmoefp8.so")


def test_path_dispatch_bounds(lib):
    """moefp8_path: T <= 64 streams weights; from T = 128 the 128-row kernels run unless their
    32-bit DMA offsets could wrap (T x H >= 2^31, or Pmax x 2I >= 2^32 with Pmax = T x min(8,
    E_local)), or H is not a multiple of 256, or a K range exceeds 64 blocks; those shapes take
    the 4-wave grouped kernels (64-bit addresses)."""
    p = lib.moefp8_path
    H, I = 7168, 2048
    assert p(1, 32, H, I) == _abi.PATH_SMALL_T
    assert p(64, 32, H, I) == _abi.PATH_SMALL_T
    assert p(65, 32, H, I) == _abi.PATH_GROUPED
    assert p(127, 32, H, I) == _abi.PATH_GROUPED
    assert p(128, 32, H, I) == _abi.PATH_ROWS128
    assert p(8192, 32, H, I) == _abi.PATH_ROWS128
    # Pmax x 2I at the 2^32 edge (E_local >= 8: Pmax = 8T)
    assert 8 * 131071 * 2 * I < 1 << 32 <= 8 * 131072 * 2 * I
    assert p(131071, 256, H, I) == _abi.PATH_ROWS128
    assert p(131072, 256, H, I) == _abi.PATH_GROUPED
    assert p(131072, 4, H, I) == _abi.PATH_ROWS128          # Pmax = 4T
    # T x H at the 2^31 edge
    t = (1 << 31) // H
    assert p(t, 1, H, 128) == _abi.PATH_ROWS128
    assert p(t + 1, 1, H, 128) == _abi.PATH_GROUPED
    # shapes the 128-row kernels do not take
    assert p(4096, 32, 384, I) == _abi.PATH_GROUPED         # H % 256 != 0
    assert p(4096, 32, 128 * 65 * 2, I) == _abi.PATH_GROUPED  # H / 128 > 64
    assert p(4096, 32, H, 128 * 65) == _abi.PATH_GROUPED    # I / 128 > 64
    # invalid sizes
    assert p(-1, 32, H, I) == -2
    assert p(16, 0, H, I) == -2
    assert p(16, 32, 100, I) == -2


def test_noalloc_entry_point_limits_before_any_launch(lib):
    """moefp8_run_noalloc validates like moefp8_run and rejects sizes whose workspace exceeds its
    64 MiB static scratch with MOEFP8_ERR_SCRATCH_LIMIT, before touching the device."""
    f = lambda a: lib.moefp8_run_noalloc(ctypes.byref(a), None)
    assert lib.moefp8_run_noalloc(None, None) == -1
    assert f(_args(hidden_size=100)) == -2
    assert f(_args(routing_logits=None)) == -1
    assert f(_args(hidden_states=0x100001)) == -4
    assert f(_args(num_tokens=0)) == 0
    assert f(_args(num_tokens=8192)) == -8
    assert f(_args(num_tokens=1024)) == -8
    assert lib.moefp8_strerror(-8).startswith(b"sizes need more workspace")
    # every small-T shape of the operator fits the scratch
    for T in (1, 4, 16, 64):
        for E in (1, 32, 256):
            assert _abi.workspace_size(lib, T, E, 7168, 2048) <= _abi.NOALLOC_SCRATCH_BYTES
