"""flashinfer-bench packaging of this implementation.

Writes a ``solution.json`` in the format of the reference's packer
(``tools/pack_solution.py:33-46``: name, definition, author, spec {language,
target_hardware, entry_point, dependencies, destination_passing_style}, sources
[{path, content}], description) for the definition
``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``.

Solution sources are text, so the HIP library cannot travel inside the JSON.  The
package carries the HIP sources, the C header, the ctypes binding, the operator module
(``moe_fp8_op.py``, this package's ``main.py``) and a loader ``main.py`` (entry point
``main.py::run``) that, on first import, compiles ``libmoefp8.so`` beside itself with
hipcc for gfx950 and then serves ``run`` from the operator module.  There is still no
fallback: without hipcc or a gfx950 device the import or the call raises.

    python -m moe_fp8.pack --out solution.json        (rocm-flashinfer-contest_amd/ on sys.path)
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

from . import build as B
from .contest import DEFINITION

PKG_DIR = Path(__file__).resolve().parent

LOADER = '''"""flashinfer-bench entry point (main.py::run) of the MI355X (gfx950) HIP implementation of
{definition}.  On first import it compiles libmoefp8.so from the bundled sources with hipcc
(solution sources are text only), then serves run() from the bundled operator module."""
import importlib.util
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

_HERE = Path(__file__).resolve().parent
_LIB = _HERE / "libmoefp8.so"
_FLAGS = {flags!r}


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise FileNotFoundError("hipcc not found: the ROCm toolchain is needed to build libmoefp8.so")


def _build():
    cc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="moefp8_") as tmp:
        objs, procs = [], []
        for src in sorted((_HERE / "csrc").glob("*.hip")):
            obj = Path(tmp) / (src.stem + ".o")
            procs.append(subprocess.Popen([cc, *_FLAGS, "-I" + str(_HERE / "include"), "-c", str(src), "-o", str(obj)],
                                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT))
            objs.append(str(obj))
        for p in procs:
            log, _ = p.communicate()
            if p.returncode != 0:
                raise RuntimeError("hipcc failed:\\n" + log.decode(errors="replace"))
        out = Path(tmp) / _LIB.name
        subprocess.run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(out), *objs], check=True,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        shutil.copyfile(out, str(_LIB) + ".tmp")
        os.replace(str(_LIB) + ".tmp", _LIB)


if not _LIB.exists():
    _build()

_spec = importlib.util.spec_from_file_location("moe_fp8_op", _HERE / "moe_fp8_op.py")
_op = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(_op)
run = _op.run
'''


def sources() -> list[dict]:
    """The solution's source files, paths relative to the solution directory."""
    out = [{"path": "main.py", "content": LOADER.format(definition=DEFINITION, flags=list(B.HIPCC_FLAGS))},
           {"path": "moe_fp8_op.py", "content": (PKG_DIR / "main.py").read_text()},
           {"path": "_abi.py", "content": (PKG_DIR / "_abi.py").read_text()},
           {"path": "include/moefp8.h", "content": (B.INCLUDE / "moefp8.h").read_text()}]
    for f in sorted(B.CSRC.iterdir()):
        if f.suffix in (".hip", ".h"):
            out.append({"path": f"csrc/{f.name}", "content": f.read_text()})
    return out


def solution(name: str = "moefp8_mi355x_hip") -> dict:
    return {
        "name": name,
        "definition": DEFINITION,
        "author": "rocm-flashinfer-contest_amd",
        "spec": {
            "language": "python",
            "target_hardware": ["AMD MI355X"],
            "entry_point": "main.py::run",
            "dependencies": [],
            "destination_passing_style": False,
        },
        "sources": sources(),
        "description": "gfx950 HIP kernels behind a C ABI: wavefront routing, permutation, fp8 MFMA grouped "
                       "GEMMs with SwiGLU, weighted combine; built with hipcc at first import",
    }


def unpack(sol: dict, dest) -> Path:
    """Write a solution's sources into ``dest`` (what a harness builder does before importing
    the entry point); returns the entry module's path."""
    dest = Path(dest)
    for s in sol["sources"]:
        p = dest / s["path"]
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(s["content"])
    return dest / sol["spec"]["entry_point"].split("::")[0]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default="solution.json")
    ap.add_argument("--name", default="moefp8_mi355x_hip")
    args = ap.parse_args(argv)
    sol = solution(args.name)
    Path(args.out).write_text(json.dumps(sol, indent=2))
    print(f"wrote {args.out} with {len(sol['sources'])} source files")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
