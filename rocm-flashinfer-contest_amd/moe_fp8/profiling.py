"""Summaries of rocprofv3 output for the operator's kernels, as committed under ``profiles/``.

The measurement method follows the reference's profiling tools (``tools/profile_kernel.py:87-94``
runs ``run()`` under ``rocprofv3 --kernel-trace``; ``tools/summarize_rocprof_trace.py:19-70``
buckets the dispatches by kernel name into stages).  Here every record is stamped with the
kernel-source hash (``build.source_hash()``), so ``bench.py`` can tell a record taken with the
current kernels from a stale one.

    python -m moe_fp8.profiling trace    <rocprof-dir> --workload W --steps K --warmup N --cmd "..." --out F
    python -m moe_fp8.profiling counters <rocprof-dir> [<rocprof-dir> ...] --workload W --cmd "..." [--cmd ...]
                                         [--copy-record profiles/traffic_copy.txt] --out F
    python -m moe_fp8.profiling traffic  <fetch-dir> <write-dir> --kernel K --workload W --cmd "..." --cmd "..." --out F

``trace`` reads ``*kernel_trace.csv``; ``counters`` and ``traffic`` read
``*counter_collection.csv`` (``rocprofv3 --output-format csv``).  The bench command the
records come from runs one workload: one first call, N warmup calls, K timed calls, K calls
with stage events, K warm back-to-back calls and the timed ``run()`` calls; every call but
the warm ones follows a cache flush.

Every figure is per operator call: the dispatches of one kernel within a call (the 128-row
path launches GEMM2 and the combine once per output pass, the second launch returning at once
when the call needs one pass) are summed, then averaged over calls.  A call starts at its
routing kernel's dispatch.
"""
from __future__ import annotations

import argparse
import csv
import glob
import statistics
import sys
from collections import defaultdict
from pathlib import Path

try:
    from .build import source_hash
except ImportError:  # run as a script
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from moe_fp8.build import source_hash

FIRST_KERNEL = "route_kernel"     # every operator call starts with the routing kernel
MI355X_CUS = 256
MI355X_XCDS = 8           # GRBM_GUI_ACTIVE reads the sum over the XCDs
SIMDS_PER_CU = 4


def _kernel(name: str) -> str | None:
    """'void moefp8::gemm2_big_kernel(...)' -> 'gemm2_big_kernel'; None for other libraries' kernels."""
    if "moefp8::" not in name:
        return None
    return name.split("(")[0].split("moefp8::")[-1].strip()


def _csvs(d, suffix):
    return sorted(glob.glob(str(Path(d) / "**" / f"*{suffix}"), recursive=True))


def _stamp_lines(workload, cmd):
    cmds = [cmd] if isinstance(cmd, str) else list(cmd)
    return ([f"source {source_hash()} (kernel-source hash of the library the numbers were taken with)",
             f"workload {workload}"] + [f"command: cd /tmp && {c}" for c in cmds])


def trace_calls(d):
    """Operator calls in dispatch order: lists of (kernel, start_ns, end_ns)."""
    files = _csvs(d, "kernel_trace.csv")
    if not files:
        raise FileNotFoundError(f"no *kernel_trace.csv under {d}")
    rows = []
    for f in files:
        for r in csv.DictReader(open(f)):
            k = _kernel(r["Kernel_Name"])
            if k:
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), k))
    rows.sort()
    calls, cur = [], []
    for a, b, k in rows:
        if k == FIRST_KERNEL and cur:
            calls.append(cur)
            cur = []
        cur.append((k, a, b))
    if cur:
        calls.append(cur)
    return calls


def _per_call(call):
    """{kernel: (dispatches, summed µs)} of one call."""
    out = {}
    for k, a, b in call:
        n, t = out.get(k, (0, 0.0))
        out[k] = (n + 1, t + (b - a) / 1e3)
    return out


def trace_summary(d, steps, warmup):
    """Per kernel: its summed duration per call (µs), averaged over the cold timed calls (the
    timed and stage-event passes) and over all calls, with min and max over calls; and the cold
    calls' first-start to last-end span."""
    calls = trace_calls(d)
    cold = calls[1 + warmup: 1 + warmup + 2 * steps]
    if not cold:
        raise ValueError(f"{len(calls)} operator calls in the trace; expected >= {1 + warmup + 2 * steps}")
    names = []
    for c in calls:
        for k, _, _ in c:
            if k not in names:
                names.append(k)
    pc_all = [_per_call(c) for c in calls]
    pc_cold = [_per_call(c) for c in cold]
    out = []
    for k in names:
        allv = [pc[k][1] for pc in pc_all if k in pc]
        coldv = [pc[k][1] for pc in pc_cold if k in pc]
        per = max(pc[k][0] for pc in pc_all if k in pc)
        out.append(dict(kernel=k, calls=len(allv), per_call=per,
                        cold_mean_us=statistics.fmean(coldv) if coldv else None,
                        all_mean_us=statistics.fmean(allv), min_us=min(allv), max_us=max(allv)))
    out.sort(key=lambda r: -(r["cold_mean_us"] or 0.0))
    span = [(c[-1][2] - c[0][1]) / 1e3 for c in cold]
    return out, statistics.fmean(span), len(calls)


def write_trace(d, workload, steps, warmup, cmd, out):
    rows, span, n = trace_summary(d, steps, warmup)
    lines = [f"# Kernel trace: moe_fp8 operator, {workload}", ""] + [f"    {x}" for x in _stamp_lines(workload, cmd)]
    lines += ["", f"{n} operator calls traced; 'cold' = the {2 * steps} timed and stage-event calls (each after a "
              f"768 MiB read flush), the calls bench.py's figures come from.", "",
              "Durations are per call: a kernel launched more than once per call (GEMM2 and the combine of the "
              "128-row path, once per output pass) counts the sum of its launches.", "",
              "| Kernel | Calls | Launches per call | Cold avg µs | All-call avg µs | Min µs | Max µs |",
              "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        lines.append(f"| `{r['kernel']}` | {r['calls']} | {r['per_call']} | {r['cold_mean_us']:.1f} | "
                     f"{r['all_mean_us']:.1f} | {r['min_us']:.1f} | {r['max_us']:.1f} |")
    lines += ["", f"Cold call span (first kernel start to last kernel end): {span:.1f} µs", ""]
    for r in rows:
        lines.append(f"record kernel={r['kernel']} workload={workload} cold_us={r['cold_mean_us']:.2f} "
                     f"source={source_hash()}")
    Path(out).write_text("\n".join(lines) + "\n")
    return rows


VGPR_FIELD_SCALE = 2


def counter_means(dirs):
    """{kernel: {counter: mean per call}} over every counter CSV under the given dirs (each
    counter summed over the kernel's dispatches in a call, then averaged over calls), plus the
    dispatch's resources (grid, workgroup, LDS, VGPRs)."""
    vals = defaultdict(lambda: defaultdict(list))
    res = {}
    for d in dirs:
        files = _csvs(d, "counter_collection.csv")
        if not files:
            raise FileNotFoundError(f"no *counter_collection.csv under {d}")
        for f in files:
            disp = {}
            for r in csv.DictReader(open(f)):
                k = _kernel(r["Kernel_Name"])
                if not k:
                    continue
                ent = disp.setdefault(int(r["Dispatch_Id"]), (k, {}))
                ent[1][r["Counter_Name"]] = ent[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
                # rocprofv3's VGPR_Count is the descriptor's granule count x 4, while a gfx950
                # wave64 allocates VGPRs in granules of 8: the allocation is twice the field
                # (gemm1_big_kernel: field 112, compiler 217 VGPRs -> 224 allocated)
                res.setdefault(k, dict(grid=int(r["Grid_Size"]), wg=int(r["Workgroup_Size"]),
                                       lds=int(r["LDS_Block_Size"]), vgpr=VGPR_FIELD_SCALE * int(r["VGPR_Count"]),
                                       agpr=int(r.get("Accum_VGPR_Count") or 0), sgpr=int(r["SGPR_Count"])))
            call = None
            for _, (k, cs) in sorted(disp.items()):
                if k == FIRST_KERNEL or call is None:
                    for kk, sums in (call or {}).items():
                        for c, v in sums.items():
                            vals[kk][c].append(v)
                    call = {}
                sums = call.setdefault(k, {})
                for c, v in cs.items():
                    sums[c] = sums.get(c, 0.0) + v
            for kk, sums in (call or {}).items():
                for c, v in sums.items():
                    vals[kk][c].append(v)
    return {k: {c: statistics.fmean(v) for c, v in cs.items()} for k, cs in vals.items()}, res


def derived(c):
    """Ratios from one kernel's counters (None where a counter is missing):
    mfma_busy   = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x CUs x 4 SIMDs), the fraction
                  of SIMD-cycles the matrix cores were busy while the GPU was (GRBM_GUI_ACTIVE is
                  summed over the XCDs, SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs);
    lds_conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE, the share of LDS-active cycles lost
                  to bank conflicts;
    valu_per_mfma = SQ_INSTS_VALU / SQ_INSTS_MFMA (the MFMA instructions are counted in both)."""
    def g(n):
        return c.get(n)
    out = {}
    if g("SQ_VALU_MFMA_BUSY_CYCLES") is not None and g("GRBM_GUI_ACTIVE"):
        out["mfma_busy"] = g("SQ_VALU_MFMA_BUSY_CYCLES") / (g("GRBM_GUI_ACTIVE") / MI355X_XCDS * MI355X_CUS * SIMDS_PER_CU)
    if g("SQ_LDS_BANK_CONFLICT") is not None and g("SQ_LDS_IDX_ACTIVE"):
        out["lds_conflict"] = g("SQ_LDS_BANK_CONFLICT") / g("SQ_LDS_IDX_ACTIVE")
    if g("SQ_INSTS_VALU") is not None and g("SQ_INSTS_MFMA"):
        out["valu_per_mfma"] = g("SQ_INSTS_VALU") / g("SQ_INSTS_MFMA")
    return out


def write_counters(dirs, workload, cmd, out, calibration=None):
    means, res = counter_means(dirs)
    names = sorted({n for cs in means.values() for n in cs})
    lines = [f"# Counters: moe_fp8 operator kernels, {workload}", ""] + [f"    {x}" for x in _stamp_lines(workload, cmd)]
    lines += ["", "Mean per operator call over the run's calls, a kernel's dispatches within one call summed "
              "(rocprofv3 --pmc, one pass per counter group).", ""]
    lines += ["| Kernel | grid x wg | LDS B | VGPRs allocated / AGPR | " + " | ".join(names) + " |",
              "|---|---|---:|---|" + "---:|" * len(names)]
    for k in sorted(means):
        r = res[k]
        lines.append(f"| `{k}` | {r['grid'] // max(r['wg'], 1)} x {r['wg']} | {r['lds']} | {r['vgpr']}/{r['agpr']} | "
                     + " | ".join(f"{means[k][n]:.4g}" if n in means[k] else "" for n in names) + " |")
    lines += ["", "Derived (formulas in moe_fp8/profiling.py `derived`):", "",
              "| Kernel | MFMA busy | LDS bank-conflict share | VALU / MFMA instructions | HBM read GB | HBM write GB |",
              "|---|---:|---:|---:|---:|---:|"]
    for k in sorted(means):
        dv = derived(means[k])
        rd = wr = None
        if calibration and "FETCH_SIZE" in means[k]:
            rd = means[k]["FETCH_SIZE"] * 1024 / calibration[0] / 1e9
        if calibration and "WRITE_SIZE" in means[k]:
            wr = means[k]["WRITE_SIZE"] * 1024 / calibration[1] / 1e9

        def f(v, fmt):
            return format(v, fmt) if v is not None else ""
        lines.append(f"| `{k}` | {f(dv.get('mfma_busy'), '.3f')} | {f(dv.get('lds_conflict'), '.3f')} | "
                     f"{f(dv.get('valu_per_mfma'), '.2f')} | {f(rd, '.3f')} | {f(wr, '.3f')} |")
    Path(out).write_text("\n".join(lines) + "\n")
    return means


def copy_calibration(record_file):
    """(FETCH_SIZE KiB, WRITE_SIZE KiB) per byte of a plain device copy, from traffic_copy.txt."""
    for line in Path(record_file).read_text().splitlines():
        if line.startswith("record "):
            kv = dict(x.split("=", 1) for x in line.split()[1:])
            return (float(kv["fetch_kib"]) * 1024 / float(kv["bytes"]), float(kv["write_kib"]) * 1024 / float(kv["bytes"]))
    raise ValueError(f"no record line in {record_file}")


def write_traffic(fetch_dir, write_dir, kernel, workload, cmd, out):
    fm, _ = counter_means([fetch_dir])
    wm, _ = counter_means([write_dir])
    if kernel not in fm or kernel not in wm:
        raise KeyError(f"{kernel} not in the counter runs ({sorted(fm)})")
    fk, wk = fm[kernel]["FETCH_SIZE"], wm[kernel]["WRITE_SIZE"]
    txt = "\n".join([f"# HBM traffic per call of {kernel} on the {workload} workload",
                     "# rocprofv3 FETCH_SIZE and WRITE_SIZE readings, KiB per operator call (the kernel's dispatches "
                     "in a call summed, mean over calls), one pass each:"]
                    + [f"#   {x}" for x in _stamp_lines(workload, cmd)]
                    + [f"record kernel={kernel} workload={workload} fetch_kib={fk:.1f} write_kib={wk:.1f} "
                       f"source={source_hash()}"]) + "\n"
    Path(out).write_text(txt)
    return fk, wk


def read_record(path, **match):
    """The key=value fields of the first 'record' line of a profiles/ file whose fields match."""
    p = Path(path)
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("record "):
            kv = dict(x.split("=", 1) for x in line.split()[1:])
            if all(kv.get(k) == v for k, v in match.items()):
                return kv
    return None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--workload", required=True)
    t.add_argument("--steps", type=int, required=True)
    t.add_argument("--warmup", type=int, required=True)
    t.add_argument("--cmd", required=True, action="append", help="a command the numbers come from (repeatable)")
    t.add_argument("--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--workload", required=True)
    c.add_argument("--cmd", required=True, action="append", help="a command the numbers come from (repeatable)")
    c.add_argument("--out", required=True)
    c.add_argument("--copy-record", default=None, help="traffic_copy.txt, to turn FETCH/WRITE_SIZE into bytes")
    r = sub.add_parser("traffic")
    r.add_argument("fetch_dir")
    r.add_argument("write_dir")
    r.add_argument("--kernel", required=True)
    r.add_argument("--workload", required=True)
    r.add_argument("--cmd", required=True, action="append", help="a command the numbers come from (repeatable)")
    r.add_argument("--out", required=True)
    a = ap.parse_args(argv)
    if a.what == "trace":
        for row in write_trace(a.dir, a.workload, a.steps, a.warmup, a.cmd, a.out):
            print(f"{row['kernel']:28s} {row['cold_mean_us']:8.1f} µs")
    elif a.what == "counters":
        cal = copy_calibration(a.copy_record) if a.copy_record else None
        write_counters(a.dirs, a.workload, a.cmd, a.out, cal)
        print(Path(a.out).read_text())
    else:
        print(write_traffic(a.fetch_dir, a.write_dir, a.kernel, a.workload, a.cmd, a.out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
