"""The rocprofv3 summariser (moe_fp8/profiling.py) and bench.py's use of its records, on synthetic
CSV files laid out as rocprofv3 --output-format csv writes them.  CPU only."""
import csv
import importlib
import sys
from pathlib import Path

import pytest

from moe_fp8 import build, profiling

REPO = Path(__file__).resolve().parents[1]

TRACE_FIELDS = ["Kernel_Name", "Start_Timestamp", "End_Timestamp"]
COUNTER_FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Grid_Size", "Workgroup_Size",
                  "LDS_Block_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count"]


def write_csv(path, fields, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def fake_trace(d, calls):
    """calls: list of [(kernel, duration_ns), ...] run back to back, 1 µs apart."""
    rows, t = [], 1000
    for call in calls:
        for k, dur in call:
            rows.append({"Kernel_Name": f"void moefp8::{k}(moefp8::Problem, moefp8::Plan)",
                         "Start_Timestamp": t, "End_Timestamp": t + dur})
            t += dur + 1000
        # another library's kernel between calls is ignored
        rows.append({"Kernel_Name": "at::native::reduce_kernel<512, 1>", "Start_Timestamp": t, "End_Timestamp": t + 50})
        t += 2000
    write_csv(d / "run_kernel_trace.csv", TRACE_FIELDS, rows)


def test_kernel_names_and_call_split(tmp_path):
    assert profiling._kernel("void moefp8::gemm2_big_kernel(moefp8::Problem, float*)") == "gemm2_big_kernel"
    assert profiling._kernel("void at::native::foo()") is None
    calls = [[("route_kernel", 5000), ("gemm1_decode_kernel", 50000 + 1000 * i), ("gemm2_decode_kernel", 25000)]
             for i in range(8)]
    fake_trace(tmp_path, calls)
    got = profiling.trace_calls(tmp_path)
    assert len(got) == 8 and [k for k, _, _ in got[0]] == ["route_kernel", "gemm1_decode_kernel", "gemm2_decode_kernel"]
    # steps=3, warmup=1: calls 2..7 are the cold ones (the first call and one warmup skipped;
    # 2 x steps cold calls: the timed and the stage-event passes)
    rows, span, n = profiling.trace_summary(tmp_path, steps=3, warmup=1)
    by = {r["kernel"]: r for r in rows}
    assert n == 8
    assert by["gemm1_decode_kernel"]["cold_mean_us"] == pytest.approx((52 + 53 + 54 + 55 + 56 + 57) / 6)
    assert by["gemm1_decode_kernel"]["min_us"] == pytest.approx(50.0)
    assert rows[0]["kernel"] == "gemm1_decode_kernel"          # longest first
    assert span == pytest.approx(5 + 1 + 54.5 + 1 + 25)          # first start to last end of a cold call


def test_kernel_launched_twice_per_call_is_summed(tmp_path):
    # the 128-row path launches GEMM2 and the combine once per output pass; a one-pass call's
    # second launches return at once and still count towards the call
    calls = [[("route_kernel", 4000), ("gemm2_big_kernel", 400000 + 1000 * i), ("combine_kernel", 60000),
              ("gemm2_big_kernel", 3000), ("combine_kernel", 2000)] for i in range(4)]
    fake_trace(tmp_path, calls)
    rows, _, n = profiling.trace_summary(tmp_path, steps=1, warmup=1)
    by = {r["kernel"]: r for r in rows}
    assert n == 4 and by["gemm2_big_kernel"]["per_call"] == 2 and by["gemm2_big_kernel"]["calls"] == 4
    assert by["gemm2_big_kernel"]["cold_mean_us"] == pytest.approx((402 + 403) / 2 + 3)
    assert by["combine_kernel"]["min_us"] == pytest.approx(62.0)


def test_trace_record_roundtrip_and_staleness(tmp_path, monkeypatch):
    fake_trace(tmp_path / "kt", [[("route_kernel", 4000), ("gemm2_big_kernel", 400000)]] * 4)
    out = tmp_path / "moe_fp8_kernels_w.md"
    profiling.write_trace(tmp_path / "kt", "w", 1, 1, ["rocprofv3 --kernel-trace -- python3 bench.py"], out)
    text = out.read_text()
    assert f"source {build.source_hash()}" in text and "command: cd /tmp && rocprofv3" in text
    rec = profiling.read_record(out, kernel="gemm2_big_kernel")
    assert rec["workload"] == "w" and float(rec["cold_us"]) == pytest.approx(400.0)
    assert profiling.read_record(out, kernel="nope") is None
    assert profiling.read_record(tmp_path / "missing.md", kernel="x") is None

    sys.path.insert(0, str(REPO))
    bench = importlib.import_module("bench")
    monkeypatch.setattr(bench, "PROFILES", tmp_path)
    (tmp_path / "moe_fp8_kernels_w.md").write_text(text)
    assert bench.traced_us("gemm2_big_kernel", "w") == pytest.approx(400.0)
    # a record taken with other kernel sources is not used
    (tmp_path / "moe_fp8_kernels_w.md").write_text(text.replace(build.source_hash(), "0" * 16))
    assert bench.traced_us("gemm2_big_kernel", "w") is None


def test_counters_derived_and_traffic(tmp_path, monkeypatch):
    res = {"Grid_Size": 131072, "Workgroup_Size": 512, "LDS_Block_Size": 150016, "VGPR_Count": 112,
           "Accum_VGPR_Count": 0, "SGPR_Count": 112}
    k = "void moefp8::gemm1_big_kernel(moefp8::Problem)"
    r0 = "void moefp8::route_kernel(int)"
    k2 = "void moefp8::gemm2_big_kernel(moefp8::Problem)"
    sq = [dict(res, Dispatch_Id=1, Kernel_Name=r0, Counter_Name="GRBM_GUI_ACTIVE", Counter_Value=1.0)]
    sq += [dict(res, Dispatch_Id=2, Kernel_Name=k, Counter_Name=n, Counter_Value=v) for n, v in
           (("GRBM_GUI_ACTIVE", 8.0e6), ("SQ_VALU_MFMA_BUSY_CYCLES", 2.56e8), ("SQ_LDS_BANK_CONFLICT", 1.0e6),
            ("SQ_LDS_IDX_ACTIVE", 4.0e6), ("SQ_INSTS_VALU", 9.0e7), ("SQ_INSTS_MFMA", 1.0e7))]
    write_csv(tmp_path / "sq" / "run_counter_collection.csv", COUNTER_FIELDS, sq)
    # two calls: route, GEMM1, GEMM2 twice (its second launch nearly empty); rows in any order
    fetch = [dict(res, Dispatch_Id=d, Kernel_Name=n, Counter_Name="FETCH_SIZE", Counter_Value=v) for d, n, v in
             ((1, r0, 5.0), (2, k, 1000.0), (3, k2, 700.0), (4, k2, 14.0),
              (5, r0, 5.0), (6, k, 3000.0), (7, k2, 900.0), (8, k2, 14.0))]
    write_csv(tmp_path / "fetch" / "run_counter_collection.csv", COUNTER_FIELDS, fetch[::-1])
    write_csv(tmp_path / "write" / "run_counter_collection.csv", COUNTER_FIELDS,
              [dict(res, Dispatch_Id=1, Kernel_Name=k, Counter_Name="WRITE_SIZE", Counter_Value=500.0)])
    means, resources = profiling.counter_means([tmp_path / "sq", tmp_path / "fetch"])
    assert means["gemm1_big_kernel"]["FETCH_SIZE"] == pytest.approx(2000.0)   # mean per call
    assert means["gemm2_big_kernel"]["FETCH_SIZE"] == pytest.approx(814.0)    # both launches of a call
    assert resources["gemm1_big_kernel"]["wg"] == 512
    assert resources["gemm1_big_kernel"]["vgpr"] == 224                        # the field x 2
    d = profiling.derived(means["gemm1_big_kernel"])
    # 2.56e8 busy SIMD-cycles over (8e6 / 8 XCDs) cycles x 256 CUs x 4 SIMDs
    assert d["mfma_busy"] == pytest.approx(0.25)
    assert d["lds_conflict"] == pytest.approx(0.25)
    assert d["valu_per_mfma"] == pytest.approx(9.0)

    out = tmp_path / "traffic_gemm1_big_kernel_w.txt"
    fk, wk = profiling.write_traffic(tmp_path / "fetch", tmp_path / "write", "gemm1_big_kernel", "w",
                                     ["rocprofv3 --pmc FETCH_SIZE", "rocprofv3 --pmc WRITE_SIZE"], out)
    assert (fk, wk) == (pytest.approx(2000.0), pytest.approx(500.0))
    cal = tmp_path / "traffic_copy.txt"
    cal.write_text("# copy\nrecord kernel=copy workload=copy fetch_kib=512.0 write_kib=1024.0 bytes=1048576\n")
    assert profiling.copy_calibration(cal) == (pytest.approx(0.5), pytest.approx(1.0))
    sys.path.insert(0, str(REPO))
    bench = importlib.import_module("bench")
    monkeypatch.setattr(bench, "PROFILES", tmp_path)
    # 2000 KiB fetched at 0.5 per byte + 500 KiB written at 1.0 per byte
    assert bench.measured_traffic("gemm1_big_kernel", "w") == 2000 * 1024 * 2 + 500 * 1024
    out.write_text(out.read_text().replace(build.source_hash(), "f" * 16))
    assert bench.measured_traffic("gemm1_big_kernel", "w") is None

    md = tmp_path / "counters.md"
    profiling.write_counters([tmp_path / "sq", tmp_path / "fetch", tmp_path / "write"], "w", ["a", "b"], md,
                             calibration=(0.5, 1.0))
    text = md.read_text()
    assert "| `gemm1_big_kernel` | 0.250 | 0.250 | 9.00 | 0.004 | 0.001 |" in text
