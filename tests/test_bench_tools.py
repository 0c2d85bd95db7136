"""CPU checks of bench.py's profile summarisers (the tables under profiles/ come
from them) and of its refusal to run on more than one GPU."""
import csv
import subprocess
import sys

import pytest

import bench

PREFILL = ("void sl8::(anonymous namespace)::attn_fwd_wide_kernel<128, true, 0, false, 1, 8, "
           "false, false>(sl8::(anonymous namespace)::FwdArgs)")


def test_short_kernel_name():
    assert bench._short_kernel_name(PREFILL) == bench.PREFILL_KERNEL
    assert bench._short_kernel_name("void at::native::(anonymous namespace)::k<float>(int)") == \
        "at::native::anon::k<float>"
    assert bench._short_kernel_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def _write_trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, t0, dur_ns in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": t0, "End_Timestamp": t0 + dur_ns})


def test_trace_summary_takes_the_last_steps_dispatches(tmp_path):
    # spin-up calls of 200 us, then 3 timed calls of 100, 110, 120 us
    rows = [(PREFILL, 1000 * i, 200_000) for i in range(5)]
    rows += [(PREFILL, 10_000_000 + 1_000_000 * i, 100_000 + 10_000 * i) for i in range(3)]
    rows += [("void sl8::(anonymous namespace)::other_kernel(int)", 5, 1000)]
    p = tmp_path / "t.csv"
    _write_trace(p, rows)
    out = bench.trace_summary(str(p), 3)
    assert "| attn_fwd_wide_kernel<128, true, 0, false, 1, 8, false, false> | 8 |" in out
    assert "| other_kernel | 1 |" in out
    assert "mean 110.00 us, median 110.00 us, min 100.00, max 120.00" in out
    assert "start-to-start spacing 1000.00 us" in out


def test_pmc_summary_sums_rows_per_dispatch(tmp_path):
    p = tmp_path / "c.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for d, vals in ((1, (1, 2)), (2, (3, 4)), (3, (10, 10))):  # two rows (XCDs) per dispatch
            for v in vals:
                w.writerow({"Dispatch_Id": d, "Kernel_Name": PREFILL, "Counter_Name": "FETCH_SIZE",
                            "Counter_Value": v})
    out = bench.pmc_summary(str(p))
    # per-dispatch sums 3, 7, 20: median 7, max 20
    assert "| attn_fwd_wide_kernel<128, true, 0, false, 1, 8, false, false> | 3 | 7 / 20 |" in out


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                       cwd=bench.HERE, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
