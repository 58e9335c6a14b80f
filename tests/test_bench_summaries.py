"""The arithmetic of bench.py's summaries, which turn rocprofv3 and amd-smi
output into the committed profiles' numbers: sampled power and clock per
phase, HBM bytes per launch scaled by the calibration kernel, and the clock
and MFMA-busy share per operand case. Synthetic inputs of the tools' formats,
with answers worked out by hand. CPU only."""
from __future__ import annotations

import csv
import importlib.util
import json
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _smi(power, clocks):
    """The part of `amd-smi metric -g 0 -p -c --json` the summary reads."""
    return {"gpu_data": [{"gpu": 0, "power": {"socket_power": {"value": power, "unit": "W"}},
                          "clock": {f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"},
                                                 "max_clk": {"value": 2400, "unit": "MHz"}}
                                    for i, c in enumerate(clocks)}}]}


def test_sustain_summary_averages_samples_inside_each_phase(bench, tmp_path, capsys):
    phases = tmp_path / "phases.log"
    phases.write_text("\n".join(json.dumps(p) for p in [
        {"phase": "idle", "t0": 100.0, "t1": 102.0},
        {"phase": "workload data", "t0": 102.0, "t1": 110.0, "launches": 10, "TFLOP/s": 1000.0},
    ]) + "\n")
    samples = [
        (101.5, 300, [2400, 2400]),          # idle, after its first second
        (102.5, 9999, [100, 100]),           # the phase's first second: left out
        (104.0, 1380, [1700, 1760]),
        (108.0, 1390, [1720, 1740]),
        (111.0, 5000, [100, 100]),           # after the phase
    ]
    smi = tmp_path / "smi.log"
    with open(smi, "w") as f:
        for t, p, c in samples:
            f.write(f"T {t}\n{json.dumps(_smi(p, c), indent=2)}\n")
        f.write("T 112.0\nnot json\n")     # a sample amd-smi failed to print is skipped
    assert bench.sustain_summary(str(phases), str(smi)) == 0
    out = {r["phase"]: r for r in json.loads(capsys.readouterr().out)}
    assert out["idle"]["samples"] == 1 and out["idle"]["socket_power_W"] == 300.0
    wl = out["workload data"]
    assert wl["samples"] == 2 and wl["TFLOP/s"] == 1000.0
    assert wl["socket_power_W"] == 1385.0                        # (1380 + 1390) / 2
    assert wl["gfx_clock_mhz"] == 1730.0                         # the mean of the four XCD readings


def _counter_csv(path, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_traffic_summary_scales_by_the_calibration_kernel(bench, tmp_path, capsys):
    calib_bytes = bench.CALIB_FLOATS * 4.0
    # the counters read half the calibration kernel's true bytes: factor 2
    for counter, gemm_kib in (("FETCH_SIZE", [100.0, 300.0]), ("WRITE_SIZE", [50.0, 50.0])):
        rows = [{"Dispatch_Id": i, "Kernel_Name": "void gemm_kernel<...>", "Counter_Name": counter,
                 "Counter_Value": v} for i, v in enumerate(gemm_kib)]
        rows.append({"Dispatch_Id": 9, "Kernel_Name": "void scale_kernel<...>", "Counter_Name": counter,
                     "Counter_Value": calib_bytes / 2 / 1024})
        _counter_csv(tmp_path / counter / "run_counter_collection.csv", rows)
    assert bench.traffic_summary(str(tmp_path / "FETCH_SIZE"), str(tmp_path / "WRITE_SIZE")) == 0
    line = json.loads(capsys.readouterr().out)
    assert line["fetch"]["factor"] == pytest.approx(2.0)
    assert line["fetch"]["bytes_per_launch"] == pytest.approx(200.0 * 1024 * 2)
    assert line["write"]["bytes_per_launch"] == pytest.approx(50.0 * 1024 * 2)
    assert line["traffic_bytes_per_launch"] == pytest.approx(250.0 * 1024 * 2)


def test_activity_summary_clock_and_busy_per_case(bench, tmp_path, capsys, monkeypatch):
    # one shape, two cases, three timed launches after a warm one each
    monkeypatch.setattr(bench, "ACTIVITY_SHAPES", ((1024, 1024, 1024),))
    monkeypatch.setattr(bench, "ACTIVITY_CASES", ("a", "b"))
    monkeypatch.setattr(bench, "activity_reps", lambda m, n, k: 3)
    us = [10.0, 10.0, 10.0, 10.0, 20.0, 8.0, 8.0, 8.0]         # the 1st and 5th are the warm launches
    trace = tmp_path / "trace" / "run_kernel_trace.csv"
    trace.parent.mkdir(parents=True)
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 1_000_000
        for d in us:
            w.writerow({"Kernel_Name": "void gemm_kernel<...>", "Start_Timestamp": t, "End_Timestamp": t + int(d * 1e3)})
            t += 100_000
    rows = []
    for i, d in enumerate(us):
        ghz = 2.0 if i < 4 else 1.5
        rows.append({"Dispatch_Id": i, "Kernel_Name": "void gemm_kernel<...>", "Counter_Name": "GRBM_GUI_ACTIVE",
                     "Counter_Value": 8 * ghz * d * 1e3})     # summed over the 8 XCDs
        rows.append({"Dispatch_Id": i, "Kernel_Name": "void gemm_kernel<...>",
                     "Counter_Name": "SQ_VALU_MFMA_BUSY_CYCLES", "Counter_Value": 0.5 * 1024 * ghz * d * 1e3})
    _counter_csv(tmp_path / "pmc" / "run_counter_collection.csv", rows)
    assert bench.activity_summary(str(tmp_path / "pmc"), str(tmp_path / "trace")) == 0
    out = {r["case"]: r for r in json.loads(capsys.readouterr().out)}
    assert out["a"]["us"] == 10.0 and out["a"]["clock_ghz"] == 2.0 and out["a"]["mfma_busy_pct"] == 50.0
    assert out["b"]["us"] == 8.0 and out["b"]["clock_ghz"] == 1.5       # the 20 us warm launch left out
    assert out["b"]["TFLOP/s"] == pytest.approx(2.0 * 1024 ** 3 / 8.0 / 1e6, rel=1e-3)
