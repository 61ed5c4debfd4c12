"""bench.py's host logic, on the CPU: the algorithmic byte counts of each
benchmarked configuration (1,088 cache bytes per token at d = 128 and 8 kv
heads, plus tables, q and out), the one-GPU refusal, and the PMC and
kernel-trace summaries on small synthetic rocprofv3 CSV files."""
import csv
import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
import bench  # noqa: E402


def test_algorithmic_bytes_match_the_baseline_table():
    # the A8 strip, the 1024-token BF16 writer, and the decode at ctx 4096,
    # 16384, 32768 and the ragged 4103
    assert bench.writer_algorithmic_bytes(16, 8, 128, 1) == 50_240
    assert bench.writer_algorithmic_bytes(1024, 8, 128, 2) == 5_312_512
    for ctx, want in ((4096, 4_473_860), (16384, 17_846_276), (32768, 35_676_164),
                      (4103, 4_481_480)):
        assert bench.decode_algorithmic_bytes([ctx], 32, 8, 128, 16) == want
    # 1,088 cache bytes per token at d = 128, 8 kv heads
    assert (bench.decode_algorithmic_bytes([8192], 32, 8, 128, 16)
            - bench.decode_algorithmic_bytes([4096], 32, 8, 128, 16)) == 4096 * 1088 + 256 * 4


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _write_counters(path, rows):
    cols = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
            "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
            "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
            "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, cols)
        w.writeheader()
        for i, (name, grid, counter, value) in enumerate(rows):
            w.writerow({c: 0 for c in cols} | {"Dispatch_Id": i, "Grid_Size": grid * 256,
                                               "Workgroup_Size": 256, "Kernel_Name": name,
                                               "Counter_Name": counter, "Counter_Value": value})


def test_pmc_summary_scales_by_the_calibration_copy(tmp_path, monkeypatch):
    """Each row's dispatches (its kernel and grid) are averaged over the passes
    of its own directory and scaled by that run's plain copy."""
    monkeypatch.setattr(bench, "PMC_FILE", str(tmp_path / "pmc.json"))
    copy = "void at::native::vectorized_elementwise_kernel<4, MulFunctor<float> >"
    dec = "void tq4::(anonymous namespace)::decode_kernel<128, 1>(tq4::DecodeParams)"
    cal_kib = bench.CALIB_BYTES / 1024
    row = tmp_path / "configs2_decode"
    _write_counters(str(row / "p1" / "run_counter_collection.csv"), [
        (copy, 4096, "FETCH_SIZE", cal_kib / 2),  # the counter reads half the bytes
        (copy, 64, "FETCH_SIZE", 1.0),            # a smaller multiply is not the copy
        (dec, 128, "FETCH_SIZE", 1000.0), (dec, 128, "FETCH_SIZE", 3000.0),
        (dec, 16, "FETCH_SIZE", 7.0)])           # another grid: not this row's kernel
    _write_counters(str(row / "p2" / "run_counter_collection.csv"), [
        (copy, 4096, "WRITE_SIZE", cal_kib), (dec, 128, "WRITE_SIZE", 100.0),
        (dec, 16, "WRITE_SIZE", 1.0)])
    sw = tmp_path / "sweep_ctx4096_K2"
    _write_counters(str(sw / "p1" / "run_counter_collection.csv"), [
        (copy, 4096, "FETCH_SIZE", cal_kib), (dec, 16, "FETCH_SIZE", 7.0)])
    _write_counters(str(sw / "p2" / "run_counter_collection.csv"), [
        (copy, 4096, "WRITE_SIZE", cal_kib), (dec, 16, "WRITE_SIZE", 1.0)])
    bench.summarize_pmc(str(tmp_path))
    out = json.load(open(tmp_path / "pmc.json"))
    e = out["configs2_decode"]
    assert e["calibration"]["fetch_scale"] == pytest.approx(2.0)
    assert e["calibration"]["write_scale"] == pytest.approx(1.0)
    assert e["dispatches"] == 2 and e["workgroups"] == 128
    assert e["fetch_bytes"] == pytest.approx(2000.0 * 1024 * 2)
    assert e["write_bytes"] == pytest.approx(100.0 * 1024)
    assert out["sweep_ctx4096_K2"]["fetch_bytes"] == pytest.approx(7.0 * 1024)
    r = bench.roofline(4_473_860, 0.01, "configs2_decode", out)
    assert r["traffic"] == round(e["traffic_bytes"])
    assert r["frac"] == pytest.approx(4_473_860 / 1e-5 / 1e9 / 8000, abs=1e-4)


def test_pmc_summary_keeps_committed_rows_only_when_merging(tmp_path, monkeypatch):
    """Summarising a run of some rows over a summary that holds others is
    refused unless merging, which keeps the others and replaces the re-run."""
    pmc = tmp_path / "pmc.json"
    monkeypatch.setattr(bench, "PMC_FILE", str(pmc))
    pmc.write_text(json.dumps({"configs1_writer": {"kernel": "w", "workgroups": 512,
                                                   "dispatches": 8, "counters": {}},
                               "rms_writer": {"kernel": "old", "workgroups": 1024,
                                              "dispatches": 8, "counters": {}}}))
    copy = "void at::native::vectorized_elementwise_kernel<4, MulFunctor<float> >"
    rms = "void tq4::(anonymous namespace)::rms_writer<128, 1>(tq4::RmsParams)"
    cal_kib = bench.CALIB_BYTES / 1024
    runs = tmp_path / "runs"
    _write_counters(str(runs / "rms_writer" / "p1" / "run_counter_collection.csv"), [
        (copy, 4096, "FETCH_SIZE", cal_kib), (rms, 1024, "FETCH_SIZE", 5.0)])
    with pytest.raises(SystemExit, match="configs1_writer"):
        bench.summarize_pmc(str(runs))
    assert json.loads(pmc.read_text())["rms_writer"]["kernel"] == "old"  # untouched
    bench.summarize_pmc(str(runs), merge=True)
    out = json.loads(pmc.read_text())
    assert set(out) == {"configs1_writer", "rms_writer"}
    assert out["rms_writer"]["kernel"] != "old" and out["configs1_writer"]["kernel"] == "w"


def test_trace_summary_limits_per_kernel_and_grid(tmp_path, capsys):
    cols = ["Kernel_Name", "Dispatch_Id", "Start_Timestamp", "End_Timestamp", "Grid_Size_X",
            "Grid_Size_Y", "Grid_Size_Z", "Workgroup_Size_X", "Workgroup_Size_Y",
            "Workgroup_Size_Z"]
    path = tmp_path / "t" / "bench_kernel_trace.csv"
    os.makedirs(path.parent)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, cols)
        w.writeheader()
        for i, us in enumerate([8, 9, 10, 11, 50, 60]):  # two slow ones after the first four
            w.writerow({"Kernel_Name": "void k<1>(int)", "Dispatch_Id": i,
                        "Start_Timestamp": 1000 * i * 100, "End_Timestamp": 1000 * (i * 100 + us),
                        "Grid_Size_X": 256 * 4, "Grid_Size_Y": 2, "Grid_Size_Z": 1,
                        "Workgroup_Size_X": 256, "Workgroup_Size_Y": 1, "Workgroup_Size_Z": 1})
    bench.summarize_trace(str(tmp_path), limit=4)
    line = [ln for ln in capsys.readouterr().out.splitlines() if "k<1>" in ln][0]
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1] == "8" and cells[2] == "4"  # 4 x 2 workgroups, 4 dispatches kept
    assert float(cells[3]) == pytest.approx(9.5)


def test_decode_overhead_bytes_closed_form():
    """The workspace traffic reported beside the algorithmic bytes: (3 k_live
    - 1) records of (d + 4) floats per q head of every (seq, kv head) with
    more than one live split; none for a single split or a short sequence."""
    import bench
    rec = (128 + 4) * 4
    # 16 live splits, 8 kv heads x 4 q heads
    assert bench.decode_overhead_bytes([4096], 32, 8, 128, 16, 16, 256) == 8 * 47 * 4 * rec
    assert bench.decode_overhead_bytes([4096], 32, 8, 128, 16, 1, 256) == 0
    # a sequence inside the first split's window, and one reaching three splits
    assert bench.decode_overhead_bytes([100, 2 * 16 * 16 + 1], 32, 8, 128, 16, 16, 256) == \
        8 * (3 * 3 - 1) * 4 * rec
