"""bench.py's rocprofv3 readers (--traffic-from, --trace-from) on synthetic
rocprofv3 CSV files: counter scaling by the calibration copy, per-phase
kernel averages, and the round trip of the machine-readable summary line
through load_profiles (matched on build id and workload)."""
from __future__ import annotations

import csv
import os

import pytest

import bench

BWD = "void klp::klp_bwd_kernel<0, 16, 2, true, false>(klp::BwdParams)"
FWD = "void klp::klp_fwd_kernel<0, 4, 4, false, false>(klp::FwdParams)"
COPY = "void klp::klp_ceiling_copy_kernel<16, 2>(klp::CeilingParams)"
READ = "void klp::klp_ceiling_read_kernel<4, 4>(klp::CeilingParams)"
FLUSH = "void at::native::reduce_kernel<512, 1, at::native::ReduceOp<long> >(...)"

COUNTER_COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id",
                "Thread_Id", "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size",
                "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
                "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp",
                "End_Timestamp"]
TRACE_COLS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id",
              "Kernel_Id", "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]


def _write(path, cols, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols, quoting=csv.QUOTE_NONNUMERIC)
        w.writeheader()
        for r in rows:
            w.writerow({c: r.get(c, 0) for c in cols})


def _counter_dir(tmp_path, name, counter, values):
    rows = []
    for i, (kernel, v) in enumerate(values):
        rows.append({"Dispatch_Id": i + 1, "Kernel_Name": kernel, "Counter_Name": counter,
                     "Counter_Value": v})
    d = tmp_path / name
    _write(str(d / "host" / "123" / "run_counter_collection.csv"), COUNTER_COLS, rows)
    return str(d)


def test_traffic_scaled_by_the_calibration_copy(tmp_path):
    N, V, esz = bench._workload_sizes("C2")
    copy_kib = bench.ceiling_row_bytes(V, esz) * N / 1024
    # FETCH_SIZE reads half of the bytes read (as on the gfx950 box); WRITE_SIZE is exact.
    fetch = _counter_dir(tmp_path, "f", "FETCH_SIZE", [
        (COPY, copy_kib / 2), (COPY, copy_kib / 2), (BWD, 152100.0), (BWD, 152102.0),
        (FWD, 152110.0), (FLUSH, 500000.0)])
    write = _counter_dir(tmp_path, "w", "WRITE_SIZE", [
        (COPY, copy_kib), (BWD, 304130.0), (FWD, 96.0), (FLUSH, 1.0)])
    md, data = bench.summarize_traffic(fetch, write, "C2")
    assert data["fetch_factor"] == pytest.approx(2.0)
    assert data["write_factor"] == pytest.approx(1.0)
    k = data["kernels"]
    assert set(k) == {"klp_ceiling_copy_kernel<16, 2>", "klp_bwd_kernel<0, 16, 2, true, false>",
                      "klp_fwd_kernel<0, 4, 4, false, false>"}
    bwd = k["klp_bwd_kernel<0, 16, 2, true, false>"]
    assert bwd["traffic_bytes"] == round(1024 * (152101.0 * 2 + 304130.0))
    _, bb = bench.algorithmic_bytes(N, V, esz)
    assert bwd["algorithmic_bytes"] == bb
    assert bwd["ratio"] == pytest.approx(bwd["traffic_bytes"] / bb, abs=1e-4)
    assert k["klp_ceiling_copy_kernel<16, 2>"]["ratio"] == pytest.approx(1.0)
    assert "| `klp_bwd_kernel<0, 16, 2, true, false>` |" in md


def test_traffic_needs_the_calibration(tmp_path):
    fetch = _counter_dir(tmp_path, "f", "FETCH_SIZE", [(BWD, 1.0)])
    write = _counter_dir(tmp_path, "w", "WRITE_SIZE", [(BWD, 1.0)])
    with pytest.raises(RuntimeError, match="calibration"):
        bench.summarize_traffic(fetch, write, "C2")


def test_trace_phases(tmp_path):
    # flush, fwd (flushed), fwd (back to back), bwd (after fwd), bwd (back to back),
    # flush, bwd (flushed), read ceiling (other: after bwd -> klp), unrelated kernel
    seq = [(FLUSH, 100), (FWD, 50), (FWD, 52), (BWD, 110), (BWD, 106), (FLUSH, 100),
           (BWD, 120), (READ, 45), ("void at::native::elementwise(...)", 5)]
    rows, t = [], 1000
    for i, (k, dur) in enumerate(seq):
        rows.append({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": i + 1, "Kernel_Name": k,
                     "Start_Timestamp": t, "End_Timestamp": t + dur * 1000})
        t += dur * 1000 + 500
    d = tmp_path / "trace"
    _write(str(d / "run_kernel_trace.csv"), TRACE_COLS, rows[::-1])  # any row order
    md, data = bench.summarize_trace(str(d), "C2")
    fwd = data["kernels"]["klp_fwd_kernel<0, 4, 4, false, false>"]
    bwd = data["kernels"]["klp_bwd_kernel<0, 16, 2, true, false>"]
    assert fwd["flushed"]["avg_ns"] == 50000 and fwd["back to back"]["avg_ns"] == 52000
    assert fwd["all"]["n"] == 2
    assert bwd["after another klp kernel"]["avg_ns"] == 110000
    assert bwd["back to back"]["avg_ns"] == 106000
    assert bwd["flushed"]["avg_ns"] == 120000
    assert bwd["all"]["avg_ns"] == pytest.approx((110000 + 106000 + 120000) / 3, abs=0.1)
    N, V, esz = bench._workload_sizes("C2")
    _, bb = bench.algorithmic_bytes(N, V, esz)
    assert bwd["flushed"]["tbps"] == pytest.approx(bb / 120e-6 / 1e12, abs=1e-4)
    assert data["kernels"]["klp_ceiling_read_kernel<4, 4>"]["after another klp kernel"]["n"] == 1


def test_summary_round_trip(tmp_path, monkeypatch):
    d = tmp_path / "trace"
    _write(str(d / "run_kernel_trace.csv"), TRACE_COLS,
           [{"Kind": "KERNEL_DISPATCH", "Kernel_Name": BWD, "Start_Timestamp": 0,
             "End_Timestamp": 100000}])
    md, data = bench.summarize_trace(str(d), "C2", command="rocprofv3 ... -- python3 bench.py")
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "klp_C2_trace.md").write_text(md)
    monkeypatch.setattr(bench, "PROFILES_DIR", str(prof))
    got = bench.load_profiles("trace", "C2", bench.build_id())
    assert len(got) == 1 and got[0]["kernels"] == data["kernels"]
    assert bench.load_profiles("trace", "C2", "0000000000000000") == []
    assert bench.load_profiles("trace", "C3", bench.build_id()) == []
    assert bench.load_profiles("traffic", "C2", bench.build_id()) == []


def test_build_id_tracks_the_sources(tmp_path, monkeypatch):
    a = bench.build_id()
    assert a == bench.build_id() and len(a) == 16
    src = tmp_path / "pkg" / "csrc"
    src.mkdir(parents=True)
    (src / "k.hip").write_text("one")
    (tmp_path / "pkg" / "Makefile").write_text("all:")
    monkeypatch.setattr(bench, "PKG_DIR", str(tmp_path / "pkg"))
    b = bench.build_id()
    (src / "k.hip").write_text("two")
    assert bench.build_id() != b


def test_short_kernel_names():
    assert bench.short_kernel(BWD) == "klp_bwd_kernel<0, 16, 2, true, false>"
    assert bench.short_kernel("void klp::klp_fwd_shard_merge_kernel(klp::ShardMergeParams)") == \
        "klp_fwd_shard_merge_kernel"
    assert bench.short_kernel("void klp::(anonymous namespace)::klp_scale_kernel"
                              "(klp::ScaleParams)") == "klp_scale_kernel"
    assert bench.short_kernel("void klp::klp_grpo_token_weights_kernel<0, unsigned char>"
                              "(klp::TokenWeightsParams)") == \
        "klp_grpo_token_weights_kernel<0, unsigned char>"


def test_labelled_trace_is_not_the_configs(tmp_path, monkeypatch):
    """A run that mixes shapes (--label): tagged with the label, so the bench
    line's trace_check does not read it as the config's, and without TB/s."""
    d = tmp_path / "trace"
    _write(str(d / "run_kernel_trace.csv"), TRACE_COLS,
           [{"Kind": "KERNEL_DISPATCH", "Kernel_Name": BWD, "Start_Timestamp": 0,
             "End_Timestamp": 100000}])
    md, data = bench.summarize_trace(str(d), "C2", label="C2-grpo-run")
    assert data["config"] == "C2-grpo-run"
    assert data["kernels"]["klp_bwd_kernel<0, 16, 2, true, false>"]["all"]["tbps"] is None
    assert "--label C2-grpo-run" in md
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "klp_C2_grpo_trace.md").write_text(md)
    monkeypatch.setattr(bench, "PROFILES_DIR", str(prof))
    assert bench.load_profiles("trace", "C2", bench.build_id()) == []
    assert len(bench.load_profiles("trace", "C2-grpo-run", bench.build_id())) == 1


def test_matrix_traffic_groups_dispatches_between_markers(tmp_path):
    """--matrix-traffic-from: the calibration copy scales each counter; the
    dispatches after marker i (klp_ceiling_write) and before marker i + 1
    are backend i's; dispatches before the copy (warm-up) and after the last
    marker are not counted."""
    BS, V = bench.MATRIX_TRAFFIC_SHAPE
    lb = BS * V * 2
    MARK = "void klp::klp_ceiling_write_kernel<1, 2>(klp::CeilingParams)"
    NAIVE = "void klp::klp_fwd_naive_kernel<0>(klp::NaiveParams)"
    SOFT = "void at::native::softmax_kernel(...)"
    kib = lb / 1024

    def seq(fetch):
        # warm-up, calibration copy, then per backend: marker + its kernels
        f = 0.5 if fetch else 1.0
        s = [(FWD, 1e9), (COPY, kib * f),
             (MARK, 0.0), (FWD, kib * f),
             (MARK, 0.0), (BWD, kib * f) if fetch else (BWD, kib * f),
             (MARK, 0.0), (NAIVE, kib * f),
             (MARK, 0.0)] + [(SOFT, kib * f)] * 9 + [
             (MARK, 0.0), (SOFT, kib * f), (SOFT, 2 * kib * f),
             (MARK, 0.0), (FWD, 1e9)]
        return s
    fetch = _counter_dir(tmp_path, "f", "FETCH_SIZE", seq(True))
    write = _counter_dir(tmp_path, "w", "WRITE_SIZE", seq(False))
    md, data = bench.summarize_matrix_traffic(fetch, write)
    b = data["backends"]
    assert list(b) == list(bench.MATRIX_TRAFFIC_BACKENDS)
    assert b["ours_fwd"]["dispatches"] == 1
    assert b["ours_fwd"]["read_bytes"] == pytest.approx(lb, rel=1e-9)
    assert b["ours_fwd"]["amplification"] == pytest.approx(2.0)      # read + write of lb
    assert b["ours_bwd"]["required_bytes"] == 2 * lb
    assert b["ours_bwd"]["amplification"] == pytest.approx(1.0)
    assert b["trl_eager"]["dispatches"] == 9
    assert b["trl_eager"]["amplification"] == pytest.approx(18.0)
    assert b["pytorch_separate"]["dispatches"] == 2
    assert b["pytorch_separate"]["amplification"] == pytest.approx(6.0)
    assert "klp-profile" in md


def test_trace_agreement_divides_device_medians_by_the_trace():
    prof = {"file": "profiles/x.md", "kernels": {
        "klp_fwd_kernel<0, 8, 2, false, false>": {
            "back to back": {"avg_ns": 48600.0, "median_ns": 48500.0},
            "flushed": {"avg_ns": 48900.0, "median_ns": 48800.0}},
        "klp_bwd_kernel<0, 8, 2, true, false>": {
            "back to back": {"avg_ns": 102000.0, "median_ns": 102000.0}},
        "klp_ceiling_copy_kernel<8, 2>": {
            "back to back": {"avg_ns": 101000.0, "median_ns": 101000.0}}}}
    dev = {"fwd": {"warm": {"ms": 0.0485}, "flushed": {"ms": 0.0500}},
           "bwd": {"warm": {"ms": 0.0969}, "flushed": {"ms": 0.1}}}
    tc = bench.trace_agreement([prof], dev)
    assert tc["file"] == "profiles/x.md"
    assert tc["klp_fwd_kernel<0, 8, 2, false, false>"]["flushed"] == 48.9
    assert "klp_ceiling_copy_kernel<8, 2>" not in tc
    r = tc["bench_over_trace_median"]
    assert r["fwd"] == {"warm": 1.0, "flushed": round(50000 / 48800, 4)}
    assert r["bwd"] == {"warm": 0.95}  # no flushed phase in that trace
    assert bench.trace_agreement([], dev) is None
    no_dev = bench.trace_agreement([prof], None)
    assert "bench_over_trace_median" not in no_dev
    assert "ratio_over_trace" not in tc  # no read ceiling in the device figures


def test_trace_agreement_compares_ratios_to_the_ceilings():
    """ratio_over_trace: (bench fwd / read) / (trace fwd / read), likewise
    bwd / copy, per phase; a kernel with two launch shapes in the trace gives
    no ratio."""
    prof = {"file": "profiles/x.md", "kernels": {
        "klp_fwd_kernel<0, 8, 2, false, false>": {
            "back to back": {"avg_ns": 1.0, "median_ns": 48000.0},
            "flushed": {"avg_ns": 1.0, "median_ns": 48400.0}},
        "klp_ceiling_read_kernel<8, 2>": {
            "back to back": {"avg_ns": 1.0, "median_ns": 45000.0},
            "flushed": {"avg_ns": 1.0, "median_ns": 45500.0}},
        "klp_bwd_kernel<0, 4, 2, true, false>": {
            "flushed": {"avg_ns": 1.0, "median_ns": 98000.0}},
        "klp_ceiling_copy_kernel<4, 2>": {
            "flushed": {"avg_ns": 1.0, "median_ns": 104000.0}}}}
    dev = {"fwd": {"warm": {"ms": 0.0490}, "flushed": {"ms": 0.0495}},
           "read": {"warm": {"ms": 0.0450}, "flushed": {"ms": 0.0460}},
           "bwd": {"warm": {"ms": 0.0990}, "flushed": {"ms": 0.0985}},
           "copy": {"warm": {"ms": 0.1040}, "flushed": {"ms": 0.1050}}}
    r = bench.trace_agreement([prof], dev)["ratio_over_trace"]
    assert r["fwd_over_read"] == {
        "warm": round((0.0490 / 0.0450) / (48000 / 45000), 4),
        "flushed": round((0.0495 / 0.0460) / (48400 / 45500), 4)}
    assert r["bwd_over_copy"] == {"flushed": round((0.0985 / 0.1050) / (98000 / 104000), 4)}
    prof["kernels"]["klp_fwd_kernel<0, 16, 4, false, false>"] = \
        prof["kernels"]["klp_fwd_kernel<0, 8, 2, false, false>"]
    r2 = bench.trace_agreement([prof], dev)["ratio_over_trace"]
    assert "fwd_over_read" not in r2 and "bwd_over_copy" in r2


def test_configs_table_ranges_over_runs(tmp_path):
    import json

    def line(f, b):
        ceil = {"fwd_over_read": 1.07, "fwd_over_read_flushed": 1.075, "bwd_over_copy": 1.01,
                "bwd_over_read_plus_write": 1.02, "bwd_over_read_plus_write_flushed": 0.96}
        leg = {"fwd_us": f * 10, "fwd_us_flushed": f * 10, "fwd_pct_peak": 85.0,
               "fwd_pct_peak_flushed": 86.0, "bwd_us": b * 10, "bwd_us_flushed": b * 10,
               "bwd_pct_peak": 79.0, "bwd_pct_peak_flushed": 80.0, "step_us": (f + b) * 10,
               "ceilings": ceil}
        return {"build_id": "abc", "fwd_ms": f / 1e3, "fwd_ms_flushed": f / 1e3,
                "fwd_pct_peak": 80.0, "fwd_pct_peak_flushed": 79.0, "bwd_ms": b / 1e3,
                "bwd_ms_flushed": b / 1e3, "bwd_pct_peak": 76.0, "bwd_pct_peak_flushed": 77.0,
                "ms_per_step": (f + b) / 1e3, "ceilings": ceil, "configs": {"C3": leg},
                "C1": {"fwd_us": 7.0, "bwd_us": 11.5, "fwd_tbps": 4.8, "bwd_tbps": 5.7}}
    paths = []
    for i, (f, b) in enumerate(((48.1, 102.6), (48.5, 101.4))):
        p = tmp_path / f"b{i}.json"
        p.write_text("bench.py: noise\n" + json.dumps(line(f, b)) + "\n")
        paths.append(str(p))
    md = bench.configs_table(paths, "python bench.py")
    rows = {ln.split("|")[1].strip().split()[0]: ln for ln in md.splitlines()
            if ln.startswith("| C")}
    assert set(rows) == {"C1", "C2", "C3"}
    assert "48.10–48.50 / 48.10–48.50" in rows["C2"]
    assert "101.40–102.60" in rows["C2"]
    assert "481.00–485.00" in rows["C3"]
    assert "| 1.070, 1.075 |" in rows["C2"]
    assert "`abc`" in md and "python bench.py" in md


def test_counters_summed_per_dispatch_and_per_element(tmp_path):
    N, V, _ = bench._workload_sizes("C2")
    rows = []
    # Two dispatches of the forward, each reported as two shader-engine rows.
    for disp, (a, b) in ((1, (100.0, 300.0)), (2, (200.0, 200.0))):
        for v in (a, b):
            rows.append({"Dispatch_Id": disp, "Kernel_Name": FWD, "Counter_Name": "SQ_INSTS_VALU",
                         "Counter_Value": v})
        rows.append({"Dispatch_Id": disp, "Kernel_Name": FWD, "Counter_Name": "VALUBusy",
                     "Counter_Value": 50.0 + disp})
    rows.append({"Dispatch_Id": 3, "Kernel_Name": FLUSH, "Counter_Name": "SQ_INSTS_VALU",
                 "Counter_Value": 1e9})
    d = tmp_path / "cnt"
    _write(str(d / "host" / "1" / "x_counter_collection.csv"), COUNTER_COLS, rows)
    md, data = bench.summarize_counters(str(d), "C2", "rocprofv3 --pmc ...")
    k = bench.short_kernel(FWD)
    assert list(data["kernels"]) == [k]  # the non-klp kernel is left out
    assert data["kernels"][k]["dispatches"] == 2
    assert data["kernels"][k]["mean"] == {"SQ_INSTS_VALU": 400.0, "VALUBusy": 51.5}
    assert f"({400.0 * 64 / (N * V):.2f}/elem)" in md
    assert data["kind"] == "counters" and "rocprofv3 --pmc" in md
