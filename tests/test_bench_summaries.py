"""bench.py's profile tooling on the host: the summaries that turn rocprofv3
CSV output into the committed profiles, and the stamp check that decides
whether roofline.traffic is reported. Synthetic CSVs in rocprofv3's column
layout; no GPU."""
import csv
import io
import json
import sys
from contextlib import redirect_stdout
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "jalapenos-at-home_amd"))

bench = pytest.importorskip("bench")


def _write_csv(path: Path, rows: list[dict]) -> None:
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def _run(kind: str, *dirs: Path) -> str:
    buf = io.StringIO()
    with redirect_stdout(buf):
        bench.summarize(kind, [str(d) for d in dirs])
    return buf.getvalue()


def _counter_rows(kernel: str, counter: str, values, first_id: int = 1) -> list[dict]:
    return [{"Dispatch_Id": first_id + i, "Kernel_Name": kernel, "Grid_Size": 65536, "Counter_Name": counter,
             "Counter_Value": v} for i, v in enumerate(values)]


def test_traffic_summary_calibrates_and_halves(tmp_path):
    """FETCH_SIZE is scaled by the 1 GiB copy's reading (here exactly half the
    bytes, factor 2), WRITE_SIZE by its own; per-step bytes are the two steps'
    sum halved; the hbm_bytes_per_step line carries their total."""
    gemv = "void mx4::gemv_m1_head_kernel<true, 1, 2, 2>(unsigned char const*)"
    fetch, write = tmp_path / "fetch", tmp_path / "write"
    for d, counter, per_launch, copy_kib in ((fetch, "FETCH_SIZE", 1000.0, 524288.0),
                                             (write, "WRITE_SIZE", 10.0, 1048576.0)):
        d.mkdir()
        rows = _counter_rows(gemv, counter, [per_launch] * 4)
        rows += _counter_rows("__amd_rocclr_copyBuffer", counter, [copy_kib], first_id=5)
        _write_csv(d / "x_counter_collection.csv", rows)
        (d / "stamp.json").write_text(json.dumps({"steps": 2, "bytes_per_step": 4_000_000,
                                                  "calibration_copy_bytes": 1 << 30, "library_sha256": "ab"}))
    out = _run("traffic", fetch, write)
    # fetch: 4 x 1000 KiB x 2 / 2 steps; write: 4 x 10 KiB x 1 / 2 steps
    want = int(round(4 * 1000 * 1024 * 2 / 2 + 4 * 10 * 1024 / 2))
    assert f"hbm_bytes_per_step: {want}" in out
    assert "library_sha256: ab" in out


def test_traffic_reported_only_for_the_stamped_library(tmp_path, monkeypatch):
    prof = tmp_path / "traffic.md"
    prof.write_text("commit: x\nlibrary_sha256: 1234\n\nhbm_bytes_per_step: 42\n")
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", prof)
    monkeypatch.setattr(bench, "library_sha256", lambda: "1234")
    assert bench.traffic_from_profile()[0] == 42
    monkeypatch.setattr(bench, "library_sha256", lambda: "9999")
    value, note = bench.traffic_from_profile()
    assert value is None and "!=" in note
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", tmp_path / "missing.md")
    assert bench.traffic_from_profile() == (None, "no traffic profile")


def test_verify_trace_splits_blocks_at_the_input_launch(tmp_path):
    """Each (projection, M) block opens with its input's synth launch; kernels
    per call and microseconds per call come from the block's GEMV/skinny
    dispatches; other kernels (weight synthesis) are ignored."""
    d = tmp_path / "verify"
    d.mkdir()
    rows, t = [], 0

    def add(name, us, grid=1024, wg=64):
        nonlocal t
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000),
                     "Grid_Size_X": grid * wg, "Workgroup_Size_X": wg})
        t += int(us * 1000) + 100
    add("mx4::synth_weight_kernel(unsigned long)", 50.0)
    add("mx4::synth_bf16_kernel(unsigned long)", 1.0)
    for _ in range(2 * 3):  # 2 copies x 3 repeats, one launch per call
        add("void mx4::gemv_m1_one_kernel<true, 1, 2, 2, false>(int)", 4.0)
    add("mx4::synth_bf16_kernel(unsigned long)", 1.0)
    for _ in range(2 * 3):  # two launches per call
        add("void mx4::(anonymous namespace)::skinny_kernel<true, 1, 4, 1, 8, true, 1>(int)", 10.0, 250, 512)
        add("void mx4::(anonymous namespace)::skinny_kernel<true, 1, 4, 1, 8, true, 1>(int)", 10.0, 250, 512)
    _write_csv(d / "v_kernel_trace.csv", rows)
    (d / "stamp.json").write_text(json.dumps({"plan": [["q", 1, 4096, 4096, 2, 3], ["q", 32, 4096, 4096, 2, 3]],
                                              "library_sha256": "cd"}))
    out = _run("verify-trace", d)
    lines = [ln for ln in out.splitlines() if ln.startswith("| q |")]
    assert len(lines) == 2
    assert "| 1 | gemv_m1_one_kernel<true, 1, 2, 2, false>, 1024 x 64 | 4.00 |" in lines[0]
    assert lines[1].count("skinny_kernel") == 2 and "| 20.00 |" in lines[1]


def test_verify_trace_rejects_a_plan_that_does_not_match(tmp_path):
    d = tmp_path / "verify"
    d.mkdir()
    _write_csv(d / "v_kernel_trace.csv", [{"Kernel_Name": "mx4::synth_bf16_kernel(int)", "Start_Timestamp": 0,
                                           "End_Timestamp": 1, "Grid_Size_X": 64, "Workgroup_Size_X": 64}])
    (d / "stamp.json").write_text(json.dumps({"plan": [["q", 1, 8, 8, 1, 1], ["q", 2, 8, 8, 1, 1]]}))
    with pytest.raises(SystemExit, match="blocks"):
        _run("verify-trace", d)


def test_prefill_compare_groups_dispatches_by_plan(tmp_path):
    """Counters are summed per dispatch over their per-instance rows and
    averaged over each plan entry's calls, in dispatch order."""
    d = tmp_path / "cmp"
    d.mkdir()
    k1 = "void mx4::(anonymous namespace)::prefill_kernel<false, 4, 3, 1, 4, 2, 2, 32>(int)"
    k2 = "void mx4::(anonymous namespace)::prefill_lds_kernel<false, 2, 2, 2, 3, 4, 2>(int)"
    rows = []
    for i in range(2):
        for _ in range(2):  # one row per XCD sample: summed per dispatch
            rows.append({"Dispatch_Id": 1 + i, "Kernel_Name": k1, "Grid_Size": 65536, "Counter_Name": "SQ_WAVES",
                         "Counter_Value": 512.0})
    for i in range(2):
        rows.append({"Dispatch_Id": 3 + i, "Kernel_Name": k2, "Grid_Size": 65536, "Counter_Name": "SQ_WAVES",
                     "Counter_Value": 100.0 * (i + 1)})
    _write_csv(d / "c_counter_collection.csv", rows)
    (d / "stamp.json").write_text(json.dumps({"plan": [["gate", "register-direct", [0, 0, 0]],
                                                       ["gate", "shared", [128, 192, 66]]],
                                              "calls_per_instance": 2, "library_sha256": "ef"}))
    out = _run("prefill-compare", d)
    assert "| gate | register-direct | 1024 |" in out  # two rows of 512 per dispatch
    assert "| gate | shared | 150 |" in out           # mean of 100 and 200


def test_prefill_summary_is_compact_and_reads_the_stamped_counters(tmp_path, monkeypatch):
    """The top-level `prefill` object of the JSON line: every 8B shape and
    activation format in one row, the grouped layer, the largest
    requantization error, and the MFMA counters of the dominant instances
    taken from the profile only when its stamp names the loaded library; the
    whole object stays under 1.5 KB so a record keeping top-level keys keeps it."""
    prof = tmp_path / "prefill.md"
    prof.write_text(
        "commit: x\nlibrary_sha256: 1234\n\n"
        "| shape | act | kernel instance | dispatches | us | TFLOP/s | of peak | MOPS x 512 | MFMA busy |\n"
        "|---|---|---|---|---|---|---|---|---|\n"
        "| gate 512x4096->12288 | mxfp4 | prefill_kernel<false, 4, 3, 1, 4, 2, 2, 32> | 10 | 18.38 | 2804 | 27.8% "
        "| 5.154e+10 (1.000 x 2MNK) | 27.9% |\n"
        "| gate 512x4096->12288 | exact bf16 | gemm_exact_kernel<true, 2, 2, 2, 3, 3> | 5 | 54.35 | 948 | 37.9% "
        "| 5.154e+10 (1.000 x 2MNK) | 37.7% |\n")
    monkeypatch.setattr(bench, "PREFILL_PROFILE", prof)
    monkeypatch.setattr(bench, "library_sha256", lambda: "1234")
    c = bench.prefill_counters()
    assert c["gate mxfp4"] == ["prefill_kernel<false,4,3,1,4,2,2,32>", 18.38, 1.0, 0.279]
    assert "gate exact" not in c
    monkeypatch.setattr(bench, "library_sha256", lambda: "9999")
    assert "!=" in bench.prefill_counters()["note"]

    def entry(us, tf):
        return {"us": us, "TFLOPs": tf, "frac": round(tf / 10100, 4), "frac_of_measured_ceiling": 0.3}
    err = {"max_rel": 1.2e-2, "rel_l2": 8.1e-3}
    pf = {name: {"mxfp4": {"gemm": entry(18.123, 2843.4), "requant+gemm": entry(24.5, 2100.0)},
                 "mxfp8": {"gemm": entry(23.3, 2211.0), "requant+gemm": entry(29.0, 1777.0)},
                 "requant_error": {"mxfp4": err, "mxfp8": {"max_rel": 2e-3, "rel_l2": 1e-3},
                                   "exact_auto": {"max_rel": 3e-7, "rel_l2": 1e-7}}}
          for name in ("q", "o", "gate", "up", "down")}
    layer = {a: {"grouped": {"us": 108.1, "frac": 0.181}} for a in ("mxfp4", "mxfp8")}
    monkeypatch.setattr(bench, "library_sha256", lambda: "1234")
    for key in ("down mxfp4", "gate mxfp8", "q mxfp4"):  # two more rows the summary keeps, one it drops
        shape, act = key.split()
        with open(prof, "a") as f:
            f.write(f"| {shape} 512x4096->4096 | {act} | prefill_lds_kernel<false, 2, 2, 2, 1, 2, 4, 2> | 10 | 11.36 "
                    "| 1513 | 15.0% | 1.718e+10 (1.000 x 2MNK) | 15.0% |\n")
    top = bench.prefill_summary(pf, layer, {"mxfp4": 6560.4, "mxfp8": 4120.0, "bf16": 1680.0})
    assert sorted(top["counters"]) == ["cols", "down mxfp4", "gate mxfp4", "gate mxfp8", "stamp"]
    assert top["mxfp4"]["gate"] == [18.123, 2843, 0.2815, 0.3, 24.5, 2100, 0.2079]
    assert top["requant_error_vs_unquantized"]["mxfp4"]["max_rel"] == 1.2e-2
    assert len(json.dumps(top)) < 1500
