"""bench.py's harness on the CPU: its rocprofv3 summaries on synthetic
profiler CSVs (the HBM counter calibration against the copy kernel, the
per-(kernel, grid, workgroup, workload) traffic table, the lookup that fills
the bench line's `roofline.traffic`, the split of one symbol's trace rows by
shape) and the time-based pre-heat on a stand-in runtime."""
import csv
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def write_csv(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        writer.writeheader()
        writer.writerows(rows)


SYMBOL = "void jade::hipk::(anonymous namespace)::{}(float const*, float*)"
# Two instantiations with the same work-item count (1024x256 and 256x1024),
# as the 4096^3 and 1024^3 GEMM launches have.
KERNELS = [("copy_stream", 16777216, 256), ("gemm_f32_mfma<2, 2, true, 1, 1>", 262144, 256),
           ("gemm_f32_mfma<1, 1, true, 1, 4>", 262144, 1024)]


def make_profile(bench, tmp_path):
    trace, fetch, write = [], [], []
    copy_kib = bench.COPY_ELEMENTS * 4 / 1024.0
    # Counter readings: the copy reads half and writes its true size, so the
    # calibration scales FETCH_SIZE by 2 and WRITE_SIZE by 1.
    readings = {"copy_stream": (copy_kib / 2, copy_kib), "gemm_f32_mfma<2, 2, true, 1, 1>": (1000.0, 500.0),
                "gemm_f32_mfma<1, 1, true, 1, 4>": (100.0, 50.0)}
    for dispatch, (name, items, block) in enumerate(KERNELS * 2):
        full = SYMBOL.format(name)
        trace.append({"Kernel_Name": full, "Grid_Size_X": items // block, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
                      "Workgroup_Size_X": block, "Start_Timestamp": 1000, "End_Timestamp": 3000 + dispatch})
        for rows, counter, value in ((fetch, "FETCH_SIZE", readings[name][0]),
                                     (write, "WRITE_SIZE", readings[name][1])):
            rows.append({"Dispatch_Id": dispatch, "Kernel_Name": full, "Grid_Size": items, "Workgroup_Size": block,
                         "Counter_Name": counter, "Counter_Value": value})
    write_csv(str(tmp_path / "trace" / "run_kernel_trace.csv"), trace)
    write_csv(str(tmp_path / "fetch" / "w" / "run_counter_collection.csv"), fetch)
    write_csv(str(tmp_path / "write" / "w" / "run_counter_collection.csv"), write)
    return bench.summarize_rocprof(str(tmp_path / "trace"), str(tmp_path / "fetch"), str(tmp_path / "write"))


def test_traffic_table_is_keyed_by_workgroup_and_calibrated(bench, tmp_path):
    text, traffic = make_profile(bench, tmp_path)
    assert "scale FETCH_SIZE x2.0000, WRITE_SIZE x1.0000" in text
    # Keys carry the workload: the name of the directory of the counter run.
    assert set(traffic) == {"copy_stream@16777216@256@w", "gemm_f32_mfma<2, 2, true, 1, 1>@262144@256@w",
                            "gemm_f32_mfma<1, 1, true, 1, 4>@262144@1024@w"}
    assert traffic["gemm_f32_mfma<2, 2, true, 1, 1>@262144@256@w"]["bytes_per_launch"] == pytest.approx(
        (1000.0 * 2 + 500.0) * 1024)
    assert traffic["copy_stream@16777216@256@w"]["bytes_per_launch"] == pytest.approx(2 * bench.COPY_ELEMENTS * 4)


def test_traffic_lookup_picks_the_launched_instantiation(bench, tmp_path, monkeypatch):
    _, traffic = make_profile(bench, tmp_path)
    import json

    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "traffic.json").write_text(json.dumps(traffic))
    monkeypatch.setattr(bench, "PROFILE_DIR", str(tmp_path / "profiles"))
    big = bench.traffic_from_profiles("gemm_f32_mfma", {"grid": [1024, 1, 1], "block": [256, 1, 1]}, "w")
    small = bench.traffic_from_profiles("gemm_f32_mfma", {"grid": [256, 1, 1], "block": [1024, 1, 1]}, "w")
    assert big == pytest.approx(2500.0 * 1024) and small == pytest.approx(250.0 * 1024)
    # Another workload's run, no entry, or a prefix that names two
    # instantiations of one launch shape: no figure.
    assert bench.traffic_from_profiles("gemm_f32_mfma", {"grid": [1024, 1, 1], "block": [256, 1, 1]}, "x") is None
    assert bench.traffic_from_profiles("gemm_f32_mfma", {"grid": [7, 1, 1], "block": [256, 1, 1]}, "w") is None
    traffic["gemm_f32_mfma<9, 9, true, 1, 1>@262144@256@w"] = {"bytes_per_launch": 1.0}
    (tmp_path / "profiles" / "traffic.json").write_text(json.dumps(traffic))
    assert bench.traffic_from_profiles("gemm_f32_mfma", {"grid": [1024, 1, 1], "block": [256, 1, 1]}, "w") is None


def test_persistent_gemm_rows_split_by_shape(bench, tmp_path):
    # One symbol at one grid for three shapes: each dispatch goes to the shape
    # whose event-timed median is nearest, or stays unassigned beyond 25%.
    ring = SYMBOL.format("gemm_f32_ring<1, true>")
    durations_us = [935, 940, 2540, 120, 125, 180, 3300]
    trace = [{"Kernel_Name": ring, "Grid_Size_X": 256, "Grid_Size_Y": 1, "Grid_Size_Z": 1, "Workgroup_Size_X": 512,
              "Start_Timestamp": 0, "End_Timestamp": int(d * 1000)} for d in durations_us]
    write_csv(str(tmp_path / "trace" / "run_kernel_trace.csv"), trace)
    line = {"metric": "m", "gpu_kernel": {"m": 4096, "n": 4096, "k": 4096, "kernel": "gemm_f32_ring_128x128x32",
                                          "ms_per_step": 0.936},
            "extra": {"gemm_sweep": {"2048x2048x2048": {"ms": 0.122, "kernel": "gemm_f32_ring_128x128x32"},
                                     "4096x11008x4096": {"ms": 2.54, "kernel": "gemm_f32_ring_128x128x32"},
                                     "512x512x512": {"ms": 0.0064, "kernel": "gemm_f32_direct_32x32x32_w4"}}}}
    log = tmp_path / "bench.log"
    log.write_text("device: test\n" + __import__("json").dumps(line) + "\n")
    text, _ = bench.summarize_rocprof(str(tmp_path / "trace"), bench_log=str(log))
    rows = {ln.split("|")[1].strip(): ln.split("|")[4].strip() for ln in text.splitlines()
            if ln.startswith("| gemm_f32_ring")}
    assert rows == {"gemm_f32_ring<1, true> [4096x4096x4096]": "2", "gemm_f32_ring<1, true> [4096x11008x4096]": "1",
                    "gemm_f32_ring<1, true> [2048x2048x2048]": "2", "gemm_f32_ring<1, true> [unassigned]": "2"}


def test_vendor_workload_shapes_split_the_trace(bench, tmp_path):
    # `--workload vendor` prints no headline: its line holds only `extra`, and
    # this library's side of each shape names the shapes the trace rows of
    # the persistent kernel are split by. The string entry is not a shape.
    line = {"metric": "m", "workload": "vendor",
            "extra": {"vendor_gemm": {"4096x4096x4096": {"ms": 0.915, "kernel": "gemm_f32_ring_128x128x32"},
                                      "1024x1024x1024": {"ms": 0.0205, "kernel": "gemm_f32_mfma_64x64x32_k4"},
                                      "vendor": "torch.matmul FP32"}}}
    log = tmp_path / "vendor.log"
    log.write_text(__import__("json").dumps(line) + "\n")
    assert bench.bench_gemm_launches(str(log)) == [("4096x4096x4096", "gemm_f32_ring_128x128x32", 0.915),
                                                   ("1024x1024x1024", "gemm_f32_mfma_64x64x32_k4", 0.0205)]
    assert set(bench.VENDOR_SHAPES) >= {(4096, 4096, 4096), (4096, 1024, 2816), (4096, 2816, 1024)}


def test_mfma_summary_reports_busy_share_and_clock(bench, tmp_path):
    # Eight XCDs of 2.4e6 GUI cycles each over a 1 ms dispatch: 2.4 GHz. Busy
    # cycles of 0.9 x 2.4e6 per SIMD on 1024 SIMDs: 90% busy.
    name = SYMBOL.format("gemm_f32_ring<1, true>")
    rows = []
    for dispatch in range(3):
        start = 10_000_000 * dispatch
        for counter, value in (("GRBM_GUI_ACTIVE", 8 * 2.4e6), ("SQ_VALU_MFMA_BUSY_CYCLES", 0.9 * 2.4e6 * 1024)):
            rows.append({"Dispatch_Id": dispatch, "Kernel_Name": name, "Grid_Size": 131072, "Workgroup_Size": 512,
                         "Counter_Name": counter, "Counter_Value": value, "Start_Timestamp": start,
                         "End_Timestamp": start + 1_000_000})
    write_csv(str(tmp_path / "pmc" / "4096x4096x2048" / "run_counter_collection.csv"), rows)
    line = [ln for ln in bench.summarize_mfma(str(tmp_path / "pmc")).splitlines() if ln.startswith("| gemm")][0]
    cells = [x.strip() for x in line.split("|")[1:-1]]
    assert cells[1] == "4096x4096x2048" and cells[4] == "3"
    assert cells[7] == "90.0%" and cells[8] == "2.400"


def test_preheat_follows_the_command_line_value(bench, monkeypatch):
    # --preheat-ms replaces the module-level PREHEAT_MS after the classes are
    # defined; the pre-heat must read it when it runs.
    class Execution:
        gpu_ms, host_ms = 1.5, 1.5

    class FakeRuntime:
        def __init__(self):
            self.calls = []

        def execute(self, jobs, repeats):
            self.calls.append(repeats)
            result = Execution()
            result.gpu_ms = 1.5 * repeats
            return result

    for target, want_calls in ((0.0, []), (10.0, [1, 2, 4])):
        monkeypatch.setattr(bench, "PREHEAT_MS", target)
        rt = FakeRuntime()
        work = bench.Workload(rt, [], 1)
        work.preheat()
        assert rt.calls == want_calls and work.preheat_ms >= target


def test_short_workloads_sample_at_least_a_millisecond(bench, monkeypatch):
    # Outside the headline a sample holds enough steps for MIN_SAMPLE_MS of
    # device time (estimated from the pre-heat), so the idle queue's dispatch
    # latency, paid once per sample, is spread over many launches; the
    # headline (min_repeats 1) times exactly the requested steps.
    class Execution:
        def __init__(self, repeats):
            self.gpu_ms = self.host_ms = 0.006 * repeats

    class FakeRuntime:
        def __init__(self):
            self.calls = []

        def execute(self, jobs, repeats):
            self.calls.append(repeats)
            return Execution(repeats)

    monkeypatch.setattr(bench, "PREHEAT_MS", 5.0)
    rt = FakeRuntime()
    out = bench.measure({"w": bench.Workload(rt, [], 1)}, 50, 0)
    assert out["w"]["sample_steps"] == [167] * bench.SAMPLES
    assert out["w"]["ms_per_step"] == pytest.approx(0.006)
    rt = FakeRuntime()
    out = bench.measure({"w": bench.Workload(rt, [], 1)}, 50, 0, min_repeats=1)
    assert sum(out["w"]["sample_steps"]) == 50
    monkeypatch.setattr(bench, "PREHEAT_MS", 0.0)
    rt = FakeRuntime()
    out = bench.measure({"w": bench.Workload(rt, [], 1)}, 50, 0)
    assert out["w"]["sample_steps"] == [10] * bench.SAMPLES
