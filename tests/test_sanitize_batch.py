"""The host-only part of jr_execute_dispatches (csrc/batch.cpp: batch checks
and the launch planner) and the spec parser it uses, built with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer and driven by
tests/sanitize/batch_check.cpp with fake contexts: the C4 six-job batch
under four sets of shape rules, the hazard batches of tests/test_gpu_mlp.py,
malformed dispatch arrays (short and null buffer lists, null and foreign
buffers, foreign kernels, wrong lengths, write aliases, empty batches) and
20000 seeded random batches. Any out-of-bounds access, use after free, leak
or undefined behaviour aborts the run."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "jade-compute_amd", "csrc")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ is not on PATH")
    exe = str(tmp_path_factory.mktemp("sanitize") / "batch_check")
    sources = [os.path.join(ROOT, "tests", "sanitize", "batch_check.cpp")] + [
        os.path.join(CSRC, f"{name}.cpp") for name in ("batch", "spec", "json", "refusal")]
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-Wall", "-Wextra", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
           *sources, "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def test_batch_planner_under_sanitizers(driver):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([driver], capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
    lines = dict(line.split(": ", 1) for line in run.stdout.splitlines() if ": " in line)
    assert lines["c4_all"] == "single:0 gate_up_swiglu:1 gemm_residual:4"
    assert lines["c4_fuse_only"] == "single:0 gate_up_swiglu:1 gemm_residual:4"
    assert lines["c4_pair_only"] == "single:0 pair:1 single:3 single:4 single:5"
    assert lines["swiglu_writes_gate_weights"] == "pair:0 single:2"
    for case in ("short_buffer_list", "null_buffer", "null_buffer_list", "foreign_kernel", "foreign_buffer",
                 "wrong_length", "output_aliases_input", "empty_batch", "zero_repeats", "no_time_output",
                 "null_jobs"):
        assert lines[case].startswith("refused"), (case, lines[case])
    assert lines["bad_later_job"].startswith("refused job 2")
    assert run.stdout.rstrip().endswith("ok") and "ERROR" not in run.stderr, run.stderr[-3000:]
