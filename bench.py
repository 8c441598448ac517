"""Benchmark for the MI355X Jade HIP backend (one GPU).

A step is one pass of the hot path over one batch of synthetic input. The
headline step (`value`) is the FP32 GEMM C = A.B at 4096^3 from BASELINE
configs[1], inputs from validation::inputs (xorshift32 seeds 0x12345678 /
0x9abcdef1, U[-1,1)), resident in HBM before timing. The same JSON line
carries the causal attention config (B4 H32 S4096 D128), attention C3, the
Softmax 32768x4096 bandwidth case, the six-op MLP block, the rest of the GEMM
sweep and the copy calibration.

Timing follows the reference's harness (src/runtime/metal_lab.rs:75-107,
179-187): each workload gets W untimed warm-up steps and a time-based
pre-heat (--preheat-ms of device time, reported as `preheat_ms`), then nine
consecutive samples, each timed by hipEvents around its launches on the
runtime's stream (the jr_execute scope,
native/jade_runtime_corex.cpp:148-189). The headline's samples split exactly
K timed steps; every other workload's samples hold at least the reference's
ten repeats each. The reported per-step time is the median sample; the mean
and the extremes are listed beside it. The two headline workloads are not
interleaved: after a few milliseconds of the attention kernel, the first
three to four 4096^3 GEMMs run 1-1.5% slower while the clock recovers
(kernel trace of the default line), so a GEMM sample of two or three steps
placed after each attention sample measured that transient. Bandwidth-bound ops are rotated over copies of
their buffers that exceed the 256 MB MALL three times, so their GB/s are HBM
figures.

The CPU baseline is the reference's own CPU path, its FP64 oracle loops
(restated in oracle/), timed on this host on a bounded sample; those sampled
rows also check the GPU output.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jade-compute_amd"))

import numpy as np  # noqa: E402

import jade_hip  # noqa: E402

METRIC = "FP32 GEMM & attention TFLOP/s (% of MI355X peak), 1 GPU, vs host-CPU ref"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0
PROFILE_DIR = os.path.join(ROOT, "profiles")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# The reference's harness method (src/runtime/metal_lab.rs:75-107,179-187;
# reports/METAL_ADVANCES.md:109-120): warm up, then samples (interleaved when
# several workloads are measured together), report the median per-step time. Here every workload also gets a time-based
# pre-heat before its samples: the MI355X clock ramps over the first ~30 ms of
# sustained matrix work, which a fixed warm-up count does not cover for short
# launches.
SAMPLES = 9
PREHEAT_MS = 100.0
MALL_BYTES = 256 << 20  # last-level (Infinity) cache in front of HBM


def split_steps(steps, samples=SAMPLES):
    """`steps` timed steps as at most `samples` samples (sizes differ by <= 1)."""
    count = max(1, min(samples, steps))
    base, extra = divmod(steps, count)
    return [base + (1 if i < extra else 0) for i in range(count)]


def median(values):
    v = sorted(values)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


class Workload:
    """One batch of jobs on the runtime; a step is one replay of the batch
    (`launches` kernel launches of the op being measured)."""

    def __init__(self, rt, jobs, launches=1):
        self.rt, self.jobs, self.launches = rt, jobs, launches
        self.preheat_ms, self.preheat_steps = 0.0, 0
        self.samples, self.sizes, self.host = [], [], []

    def warm(self, warmup):
        if warmup:
            self.rt.execute(self.jobs, warmup)

    def preheat(self, target_ms=None):
        # The module-level PREHEAT_MS is read at call time: --preheat-ms
        # replaces it after this class is defined.
        target_ms = PREHEAT_MS if target_ms is None else target_ms
        batch = 1
        while self.preheat_ms < target_ms:
            ex = self.rt.execute(self.jobs, batch)
            self.preheat_ms += ex.gpu_ms or 0.0
            self.preheat_steps += batch
            batch = min(2 * batch, 1 << 14)

    def min_sample_steps(self):
        """Steps that make a sample last at least MIN_SAMPLE_MS of device time,
        from the pre-heat's per-step time (1 without a pre-heat)."""
        if self.preheat_steps == 0 or self.preheat_ms <= 0.0:
            return 1
        per_step = self.preheat_ms / self.preheat_steps
        return min(MAX_SAMPLE_STEPS, int(np.ceil(MIN_SAMPLE_MS / per_step)))

    def sample(self, steps):
        ex = self.rt.execute(self.jobs, steps)
        if ex.gpu_ms is None:
            raise RuntimeError("device timer returned no duration")
        self.samples.append(ex.gpu_ms / steps)
        self.host.append(ex.host_ms / steps)
        self.sizes.append(steps)

    def summary(self):
        """Per-step times in ms: median of the samples (the reported figure),
        mean over all timed steps, extremes, and per-launch median."""
        total = sum(s * n for s, n in zip(self.samples, self.sizes))
        return {"ms_per_step": median(self.samples), "mean_ms_per_step": total / sum(self.sizes),
                "min_ms_per_step": min(self.samples), "max_ms_per_step": max(self.samples),
                "wall_ms_per_step": median(self.host), "samples": len(self.samples), "timed_steps": sum(self.sizes),
                "sample_steps": list(self.sizes), "samples_ms_per_step": [round(s, 6) for s in self.samples],
                "preheat_ms": self.preheat_ms, "ms_per_launch": median(self.samples) / self.launches}


# Steps per sample outside the headline: the reference's ten repeats per
# sample (reports/METAL_ADVANCES.md:109-112), or more when `steps` asks, and
# enough that a sample runs at least MIN_SAMPLE_MS of device time. A sample is
# one jr_execute_dispatches call: its first launch starts on an idle queue and
# pays the dispatch latency once, which ten launches of a few microseconds
# would carry as a third of a microsecond each.
SAMPLE_REPEATS = 10
MIN_SAMPLE_MS = 1.0
MAX_SAMPLE_STEPS = 4096


def measure(workloads, steps, warmup, min_repeats=SAMPLE_REPEATS):
    """Warm-up, pre-heat, then SAMPLES interleaved samples of each workload:
    sample round r runs the workloads in an order rotated by r
    (metal_lab.rs:179-187). The samples split `steps` evenly, each holding at
    least `min_repeats` steps (1 for the headline, which times exactly
    `steps`); outside the headline a workload's samples also hold enough steps
    for MIN_SAMPLE_MS of device time. Returns {name: summary}."""
    names = list(workloads)
    for name in names:
        workloads[name].warm(warmup)
        workloads[name].preheat()
    sizes = [max(size, min_repeats) for size in split_steps(steps)]
    if len(sizes) < SAMPLES and min_repeats > 1:
        sizes += [min_repeats] * (SAMPLES - len(sizes))
    floor = {name: workloads[name].min_sample_steps() if min_repeats > 1 else 1 for name in names}
    for r, size in enumerate(sizes):
        for off in range(len(names)):
            name = names[(r + off) % len(names)]
            workloads[name].sample(max(size, floor[name]))
    return {name: workloads[name].summary() for name in names}


def symbol_of(launch_kernel):
    """The kernel symbol prefix (as rocprofv3 names it) of a launch that
    jr_kernel_describe reports as `launch_kernel`."""
    for prefix in ("gemm_f32_ring", "gemm_f32_mfma_256", "gemm_f32_direct", "gemm_f32_dual_swiglu",
                   "attention_online_mfma", "attention_pairs_mfma"):
        if launch_kernel.startswith(prefix):
            return prefix
    return "gemm_f32_mfma"


def traffic_from_profiles(symbol_prefix, launch, workload):
    """HBM bytes per launch of this kernel at this grid in the counter run of
    `workload` (bench.py --workload ...), from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (profiles/traffic.json), or None."""
    path = os.path.join(PROFILE_DIR, "traffic.json")
    if not os.path.exists(path):
        return None
    block = launch["block"][0]
    items = launch["grid"][0] * launch["grid"][1] * launch["grid"][2] * block
    try:
        table = json.load(open(path))
    except (OSError, ValueError):
        return None
    # Keys are "symbol@work-items@workgroup@workload"; one symbol prefix can
    # name several instantiations, so an ambiguous match gives no figure.
    found = [entry.get("bytes_per_launch") for key, entry in table.items()
             if len(key.split("@")) == 4 and key.split("@")[0].startswith(symbol_prefix)
             and key.split("@")[1:] == [str(items), str(block), workload]]
    return found[0] if len(found) == 1 else None


class Prepared:
    """Device buffers and jobs of one workload, freed by close()."""

    def __init__(self, rt, jobs, buffers, info, launches=1):
        self.workload = Workload(rt, jobs, launches)
        self.buffers, self.info = buffers, info

    def close(self):
        for b in self.buffers:
            b.free()
        self.buffers = []


def prepare_gemm(rt, m, n, k, keep=False):
    a = jade_hip.fill_values(m * k, 0x12345678, 1.0)
    b = jade_hip.fill_values(k * n, 0x9ABCDEF1, 1.0)
    kernel = rt.compile({"op": "gemm", "m": m, "n": n, "k": k, "tiled": True})
    ag, bg, cg = rt.alloc(m * k), rt.alloc(k * n), rt.alloc(m * n)
    started = time.perf_counter()
    rt.upload(ag, a)
    rt.upload(bg, b)
    upload_ms = (time.perf_counter() - started) * 1000.0
    info = {"m": m, "n": n, "k": k, "flop": 2.0 * m * n * k, "kernel": kernel.launch["kernel"],
            "launch": kernel.launch, "upload_ms": upload_ms}
    p = Prepared(rt, [(kernel, [ag, bg, cg])], [ag, bg, cg], info)
    p.keep = (a, b) if keep else None
    p.output = cg
    return p


def finish_gemm(rt, p, timing):
    info = dict(p.info)
    info.update(timing)
    started = time.perf_counter()
    c = rt.download(p.output)
    info["download_ms"] = (time.perf_counter() - started) * 1000.0
    ms = timing["ms_per_step"]
    info["tflops"] = info["flop"] / (ms * 1e-3) / 1e12
    info["pcie_inclusive_tflops"] = info["flop"] / ((ms + info["upload_ms"] + info["download_ms"]) * 1e-3) / 1e12
    if p.keep is not None:
        info["_data"] = p.keep + (c,)
    p.close()
    return info


def prepare_attention(rt, heads, seq, dim, causal, keep=False):
    n = heads * seq * dim
    q = jade_hip.fill_normal(n, 0x1111)
    k = jade_hip.fill_normal(n, 0x2222)
    v = jade_hip.fill_normal(n, 0x3333)
    kernel = rt.compile({"op": "attention_online", "heads": heads, "seq": seq, "dim": dim, "causal": causal})
    bufs = [rt.resident(x) for x in (q, k, v)] + [rt.alloc(n)]
    keys = seq * (seq + 1) // 2 if causal else seq * seq
    info = {"heads": heads, "seq": seq, "dim": dim, "causal": causal, "flop": 4.0 * heads * dim * keys,
            "kernel": kernel.launch["kernel"], "launch": kernel.launch}
    p = Prepared(rt, [(kernel, bufs)], bufs, info)
    p.keep = (q, k, v) if keep else None
    p.output = bufs[3]
    return p


def finish_attention(rt, p, timing):
    info = dict(p.info)
    info.update(timing)
    info["tflops"] = info["flop"] / (timing["ms_per_step"] * 1e-3) / 1e12
    if p.keep is not None:
        info["_data"] = p.keep + (rt.download(p.output),)
    p.close()
    return info


def bench_gemm(rt, m, n, k, steps, warmup, keep=False):
    p = prepare_gemm(rt, m, n, k, keep)
    return finish_gemm(rt, p, measure({"gemm": p.workload}, steps, warmup)["gemm"])


def bench_attention(rt, heads, seq, dim, causal, steps, warmup, keep=False):
    p = prepare_attention(rt, heads, seq, dim, causal, keep)
    return finish_attention(rt, p, measure({"attention": p.workload}, steps, warmup)["attention"])


def rotated(rt, spec, inputs, n_out, nbytes, min_total=3 * MALL_BYTES):
    """A bandwidth op launched over enough copies of its inputs and output that
    one step's footprint is at least `min_total` bytes (three times the MALL),
    so every launch streams from HBM rather than from the cache. One step is
    one launch per copy."""
    kernel = rt.compile(spec)
    sets = max(1, -(-int(min_total) // int(nbytes)))
    jobs, bufs = [], []
    for _ in range(sets):
        b = [rt.resident(t) for t in inputs] + [rt.alloc(n_out)]
        bufs += b
        jobs.append((kernel, b))
    info = {"bytes": nbytes, "kernel": kernel.launch["kernel"], "copies": sets,
            "footprint_bytes": sets * nbytes}
    return Prepared(rt, jobs, bufs, info, launches=sets)


def finish_rotated(p, timing):
    info = dict(p.info)
    ms = timing["ms_per_launch"]
    info.update({"ms": ms, "gbps": info["bytes"] / (ms * 1e-3) / 1e9,
                 "frac_hbm": info["bytes"] / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                 "samples": timing["samples"], "preheat_ms": timing["preheat_ms"]})
    p.close()
    return info


def bench_softmax(rt, rows, cols, steps, warmup):
    x = jade_hip.fill_normal(rows * cols, 0x6666, 0.0, 2.0)
    nbytes = 2.0 * rows * cols * 4
    p = rotated(rt, {"op": "softmax", "rows": rows, "cols": cols}, (x,), rows * cols, nbytes)
    out = finish_rotated(p, measure({"softmax": p.workload}, steps, warmup)["softmax"])
    out.update({"rows": rows, "cols": cols})
    return out


MLP_SEEDS = {"x": 0x1234, "gamma": 0x7777, "wg": 0x3333, "wu": 0x4444, "wd": 0x5555}


def bench_mlp(rt, batch, width, hidden, steps, warmup):
    x = jade_hip.fill_normal(batch * width, MLP_SEEDS["x"])
    gamma = jade_hip.fill_values(width, MLP_SEEDS["gamma"], 0.5) + np.float32(1.0)
    wg = jade_hip.fill_normal(width * hidden, MLP_SEEDS["wg"], 0.0, 0.02)
    wu = jade_hip.fill_normal(width * hidden, MLP_SEEDS["wu"], 0.0, 0.02)
    wd = jade_hip.fill_normal(hidden * width, MLP_SEEDS["wd"], 0.0, 0.02)
    specs = [
        ("rms_norm", {"op": "rms_norm", "rows": batch, "cols": width, "epsilon": 1e-6}),
        ("gemm_gate", {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True}),
        ("gemm_up", {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True}),
        ("swiglu", {"op": "swi_glu", "len": batch * hidden}),
        ("gemm_down", {"op": "gemm", "m": batch, "n": width, "k": hidden, "tiled": True}),
        ("add", {"op": "add", "len": batch * width}),
    ]
    kernels = [rt.compile(s) for _, s in specs]
    xg, ng, wgg, wug, wdg = (rt.resident(t) for t in (x, gamma, wg, wu, wd))
    normalized, gate, up = rt.alloc(batch * width), rt.alloc(batch * hidden), rt.alloc(batch * hidden)
    act, proj, out = rt.alloc(batch * hidden), rt.alloc(batch * width), rt.alloc(batch * width)
    jobs = [(kernels[0], [xg, ng, normalized]), (kernels[1], [normalized, wgg, gate]),
            (kernels[2], [normalized, wug, up]), (kernels[3], [gate, up, act]), (kernels[4], [act, wdg, proj]),
            (kernels[5], [proj, xg, out])]
    block = measure({"block": Workload(rt, jobs)}, steps, warmup)["block"]
    gemm_flops = {"gemm_gate": 2.0 * batch * hidden * width, "gemm_up": 2.0 * batch * hidden * width,
                  "gemm_down": 2.0 * batch * width * hidden}
    per = {}
    for (name, _), job in zip(specs, jobs):
        if name in gemm_flops:
            t = measure({name: Workload(rt, [job])}, steps, warmup)[name]
            ms = t["ms_per_step"]
            spec = dict(specs)[name]
            per[name] = {"ms": ms, "tflops": gemm_flops[name] / (ms * 1e-3) / 1e12,
                         "frac_mfma": gemm_flops[name] / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
                         "kernel": job[0].launch["kernel"], "shape": f"{spec['m']}x{spec['n']}x{spec['k']}"}
    total_flops = sum(gemm_flops.values())
    for buf in (xg, ng, wgg, wug, wdg, normalized, gate, up, act, proj, out):
        buf.free()
    # The bandwidth ops alone at the MLP shapes, streaming from HBM.
    per.update(bench_rows(rt, batch, width, hidden, steps, warmup))
    return {"batch": batch, "width": width, "hidden": hidden, "ms_per_block": block["ms_per_step"],
            "block_timing": block, "gemm_tflops_block": total_flops / (block["ms_per_step"] * 1e-3) / 1e12,
            "seeds": {k: hex(v) for k, v in MLP_SEEDS.items()}, "per_op": per}


def bench_rows(rt, batch, width, hidden, steps, warmup):
    """RMSNorm, SwiGLU and Add launched alone at the MLP shapes, each rotated
    over copies of its buffers totalling at least three times the MALL, so the
    bytes come from HBM (a launch re-reading one 16-50 MB input would be
    served by the 256 MB cache)."""
    x = jade_hip.fill_normal(batch * width, 0x1234)
    gamma = jade_hip.fill_values(width, 0x7777, 0.5) + np.float32(1.0)
    gate = jade_hip.fill_normal(batch * hidden, 0x2468)
    up = jade_hip.fill_normal(batch * hidden, 0x1357)
    proj = jade_hip.fill_normal(batch * width, 0x9999)
    cases = [
        ("rms_norm", {"op": "rms_norm", "rows": batch, "cols": width, "epsilon": 1e-6}, (x, gamma), batch * width,
         (2.0 * batch * width + width) * 4),
        ("swiglu", {"op": "swi_glu", "len": batch * hidden}, (gate, up), batch * hidden, 3.0 * batch * hidden * 4),
        ("add", {"op": "add", "len": batch * width}, (proj, x), batch * width, 3.0 * batch * width * 4),
    ]
    out = {}
    for name, spec, inputs, n_out, nbytes in cases:
        p = rotated(rt, spec, inputs, n_out, nbytes)
        out[name] = finish_rotated(p, measure({name: p.workload}, steps, warmup)[name])
    return out


COPY_ELEMENTS = 1 << 26  # 256 MiB read + 256 MiB written per launch


def bench_copy(rt, steps, warmup):
    """A plain copy of known size: the calibration point for the HBM counters
    and the practical streaming ceiling, rotated over two source/destination
    pairs (1 GiB) so it streams from HBM."""
    n = COPY_ELEMENTS
    spec = {"op": "elementwise", "len": n, "inputs": 1, "expression": {"kind": "input", "binding": 0}}
    p = rotated(rt, spec, (jade_hip.fill_values(n, 0x4242, 1.0),), n, 2.0 * n * 4)
    out = finish_rotated(p, measure({"copy": p.workload}, steps, warmup)["copy"])
    out["elements"] = n
    return out


FLOOR_QUEUED = 4000   # near-empty launches queued behind the long ones
FLOOR_LONG = 10       # 4096^3 GEMMs ahead of them (about 9 ms of device work)


def bench_floor(rt, steps, warmup):
    """Per-launch time of near-empty launches on the runtime's stream (one
    workgroup copying 64 floats; 256 workgroups adding 262144 floats, 1 MiB
    per operand), two ways:
    - back to back as the host enqueues them (jr_execute_dispatches replaying
      the one job): the host's enqueue rate bounds it;
    - behind a full queue: FLOOR_QUEUED of them enqueued after FLOOR_LONG
      4096^3 GEMMs in one batch, so all are queued before the device reaches
      them; the time over the GEMMs alone, per launch, is the device-side
      cost of a launch. Median of SAMPLES interleaved pairs of batches."""
    out = {}
    long_p = prepare_gemm(rt, 4096, 4096, 4096)
    long_job = long_p.workload.jobs[0]
    for name, spec, n in (("copy_64", {"op": "elementwise", "len": 64, "inputs": 1,
                                        "expression": {"kind": "input", "binding": 0}}, 64),
                          ("add_256_workgroups", {"op": "add", "len": 262144}, 262144)):
        kernel = rt.compile(spec)
        count = spec.get("inputs", 2)
        bufs = [rt.resident(jade_hip.fill_values(n, 0x77 + i, 1.0)) for i in range(count)] + [rt.alloc(n)]
        t = measure({name: Workload(rt, [(kernel, bufs)])}, steps, warmup)[name]
        job = (kernel, bufs)
        rt.execute([long_job] * FLOOR_LONG + [job] * FLOOR_QUEUED, 1)  # warm-up
        alone, behind = [], []
        for _ in range(SAMPLES):
            alone.append(rt.execute([long_job] * FLOOR_LONG, 1).gpu_ms)
            behind.append(rt.execute([long_job] * FLOOR_LONG + [job] * FLOOR_QUEUED, 1).gpu_ms)
        per = [1e3 * (b - a) / FLOOR_QUEUED for a, b in zip(alone, behind)]
        out[name] = {"us_per_launch": 1e3 * t["ms_per_step"], "min_us": 1e3 * t["min_ms_per_step"],
                     "behind_full_queue_us": 1e3 * (median(behind) - median(alone)) / FLOOR_QUEUED,
                     "behind_full_queue_range_us": [min(per), max(per)],
                     "queued": FLOOR_QUEUED, "long_launches": FLOOR_LONG, "launch": kernel.launch}
        for b in bufs:
            b.free()
    long_p.close()
    return out


# The shapes set beside the vendor library: the headline, the large cubes, the
# LLM-width product and the MLP's two GEMM shapes. Smaller products are left
# out: torch.matmul's per-call host path (~19 us on the pool's hosts) then
# bounds its back-to-back time, which would compare dispatch, not kernels.
VENDOR_SHAPES = ((4096, 4096, 4096), (2048, 2048, 2048), (4096, 11008, 4096), (4096, 2816, 1024),
                 (4096, 1024, 2816), (1024, 1024, 1024))
VENDOR_ROUNDS = 3


def bench_vendor(rt, steps, warmup, rounds=VENDOR_ROUNDS):
    """This library's GEMM beside torch.matmul in FP32 (TF32 off; hipBLASLt
    on ROCm) in one process, on the same validation::inputs, as the
    reference's harness sets its kernel beside the platform library
    (src/runtime/metal_lab.rs:150, native/jade_corex.cpp:91-95). Per shape,
    `rounds` rounds alternate which side runs first; each round is SAMPLES
    event-timed samples per side of at least MIN_SAMPLE_MS of device time
    (this library: measure() on the runtime's stream; torch: back-to-back
    calls on torch's stream). Reports the median over rounds of each round's
    median, and the ratio library time / this library's time."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    out = {}
    for m, n, k in VENDOR_SHAPES:
        p = prepare_gemm(rt, m, n, k)
        a = torch.from_numpy(jade_hip.fill_values(m * k, 0x12345678, 1.0).reshape(m, k)).to("cuda")
        b = torch.from_numpy(jade_hip.fill_values(k * n, 0x9ABCDEF1, 1.0).reshape(k, n)).to("cuda")
        c = torch.empty(m, n, dtype=torch.float32, device="cuda")

        def torch_ms(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                torch.matmul(a, b, out=c)
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps

        spent, reps = 0.0, 1
        while spent < PREHEAT_MS:  # the library's own pre-heat
            spent += torch_ms(reps) * reps
            reps = min(2 * reps, 1 << 12)
        per_call = torch_ms(SAMPLE_REPEATS)
        reps = max(SAMPLE_REPEATS, int(math.ceil(MIN_SAMPLE_MS / max(per_call, 1e-6))))
        ours, lib = [], []
        for r in range(rounds):
            for side in ((0, 1) if r % 2 == 0 else (1, 0)):
                if side == 0:
                    first = len(p.workload.samples)
                    measure({"gemm": p.workload}, steps, warmup)
                    ours.append(median(p.workload.samples[first:]))
                else:
                    lib.append(median([torch_ms(reps) for _ in range(SAMPLES)]))
        kernel = p.info["kernel"]
        p.close()
        del a, b, c
        flop = 2.0 * m * n * k
        mo, ml = median(ours), median(lib)
        out[f"{m}x{n}x{k}"] = {"ms": mo, "tflops": flop / (mo * 1e-3) / 1e12, "kernel": kernel,
                               "vendor_ms": ml, "vendor_tflops": flop / (ml * 1e-3) / 1e12,
                               "vendor_over_ours": ml / mo, "rounds_ms": ours, "vendor_rounds_ms": lib,
                               "vendor_calls_per_sample": reps}
        log(f"  {m}x{n}x{k}: {mo * 1e3:.2f} us ({kernel}) vs torch.matmul {ml * 1e3:.2f} us, "
            f"ratio {ml / mo:.3f}")
    out["vendor"] = f"torch {torch.__version__} torch.matmul FP32, TF32 off"
    return out


def _read_csv(path):
    import csv

    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _find_all(directory, suffix):
    found = []
    for root, _, files in os.walk(directory):
        found += [os.path.join(root, name) for name in files if name.endswith(suffix)]
    return sorted(found)


def _find(directory, suffix):
    found = _find_all(directory, suffix)
    return found[0] if found else None


def _short(name):
    name = name.replace("jade::hipk::(anonymous namespace)::", "")
    name = name[len("void "):] if name.startswith("void ") else name
    return name.split("(")[0] if "(" in name else name


def _workload_of(path):
    """The workload a counter file belongs to: the name of the directory that
    holds the rocprofv3 output of one `bench.py --workload ...` run."""
    return os.path.basename(os.path.dirname(path))


def bench_gemm_launches(bench_log):
    """(shape, launch kernel name, event-timed ms per launch) of every GEMM
    that a bench.py JSON line in `bench_log` reports: the headline, the MLP's
    GEMMs launched alone, the sweep and this library's side of the vendor
    comparison."""
    line = None
    with open(bench_log, errors="replace") as f:
        for text in f:
            if text.startswith('{"metric"'):
                line = json.loads(text)
    if line is None:
        return []
    out = []
    head = line.get("gpu_kernel", {})
    if "m" in head:
        out.append((f"{head['m']}x{head['n']}x{head['k']}", head["kernel"], head["ms_per_step"]))
    extra = line.get("extra", {})
    for name, op in extra.get("mlp_4096x1024x2816", {}).get("per_op", {}).items():
        if "shape" in op:
            out.append((op["shape"], op["kernel"], op["ms"]))
    for shape, r in extra.get("gemm_sweep", {}).items():
        out.append((shape, r["kernel"], r["ms"]))
    for shape, r in extra.get("vendor_gemm", {}).items():
        if isinstance(r, dict):
            out.append((shape, r["kernel"], r["ms"]))
    return out


def vendor_gemm_launches(bench_log):
    """(shape, "vendor", event-timed ms per call) of the library side of a
    `--workload vendor` line in `bench_log`."""
    line = None
    with open(bench_log, errors="replace") as f:
        for text in f:
            if text.startswith('{"metric"'):
                line = json.loads(text)
    if line is None:
        return []
    return [(shape, "vendor", r["vendor_ms"]) for shape, r in line.get("extra", {}).get("vendor_gemm", {}).items()
            if isinstance(r, dict)]


def split_by_shape(durations_ns, launches, tolerance=0.25):
    """Dispatches of one kernel symbol that serves several shapes at one grid
    (the persistent GEMM), assigned to the shape whose event-timed median is
    nearest in log scale; a dispatch further than `tolerance` from every
    median (warm-up at low clocks, pre-heat) stays unassigned. Returns
    {shape or None: [durations]}."""
    groups = {}
    medians = {}
    for shape, _, ms in launches:
        medians.setdefault(shape, ms * 1e6)
    for d in durations_ns:
        best = min(medians, key=lambda sh: abs(np.log(d / medians[sh])))
        label = best if abs(d / medians[best] - 1.0) <= tolerance else None
        groups.setdefault(label, []).append(d)
    return groups


def summarize_rocprof(trace_dir, fetch_dir=None, write_dir=None, bench_log=None):
    """Per (kernel, grid) durations from a rocprofv3 --kernel-trace run, plus HBM
    bytes per launch from --pmc FETCH_SIZE and WRITE_SIZE runs (one output
    directory per bench.py workload, rows kept apart by workload), scaled by
    what the same counters read for the copy kernel of known size
    (COPY_ELEMENTS). With `bench_log` (the profiled run's output), dispatches
    of the persistent GEMM, whose grid is the same at every shape, are split
    by shape against the bench's own event-timed medians."""
    trace = _read_csv(_find(trace_dir, "kernel_trace.csv"))
    groups = {}
    for row in trace:
        key = (_short(row["Kernel_Name"]), int(row["Grid_Size_X"]), int(row["Grid_Size_Y"]),
               int(row["Grid_Size_Z"]), int(row["Workgroup_Size_X"]))
        groups.setdefault(key, []).append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    launches = bench_gemm_launches(bench_log) if bench_log else []
    ring_shapes = [x for x in launches if x[1].startswith("gemm_f32_ring")]
    # The vendor library's GEMMs (hipBLASLt "Cijk_" kernels) also run one
    # grid at several shapes; the same split applies against its medians.
    vendor_shapes = vendor_gemm_launches(bench_log) if bench_log else []
    rows = []
    for key, durations in groups.items():
        if key[0].startswith("gemm_f32_ring") and ring_shapes:
            split = split_by_shape(durations, ring_shapes)
        elif key[0].startswith("Cijk_") and vendor_shapes:
            split = split_by_shape(durations, vendor_shapes)
        else:
            rows.append((key[0], key[1:], durations))
            continue
        for shape, part in split.items():
            rows.append((key[0] + (f" [{shape}]" if shape else " [unassigned]"), key[1:], part))
    counters = {}
    for directory, counter in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        if not directory:
            continue
        # One counter_collection.csv per profiled run, in a directory named
        # for its workload; a directory may hold several runs.
        for path in _find_all(directory, "counter_collection.csv"):
            for row in _read_csv(path):
                if row.get("Counter_Name") != counter:
                    continue
                key = (_short(row["Kernel_Name"]), int(row["Grid_Size"]), int(row["Workgroup_Size"]),
                       _workload_of(path))
                counters.setdefault(key, {}).setdefault(counter, []).append(float(row["Counter_Value"]))
    # The median beside the mean: a workload's dispatches include its
    # pre-heat, whose first launches run at a lower clock.
    lines = ["| kernel | grid (work-items) | block | calls | avg us | min us | max us | median us |",
             "|---|---|---|---|---|---|---|---|"]
    for name, (gx, gy, gz, wg), durations in sorted(rows, key=lambda r: -sum(r[2])):
        lines.append(f"| {name} | {gx}x{gy}x{gz} | {wg} | {len(durations)} | {np.mean(durations) / 1e3:.2f} | "
                     f"{np.min(durations) / 1e3:.2f} | {np.max(durations) / 1e3:.2f} | "
                     f"{np.median(durations) / 1e3:.2f} |")
    if ring_shapes:
        lines += ["", "Event-timed medians of the same run (bench.py's own figures, ms per launch): " +
                  ", ".join(f"{shape} {ms * 1e3:.2f} us ({kernel})" for shape, kernel, ms in launches)]
    traffic = {}
    if counters:
        copy_key = next((k for k in counters if k[0] == "copy_stream"), None)
        expected_kib = COPY_ELEMENTS * 4 / 1024.0
        scale = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            measured = np.mean(counters.get(copy_key, {}).get(counter, [np.nan])) if copy_key else np.nan
            scale[counter] = expected_kib / measured if measured and np.isfinite(measured) else np.nan
        lines += ["", f"HBM counter calibration (copy_stream, {COPY_ELEMENTS * 4 / 2**20:.0f} MiB in and out): "
                      f"scale FETCH_SIZE x{scale['FETCH_SIZE']:.4f}, WRITE_SIZE x{scale['WRITE_SIZE']:.4f}", "",
                  "| kernel | workload | grid (work-items) | block | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB "
                  "| scaled MB/launch |",
                  "|---|---|---|---|---|---|---|---|"]
        for key, vals in sorted(counters.items()):
            fetch = np.mean(vals.get("FETCH_SIZE", [np.nan]))
            write = np.mean(vals.get("WRITE_SIZE", [np.nan]))
            nbytes = (fetch * scale["FETCH_SIZE"] + write * scale["WRITE_SIZE"]) * 1024.0
            count = max(len(vals.get("FETCH_SIZE", [])), len(vals.get("WRITE_SIZE", [])))
            if key[0].startswith("__amd_rocclr"):
                continue
            lines.append(f"| {key[0]} | {key[3]} | {key[1]} | {key[2]} | {count} | {fetch:.0f} | {write:.0f} | "
                         f"{nbytes / 1e6:.1f} |")
            if np.isfinite(nbytes):
                traffic[f"{key[0]}@{key[1]}@{key[2]}@{key[3]}"] = {"bytes_per_launch": nbytes, "fetch_kib": fetch,
                                                                   "write_kib": write}
    return "\n".join(lines), traffic


# Shapes for MFMA-utilisation counter runs: each launch keeps the summed
# SQ_VALU_MFMA_BUSY_CYCLES below the 2^31 at which the counter saturates, and
# each exercises one production kernel (64x64 tiles with four K groups,
# direct-load 32x32 tiles, unaligned rows on 64x64 tiles with two K groups,
# direct-load tiles split over K; the eight-wave paired, four-wave and
# eight-wave online attention launches). The persistent GEMM launches one grid
# at every shape, so its counter rows cannot be told apart within one run:
# its shapes are counted one per run (--workload shape).
MFMA_GEMMS = ((1024, 1024, 1024), (512, 512, 512), (1000, 777, 513), (16, 1024, 2816))
MFMA_ATTENTION = ((8, 1024, 64, False), (8, 1024, 64, True), (32, 2048, 64, True), (64, 2048, 128, True))
SIMDS = 1024  # 256 CUs x 4 SIMDs
XCDS = 8


def bench_mfma_shapes(rt, steps, warmup):
    out = {}
    for m, n, k in MFMA_GEMMS:
        r = bench_gemm(rt, m, n, k, steps, warmup)
        out[f"gemm {m}x{n}x{k}"] = {"kernel": r["kernel"], "ms": r["ms_per_step"], "tflops": r["tflops"]}
    for heads, seq, dim, causal in MFMA_ATTENTION:
        r = bench_attention(rt, heads, seq, dim, causal, steps, warmup)
        out[f"attention H{heads} S{seq} D{dim} {'causal' if causal else 'noncausal'}"] = {
            "kernel": r["kernel"], "ms": r["ms_per_step"], "tflops": r["tflops"]}
    return out


def summarize_mfma(directory):
    """MFMA busy share per (kernel, grid, workload) from rocprofv3 --pmc runs
    with SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE, one output directory per
    bench.py workload: busy / (GUI cycles per XCD x SIMDs). GRBM_GUI_ACTIVE is
    summed over the 8 XCDs. The GUI clock column is GUI cycles per XCD over the
    dispatch's own duration (its start and end timestamps), median over
    dispatches: the clock during launches long enough that launch and drain
    are a small part of them."""
    vals = {}
    for path in _find_all(directory, "counter_collection.csv"):
        for row in _read_csv(path):
            key = (_short(row["Kernel_Name"]), int(row["Grid_Size"]), int(row["Workgroup_Size"]),
                   _workload_of(path))
            per = vals.setdefault(key, {})
            per.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
            if row["Counter_Name"] == "GRBM_GUI_ACTIVE" and "End_Timestamp" in row:
                ns = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
                if ns > 0:
                    per.setdefault("_ghz", []).append(float(row["Counter_Value"]) / XCDS / ns)
    lines = ["| kernel | workload | grid (work-items) | block | dispatches | GRBM_GUI_ACTIVE / XCD "
             "| SQ_VALU_MFMA_BUSY_CYCLES | MFMA busy | GUI clock GHz |",
             "|---|---|---|---|---|---|---|---|---|"]
    for key, v in sorted(vals.items()):
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in v or "GRBM_GUI_ACTIVE" not in v:
            continue
        busy = np.median(v["SQ_VALU_MFMA_BUSY_CYCLES"])
        gui = np.median(v["GRBM_GUI_ACTIVE"]) / XCDS
        if busy <= 0:
            continue
        ghz = f"{np.median(v['_ghz']):.3f}" if v.get("_ghz") else "-"
        lines.append(f"| {key[0]} | {key[3]} | {key[1]} | {key[2]} | {len(v['GRBM_GUI_ACTIVE'])} | {gui:.0f} | "
                     f"{busy:.4g} | {100.0 * busy / (gui * SIMDS):.1f}% | {ghz} |")
    return "\n".join(lines)


def summarize_counters(directory, match=""):
    """Median per dispatch of every counter of a rocprofv3 --pmc run, per
    (kernel, grid, workgroup) whose symbol contains `match`; SQ wave counters
    also per wave (grid / 64 waves). Dispatches seen fewer than 10 times are
    left out (set-up copies and fills)."""
    vals = {}
    for path in _find_all(directory, "counter_collection.csv"):
        for row in _read_csv(path):
            name = _short(row["Kernel_Name"])
            if match not in name:
                continue
            key = (name, int(row["Grid_Size"]), int(row["Workgroup_Size"]))
            per = vals.setdefault(key, {}).setdefault(row["Counter_Name"], {})
            per[row["Dispatch_Id"]] = per.get(row["Dispatch_Id"], 0.0) + float(row["Counter_Value"])
    lines = ["| kernel | grid (work-items) | block | dispatches | counter | median per dispatch | per wave |",
             "|---|---|---|---|---|---|---|"]
    for key, counters in sorted(vals.items()):
        waves = key[1] // 64
        for counter, per in sorted(counters.items()):
            if len(per) < 10:
                continue
            median = float(np.median(list(per.values())))
            per_wave = f"{median / waves:.1f}" if counter.startswith("SQ_") else ""
            lines.append(f"| {key[0]} | {key[1]} | {key[2]} | {len(per)} | {counter} | {median:.6g} | {per_wave} |")
    return "\n".join(lines)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Threads for the OpenMP oracle: every CPU this process may run on, capped
    by OMP_NUM_THREADS where the host sets it (the GPU pool sets it to the
    16-thread CPU share of one GPU)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(usable, int(cap))) if cap.isdigit() and int(cap) > 0 else max(1, usable)


def cpu_baseline(gemm, attention):
    """The reference's CPU path (FP64 oracle loops) on this host, bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_binding as orc

    cores = cpu_threads()
    a, b, c_gpu = gemm["_data"]
    m, n, k = gemm["m"], gemm["n"], gemm["k"]
    rows = max(1, min(m, int(os.environ.get("JADE_CPU_ROWS", str(m)))))
    started = time.perf_counter()
    ref = orc.gemm_reference(m, n, k, a, b, rows=(0, rows), threads=cores)
    omp_s = time.perf_counter() - started
    check = orc.compare(c_gpu[:rows * n], ref, 1e-4, 1e-4)
    single_rows = max(1, rows // 16)
    started = time.perf_counter()
    orc.gemm_reference(m, n, k, a, b, rows=(0, single_rows), threads=1)
    single_s = time.perf_counter() - started
    gemm_flop = 2.0 * rows * n * k
    out = {"value": gemm_flop / omp_s / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
           "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count(),
           "sample": f"FP64 gemm_reference (metal_lab.rs:18-31) rows 0..{rows} of the {m}x{n}x{k} GEMM "
                     f"({gemm_flop:.3e} FLOP, {omp_s:.2f} s on {cores} OpenMP threads)",
           "single_thread_tflops": 2.0 * single_rows * n * k / single_s / 1e12,
           "single_thread_sample": f"rows 0..{single_rows}, {single_s:.2f} s",
           "gpu_check_rows": rows, "gpu_check_status": int(check.status),
           "gpu_max_abs_error": check.max_abs_error, "gpu_max_rel_error": check.max_relative_error}
    if attention is not None and "_data" in attention:
        q, kk, v, o_gpu = attention["_data"]
        h, s, d = attention["heads"], attention["seq"], attention["dim"]
        r0, r1 = s - 16, s
        started = time.perf_counter()
        ref = orc.attention_reference(h, s, d, attention["causal"], q, kk, v, rows=(r0, r1), threads=cores)
        att_s = time.perf_counter() - started
        keys = sum(range(r0 + 1, r1 + 1)) if attention["causal"] else (r1 - r0) * s
        flop = 4.0 * h * d * keys
        got = o_gpu.reshape(h, s, d)[:, r0:r1].reshape(-1)
        check = orc.compare(got, ref, 2e-4, 2e-4)
        out["attention"] = {"value": flop / att_s / 1e12, "unit": "TFLOP/s", "cores": cores,
                            "sample": f"FP64 attention_reference (metal_lab.rs:33-73) query rows {r0}..{r1} of all "
                                      f"{h} heads ({flop:.3e} FLOP, {att_s:.2f} s)",
                            "gpu_check_status": int(check.status), "gpu_max_abs_error": check.max_abs_error}
    return out


def main():
    global PREHEAT_MS
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--preheat-ms", type=float, default=PREHEAT_MS,
                    help="untimed device time of each workload before its samples (0 for counter runs)")
    ap.add_argument("--workload", default="all",
                    choices=["all", "gemm", "attention", "softmax", "mlp", "rows", "sweep", "copy", "mfma", "floor",
                             "shape", "vendor"])
    ap.add_argument("--shape", default="4096x4096x2048", metavar="MxNxK",
                    help="the one GEMM of --workload shape (counter runs of one shape)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--summarize-rocprof", metavar="TRACE_DIR",
                    help="print per-kernel tables from a rocprofv3 --kernel-trace output directory and exit")
    ap.add_argument("--pmc-fetch", metavar="DIR", help="rocprofv3 --pmc FETCH_SIZE output directory")
    ap.add_argument("--pmc-write", metavar="DIR", help="rocprofv3 --pmc WRITE_SIZE output directory")
    ap.add_argument("--traffic-out", metavar="JSON", help="write HBM bytes per launch per (kernel, grid, workload)")
    ap.add_argument("--bench-log", metavar="FILE",
                    help="output of the profiled bench.py run: splits the persistent GEMM's trace rows by shape")
    ap.add_argument("--summarize-mfma", metavar="PMC_DIR",
                    help="print MFMA busy shares from a rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE "
                         "output directory and exit")
    ap.add_argument("--summarize-counters", metavar="PMC_DIR",
                    help="print the median of every counter per kernel from a rocprofv3 --pmc output directory "
                         "and exit (--match: only kernels whose symbol contains this text)")
    ap.add_argument("--match", default="")
    args = ap.parse_args()
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.match))
        return
    if args.summarize_mfma:
        print(summarize_mfma(args.summarize_mfma))
        return
    if args.summarize_rocprof:
        table, traffic = summarize_rocprof(args.summarize_rocprof, args.pmc_fetch, args.pmc_write, args.bench_log)
        print(table)
        if args.traffic_out:
            with open(args.traffic_out, "w") as f:
                json.dump(traffic, f, indent=1, sort_keys=True)
                f.write("\n")
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0 or args.warmup < 0 or args.preheat_ms < 0:
        sys.exit("steps must be positive, warmup and preheat non-negative")
    PREHEAT_MS = args.preheat_ms

    if args.workload == "vendor":
        # torch's HIP runtime must be the process's first: loaded after this
        # library's, its device init finds no GPU.
        import torch  # noqa: F401
    rt = jade_hip.HipRuntime(0)
    log(f"device: {rt.device_info}")
    K, W, wl = args.steps, args.warmup, args.workload
    extra = {}
    gemm = attention = None
    keep = not args.no_cpu_baseline
    if wl in ("all", "gemm", "attention"):
        # The two headline kernels, each sampled on its own after its pre-heat.
        heads = {}
        if wl in ("all", "gemm"):
            heads["gemm"] = prepare_gemm(rt, 4096, 4096, 4096, keep)
        if wl in ("all", "attention"):
            heads["attention"] = prepare_attention(rt, 128, 4096, 128, True, keep)
        log(f"headline {', '.join(heads)} ...")
        timing = {}
        for name, p in heads.items():
            timing.update(measure({name: p.workload}, K, W, min_repeats=1))
        if "gemm" in heads:
            gemm = finish_gemm(rt, heads["gemm"], timing["gemm"])
            log(f"  gemm 4096^3 {gemm['tflops']:.2f} TFLOP/s")
        if "attention" in heads:
            attention = finish_attention(rt, heads["attention"], timing["attention"])
            log(f"  attention B4 H32 S4096 D128 causal {attention['tflops']:.2f} TFLOP/s")
    if wl in ("all", "attention"):
        c3 = {}
        for causal in (False, True):
            r = bench_attention(rt, 8, 1024, 64, causal, K, W)
            c3["causal" if causal else "noncausal"] = {
                "ms": r["ms_per_step"], "tflops": r["tflops"], "frac_mfma": r["tflops"] / PEAK_FP32_MFMA_TFLOPS,
                "min_ms": r["min_ms_per_step"], "max_ms": r["max_ms_per_step"], "kernel": r["kernel"]}
        extra["attention_c3_b1h8s1024d64"] = c3
        log(f"  C3 {c3['noncausal']['tflops']:.1f} / {c3['causal']['tflops']:.1f} TFLOP/s")
    if wl in ("all", "softmax"):
        log("softmax 32768x4096 ...")
        sm = bench_softmax(rt, 32768, 4096, K, W)
        extra["softmax_32768x4096"] = sm
        log(f"  {sm['gbps']:.0f} GB/s")
    if wl in ("all", "mlp"):
        log("six-op MLP 4096x1024x2816 ...")
        extra["mlp_4096x1024x2816"] = bench_mlp(rt, 4096, 1024, 2816, K, W)
        log(f"  {extra['mlp_4096x1024x2816']['ms_per_block']:.3f} ms per block")
    if wl == "rows":  # counter runs only; the default line measures these ops inside bench_mlp
        extra["rows_mlp_shapes"] = bench_rows(rt, 4096, 1024, 2816, K, W)
    if wl in ("all", "copy"):
        extra["copy_calibration"] = bench_copy(rt, K, W)
    if wl == "floor":  # launch-floor measurement only; not part of the default line
        extra["launch_floor"] = bench_floor(rt, max(K, 200), W)
        for name, f in extra["launch_floor"].items():
            log(f"  floor {name}: {f['us_per_launch']:.2f} us back to back, "
                f"{f['behind_full_queue_us']:.2f} us behind a full queue")
    if wl == "mfma":  # counter runs only; not part of the default line
        extra["mfma_shapes"] = bench_mfma_shapes(rt, K, W)
    if wl == "vendor":  # this library beside torch.matmul; not part of the default line
        extra["vendor_gemm"] = bench_vendor(rt, K, W)
    if wl == "shape":  # one GEMM shape (counter runs); not part of the default line
        m, n, k = (int(x) for x in args.shape.split("x"))
        r = bench_gemm(rt, m, n, k, K, W)
        extra["gemm_shape"] = {"shape": args.shape, "ms": r["ms_per_step"], "tflops": r["tflops"],
                               "kernel": r["kernel"], "launch": r["launch"]}
        log(f"  {args.shape} {r['tflops']:.1f} TFLOP/s ({r['kernel']})")
    if wl in ("all", "sweep"):
        sweep = {}
        for m, n, k in ((512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (1000, 777, 513),
                        (4096, 11008, 4096)):
            r = bench_gemm(rt, m, n, k, K, W)
            sweep[f"{m}x{n}x{k}"] = {"ms": r["ms_per_step"], "tflops": r["tflops"],
                                     "frac_mfma": r["tflops"] / PEAK_FP32_MFMA_TFLOPS,
                                     "min_ms": r["min_ms_per_step"], "max_ms": r["max_ms_per_step"],
                                     "kernel": r["kernel"]}
            log(f"  sweep {m}x{n}x{k} {r['tflops']:.1f} TFLOP/s")
        extra["gemm_sweep"] = sweep

    head = gemm or attention
    if head is None:
        print(json.dumps({"metric": METRIC, "workload": wl, "extra": extra}))
        return
    if gemm is not None:
        config = {"workload": "FP32 GEMM C=A.B 4096x4096x4096, row-major (BASELINE configs[1] headline)",
                  "m": 4096, "n": 4096, "k": 4096,
                  "inputs": "validation::inputs xorshift32 seeds 0x12345678/0x9abcdef1, U[-1,1)"}
        symbol = symbol_of(gemm["launch"]["kernel"])
    else:
        config = {"workload": "FP32 causal attention B4 H32 S4096 D128 (BASELINE configs[4])"}
        symbol = "attention_online_mfma"
    achieved = head["flop"] / (head["ms_per_step"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": config,
        "timing": {"method": f"median of {head['samples']} consecutive samples over exactly the {K} timed steps, after "
                             f"{W} warm-up steps and a {PREHEAT_MS:.0f} ms time-based pre-heat per workload",
                   "median_ms_per_step": head["ms_per_step"], "mean_ms_per_step": head["mean_ms_per_step"],
                   "min_ms_per_step": head["min_ms_per_step"], "max_ms_per_step": head["max_ms_per_step"],
                   "sample_steps": head["sample_steps"]},
        "preheat_ms": head["preheat_ms"],
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP32_MFMA_TFLOPS,
                     "traffic": traffic_from_profiles(symbol, head["launch"], "gemm" if gemm else "attention")},
    }
    if attention is not None and gemm is not None:
        att = {k: v for k, v in attention.items() if not k.startswith("_")}
        att["roofline"] = {"bound": "mfma", "achieved": attention["tflops"], "peak": PEAK_FP32_MFMA_TFLOPS,
                           "unit": "TFLOP/s", "frac": attention["tflops"] / PEAK_FP32_MFMA_TFLOPS,
                           "traffic": traffic_from_profiles("attention_online_mfma", attention["launch"], "attention")}
        line["attention"] = att
    if not args.no_cpu_baseline and gemm is not None:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(gemm, attention)
    line["extra"] = extra
    line["gpu_kernel"] = {k: v for k, v in head.items() if not k.startswith("_")}
    print(json.dumps(line), flush=True)
    rt.close()


if __name__ == "__main__":
    main()
