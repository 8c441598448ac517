"""Six-op residual MLP (src/runtime/workloads.rs:366-525) as one ordered
execute of six jobs, against the FP64 chain oracle (workloads.rs:466-479)."""
import numpy as np
import pytest

import oracle_binding as orc

pytestmark = pytest.mark.gpu


def mlp_jobs(runtime, batch, width, hidden, x, norm, wg, wu, wd, eps):
    specs = [
        {"op": "rms_norm", "rows": batch, "cols": width, "epsilon": eps},
        {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True},
        {"op": "gemm", "m": batch, "n": hidden, "k": width, "tiled": True},
        {"op": "swi_glu", "len": batch * hidden},
        {"op": "gemm", "m": batch, "n": width, "k": hidden, "tiled": True},
        {"op": "add", "len": batch * width},
    ]
    k = [runtime.compile(s) for s in specs]
    xg, ng, wgg, wug, wdg = (runtime.resident(t) for t in (x, norm, wg, wu, wd))
    normalized, gate, up = runtime.alloc(batch * width), runtime.alloc(batch * hidden), runtime.alloc(batch * hidden)
    act, proj, out = runtime.alloc(batch * hidden), runtime.alloc(batch * width), runtime.alloc(batch * width)
    jobs = [(k[0], [xg, ng, normalized]), (k[1], [normalized, wgg, gate]), (k[2], [normalized, wug, up]),
            (k[3], [gate, up, act]), (k[4], [act, wdg, proj]), (k[5], [proj, xg, out])]
    return jobs, out


@pytest.mark.parametrize("batch,width,hidden", [(8, 128, 256), (3, 33, 65), (64, 512, 1024)])
def test_reference_mlp_workload(runtime, batch, width, hidden):
    # workloads::mlp_with_gemm inputs (389-394), eps 1e-5, tolerance 5e-5.
    x = orc.values(batch * width, 0x1234, 1.0)
    norm = np.ones(width, np.float32)
    wg = orc.values(width * hidden, 0x3333, np.float32(1.0) / np.sqrt(np.float32(width)))
    wu = orc.values(width * hidden, 0x4444, np.float32(1.0) / np.sqrt(np.float32(width)))
    wd = orc.values(hidden * width, 0x5555, np.float32(1.0) / np.sqrt(np.float32(hidden)))
    eps = float(np.float32(1e-5))
    jobs, out = mlp_jobs(runtime, batch, width, hidden, x, norm, wg, wu, wd, 1e-5)
    timing = runtime.execute(jobs, 3)
    assert timing.dispatches == 18
    want = orc.mlp(batch, width, hidden, x, norm, wg, wu, wd, eps)
    check = orc.compare(runtime.download(out), want, 5e-5, 5e-5)
    assert check.status == 0, check.first_bad


def test_config_c4_mlp(runtime):
    batch, width, hidden = 4096, 1024, 2816
    x = orc.normal(batch * width, 0x1234)
    gamma = orc.values(width, 0x7777, 0.5) + np.float32(1.0)
    wg = orc.normal(width * hidden, 0x3333, 0.0, 0.02)
    wu = orc.normal(width * hidden, 0x4444, 0.0, 0.02)
    wd = orc.normal(hidden * width, 0x5555, 0.0, 0.02)
    eps = 1e-6
    jobs, out = mlp_jobs(runtime, batch, width, hidden, x, gamma, wg, wu, wd, eps)
    runtime.execute(jobs, 1)
    got = runtime.download(out).reshape(batch, width)
    rows = np.r_[0:64, 2016:2080, batch - 64:batch]
    want = orc.mlp(rows.size, width, hidden, x.reshape(batch, width)[rows], gamma, wg, wu, wd,
                   float(np.float32(eps)))
    check = orc.compare(got[rows].reshape(-1), want, 1e-4, 1e-4)
    assert check.status == 0, check.first_bad
