"""The CPU baseline leg (oracle/cpu_bench.py): host facts it reports and the reference entry points
it times, on a tiny shape (a timing baseline, never a parity check: q4g_gemm_mat quantizes the
activations to int16, so its outputs sit near, not on, the oracle's)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "kestrel-llm_amd"))

import oracle  # noqa: E402
import synth  # noqa: E402

needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


def test_host_info():
    import cpu_bench
    h = cpu_bench.host_info()
    assert h["cpus_available"] >= 1
    assert 1 <= h["physical_cores_available"] <= h["cpus_available"]
    assert "socket" in h["lscpu"]


def test_median_and_rotation():
    import cpu_bench
    calls = []
    us = cpu_bench.median_us(cpu_bench.Cycle([1, 2, 3], calls.append), reps=5, warm=1)
    assert us >= 0 and calls == [1, 2, 3, 1, 2, 3]
    assert cpu_bench.n_rot(100 << 20, 0) == 6          # 512 MiB / 100 MiB, rounded up
    assert cpu_bench.n_rot(1 << 30, 0) == 2


@needs_ref
def test_ref_gemm_mat_runs(orc):
    r = oracle.ref()
    r.kref_init(2)
    assert r.kref_num_cpus() >= 1 and r.kref_threads() == 2
    rows, cols, m = 64, 256, 5
    w = synth.make_q4_weights(rows, cols, 3)
    x = synth.make_activations(m, cols, 4)
    out = np.full((m, rows), np.nan, np.float32)
    assert r.kref_gemm_mat(out.ctypes.data, None, w.ctypes.data, x.ctypes.data, rows, cols, m) == 0
    want = orc.matmul(w, x, rows, cols)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - want)) <= 2e-2 * np.max(np.abs(want))
