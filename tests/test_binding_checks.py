"""The Python binding refuses tensors the library would read out of bounds (wrong device, dtype
or size) before any call reaches libkq4; these checks need no GPU."""
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_tensor_refused(kq4_cpu):
    import torch
    x = torch.zeros((2, 64))
    out = torch.zeros((2, 8))
    w = torch.zeros(kq4_cpu.stream_bytes(8, 64), dtype=torch.uint8)
    with pytest.raises(kq4_cpu.KQ4Error, match="device tensor"):
        kq4_cpu.matmul_dev(out, x, w, 8, 64)


def test_shape_mismatch_refused(kq4_cpu):
    import torch
    x = torch.zeros((2, 32))
    with pytest.raises(kq4_cpu.KQ4Error, match="shape"):
        kq4_cpu.matmul_dev(torch.zeros((2, 8)), x, torch.zeros(1, dtype=torch.uint8), 8, 64)


def test_workspace_sizes(kq4_cpu):
    """kq4_matmul_workspace_bytes / kq4_moe_workspace_bytes: 0 for bad shapes, growing with the
    token count, at least the quantized activations' bytes."""
    assert kq4_cpu.matmul_workspace_bytes(4, 33) == 0
    assert kq4_cpu.matmul_workspace_bytes(2048, 12288) >= 2048 * 12288 * 33 // 32
    assert kq4_cpu.matmul_workspace_bytes(8, 4096) > kq4_cpu.matmul_workspace_bytes(1, 4096)
    assert kq4_cpu.moe_workspace_bytes(1, 8, 128, 2048, 33) == 0
    b1 = kq4_cpu.moe_workspace_bytes(1, 8, 128, 2048, 768)
    b64 = kq4_cpu.moe_workspace_bytes(64, 8, 128, 2048, 768)
    assert 0 < b1 < b64 and b64 >= 64 * 8 * 2048 * 4
    assert np.uint64(b64) > 0


def test_option_reset_restores_environment_value():
    """kq4_set_option(name, -1) restores the value the KQ4_* environment variable gave at load,
    not the built-in default (no device needed; a child process, since the environment is read
    once per process)."""
    import subprocess
    import sys
    code = (
        "import kq4\n"
        "assert kq4.get_option('gemv_wpcu') == 40\n"
        "assert kq4.get_option('gemm_tile') == 0\n"
        "with kq4.options(gemv_wpcu=16, gemm_tile=2):\n"
        "    assert kq4.get_option('gemv_wpcu') == 16 and kq4.get_option('gemm_tile') == 2\n"
        "assert kq4.get_option('gemv_wpcu') == 40 and kq4.get_option('gemm_tile') == 0\n"
        "print('ok')\n")
    env = dict(os.environ, KQ4_GEMV_WPCU="40")
    env.pop("KQ4_GEMM_TILE", None)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       cwd=os.path.join(ROOT, "kestrel-llm_amd"), timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr
