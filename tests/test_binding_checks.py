"""The Python binding refuses tensors the library would read out of bounds (wrong device, dtype
or size) before any call reaches libkq4; these checks need no GPU."""
import numpy as np
import pytest


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
