"""A compiled C11 consumer of the drop-in boundary (tests/c/kq4_consumer.c): include/kq4_ops.h and
-lkq4 must compile and link with the reference's C dialect (-std=gnu11 -D_GNU_SOURCE, its x86 flags
tools/build/build_x64.ps1:58-61) under -Wall -Wextra -Werror (CPU), and on the GPU every wrapper,
called with the reference's argument lists (vllm_safetensors.c:8628-8786, :8509-8610, :12921,
:14426), returns 1 and matches the fixtures: tests/golden/dense.npz (the oracle's chains) and
tests/golden/moe.npz (the reference's own MoE output), bar max|got-ref| / max|ref| <= 1e-5."""
import os
import subprocess

import numpy as np
import pytest

import synth
from conftest import rel_err

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c", "kq4_consumer.c")
PKG = os.path.join(ROOT, "kestrel-llm_amd")
GOLD = os.path.join(ROOT, "tests", "golden")
CFLAGS = ["-std=gnu11", "-O2", "-D_GNU_SOURCE", "-mavx2", "-mfma", "-ffp-contract=off", "-Wall",
          "-Wextra", "-Werror"]


def build(tmp_path):
    if not os.path.exists(os.path.join(PKG, "libkq4.so")):
        pytest.fail("libkq4.so not built (run `make -C kestrel-llm_amd`)")
    exe = str(tmp_path / "kq4_consumer")
    cmd = ["gcc", *CFLAGS, "-I", os.path.join(ROOT, "include"), SRC, "-L", PKG, "-lkq4",
           f"-Wl,-rpath,{PKG}", "-Wl,-rpath-link,/opt/rocm/lib", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_consumer_compiles_and_links_as_c11(tmp_path):
    build(tmp_path)


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


@pytest.mark.gpu
def test_consumer_runs_every_wrapper(tmp_path, orc):
    exe = build(tmp_path)
    dense, moe = load("dense.npz"), load("moe.npz")
    rows, cols = int(dense["rows"]), int(dense["cols"])
    assert (rows, cols) == (12, 96) and dense["x"].shape[0] == 5
    rng = np.random.default_rng(77)
    w8 = orc.q8_tiles((rng.standard_normal((16, cols)) * 0.05).astype(np.float32), 16, cols, 8)
    inputs = {"w": dense["w"], "w8": w8, "x": dense["x"], "res": dense["residual"],
              "up": rng.uniform(-2, 2, (5, cols)).astype(np.float32),
              "res8": rng.standard_normal((5, 16)).astype(np.float32),
              "router": moe["router"], "G": moe["G"], "U": moe["U"], "D": moe["D"], "X": moe["X"]}
    for k, v in inputs.items():
        np.ascontiguousarray(v).tofile(str(tmp_path / f"{k}.bin"))
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr

    x, up, res, res8 = inputs["x"], inputs["up"], inputs["res"], inputs["res8"]
    w = dense["w"]
    want = {
        "mv": dense["out_c2"][0], "gu_gate": dense["out_c2"][0], "gu_up": dense["out_c2"][0],
        "qkv_q": dense["out_c2"][0], "qkv_v": dense["out_c2"][0],
        "o_res": dense["res_c2"][0], "down_res": dense["res_c2"][0],
        "silu_down_res": orc.matmul_silu(w, x[:1], up[:1], rows, cols, residual=res[:1])[0],
        "qkv_b_q": dense["out_c0"], "qkv_b_k": dense["out_c0"], "o_res_b": dense["res_c0"],
        "gu_b_up": dense["out_c0"], "down_res_b": dense["res_c0"],
        "silu_down_res_b": orc.matmul_silu(w, x, up, rows, cols, residual=res),
        "q8_mv": orc.q8_matmul(w8, x[:1], 16, cols)[0],
        "q8_o_res": orc.q8_matmul(w8, x[:1], 16, cols, residual=res8[:1])[0],
        "q8_down_res": orc.q8_matmul(w8, x[:1], 16, cols, residual=res8[:1])[0],
        "q8_qkv_b_q": orc.q8_matmul(w8, x, 16, cols),
        "q8_o_res_b": orc.q8_matmul(w8, x, 16, cols, residual=res8),
        "q8_gu_b_gate": orc.q8_matmul(w8, x, 16, cols),
        "q8_down_res_b": orc.q8_matmul(w8, x, 16, cols, residual=res8),
        "moe_1": moe["Y"][0], "moe_b": moe["Y"],
    }
    for name, ref in want.items():
        got = np.fromfile(str(tmp_path / f"{name}.out"), np.float32)
        ref = np.asarray(ref, np.float32).reshape(-1)
        assert got.shape == ref.shape, name
        e, a = rel_err(got, ref)
        print(f"{name}: rel={e:.3e} maxabs={a:.3e}")
        assert e <= 1e-5, name
