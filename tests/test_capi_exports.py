"""libkq4.so loads without a GPU and exports every entry point include/kq4.h, include/kq4_ops.h
and include/kq4_vqf.h declare (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kq4.h", "kq4_ops.h", "kq4_vqf.h")]


def declared(path):
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(kq4_\w+)\s*\(", src, flags=re.M)))


def test_headers_declare_entry_points():
    names = declared(HEADERS[0])
    assert {"kq4_init", "kq4_matmul", "kq4_matmul_dev", "kq4_moe_ffn_dev"} <= set(names)
    assert "kq4_dyn_matvec_q4_q8_fused_gate_up_batched" in declared(HEADERS[1])


@pytest.mark.parametrize("header", HEADERS)
def test_library_exports_every_declared_symbol(header):
    import kq4
    if not os.path.exists(kq4.LIB_PATH):
        pytest.fail(f"{kq4.LIB_PATH} not built (run `make -C kestrel-llm_amd`)")
    lib = ctypes.CDLL(kq4.LIB_PATH)
    missing = [n for n in declared(header) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_symbol():
    import kq4
    bound = {n for n, _, _ in kq4.SIGNATURES}
    for h in HEADERS:
        assert set(declared(h)) <= bound, set(declared(h)) - bound
