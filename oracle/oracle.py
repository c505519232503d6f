"""ctypes wrapper of the parity oracle (oracle/libkq4_oracle.so) and of the reference harness
(oracle/_ref/libkref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, and there only as the checker or the CPU baseline.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libkq4_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkref.so")

CHAIN_AUTO, CHAIN_CTILE, CHAIN_GEMV32, CHAIN_ASM, CHAIN_Q8GEMM = 0, 1, 2, 3, 4

_P = ctypes.c_void_p
_I = ctypes.c_int

_ORACLE_SIGS = [
    ("kqo_f16_to_f32_bits", ctypes.c_uint32, [ctypes.c_uint16]),
    ("kqo_f32_to_f16_bits", ctypes.c_uint16, [ctypes.c_float]),
    ("kqo_f32_to_q4_0", None, [_P, _P, _I]),
    ("kqo_repack_q4_0_4x4", _I, [_P, _P, _I, _I]),
    ("kqo_unpack_4x4_to_q4_0", _I, [_P, _P, _I, _I]),
    ("kqo_tile_weight", _I, [_P, _I, _I]),
    ("kqo_quantize_rows", None, [_P, _P, _P, _I, _I]),
    ("kqo_block_sums", None, [_P, _P, _I, _I, _I, _P, _P]),
    ("kqo_matmul", _I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    ("kqo_matmul_q", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    ("kqo_matmul_q_sample", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I]),
    ("kqo_matmul_f64", None, [_P, _P, _P, _P, _I, _I, _I]),
    ("kqo_moe_route", None, [_P, _I, _I, _P, _P]),
    ("kqo_router_logits", None, [_P, _P, _I, _I, _P]),
    ("kqo_silu_mul", ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
    ("kqo_exp_neon", ctypes.c_float, [ctypes.c_float]),
    ("kqo_frecpe", ctypes.c_float, [ctypes.c_float]),
    ("kqo_silu_mul_neon", ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
    ("kqo_fast_silu", ctypes.c_float, [ctypes.c_float]),
    ("kqo_silu_mul_rows", None, [_P, _P, ctypes.c_long]),
    ("kqo_matmul_silu", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    ("kqo_rms_norm", None, [_P, _P, _P, _I, _I, ctypes.c_float, _I]),
    ("kqo_f32_to_q8_0", None, [_P, _P, _I]),
    ("kqo_repack_q8_0_tiled", _I, [_P, _P, _I, _I, _I]),
    ("kqo_q8_matmul_q", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    ("kqo_q8_matmul", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
    ("kqo_moe_ffn", _I, [_P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I,
                         _P, _P, _P, _P, _P, _P, _P]),
]

_REF_SIGS = [
    ("kref_init", _I, [_I]),
    ("kref_f16_to_f32_bits", ctypes.c_uint32, [ctypes.c_uint16]),
    ("kref_f32_to_f16_bits", ctypes.c_uint16, [ctypes.c_float]),
    ("kref_vq_f16", ctypes.c_float, [ctypes.c_uint16]),
    ("kref_quantize_row", None, [_P, _P, _P, _I]),
    ("kref_f32_to_q4_0", None, [_P, _P, _I]),
    ("kref_repack_q4_0_4x4", _I, [_P, _I, _I]),
    ("kref_moe_ffn", _I, [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I]),
    ("kref_gate_up_batched", None, [_P, _P, _P, _P, _P, _I, _I, _I]),
    ("kref_qkv_batched", None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
    ("kref_o_residual_batched", None, [_P, _P, _P, _P, _I, _I, _I]),
    ("kref_down_residual_batched", None, [_P, _P, _P, _P, _I, _I, _I]),
    ("kref_matvec", None, [_P, _P, _P, _I, _I]),
    ("kref_silu_mul", None, [_P, _P, _I]),
    ("kref_rms_norm", None, [_P, _P, _P, _I, ctypes.c_float]),
    ("kref_f32_to_q8_0", None, [_P, _P, _I]),
    ("kref_repack_q8_0_8x8", _I, [_P, _I, _I]),
    ("kref_repack_q8_0_4x4", _I, [_P, _I, _I]),
    ("kref_rms_norm_batch", None, [_P, _P, _P, _I, _I, ctypes.c_float]),
    ("kref_gemm_mat", _I, [_P, _P, _P, _P, _I, _I, _I]),
    ("kref_num_cpus", ctypes.c_long, []),
    ("kref_threads", _I, []),
]

_oracle = None
_ref = None


def build(with_ref=True):
    """Builds the oracle (and the reference harness when /root/reference exists)."""
    target = "all" if with_ref else "oracle"
    subprocess.run(["make", "-s", "-C", HERE, target], check=True)


def _bind(path, sigs, mode=0):
    h = ctypes.CDLL(path, mode=mode)
    for name, res, args in sigs:
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def lib():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build(with_ref=False)
        _oracle = _bind(ORACLE_SO, _ORACLE_SIGS)
    return _oracle


def ref_available():
    return os.path.exists(REF_SO)


def ref(threads=1):
    """The reference's own x86-64 code (see ref_harness.c); RTLD_LAZY because the RK3588 NPU
    entry points it never reaches stay unresolved."""
    global _ref
    if _ref is None:
        _ref = _bind(REF_SO, _REF_SIGS, mode=os.RTLD_LAZY)
        _ref.kref_init(threads)
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def quantize(x, cols):
    x = _c(x, np.float32).reshape(-1, cols)
    n = x.shape[0]
    q = np.empty((n, cols), np.int8)
    d = np.empty((n, cols // 32), np.float32)
    lib().kqo_quantize_rows(_p(x), _p(q), _p(d), n, cols)
    return q, d


def block_sums(w, xq, rows, cols):
    xq = _c(xq, np.int8).reshape(-1, cols)
    n = xq.shape[0]
    lo = np.empty((n, rows, cols // 32), np.int32)
    hi = np.empty_like(lo)
    lib().kqo_block_sums(_p(_c(w, np.uint8)), _p(xq), rows, cols, n, _p(lo), _p(hi))
    return lo, hi


def matmul(w, x, rows, cols, residual=None, chain=CHAIN_AUTO):
    x = _c(x, np.float32).reshape(-1, cols)
    n = x.shape[0]
    out = np.empty((n, rows), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_matmul(_p(out), _p(x), _p(res), _p(_c(w, np.uint8)), rows, cols, n, chain)
    assert rc == 0
    return out


def matmul_q(w, xq, xd, rows, cols, residual=None, chain=CHAIN_AUTO):
    xq = _c(xq, np.int8).reshape(-1, cols)
    n = xq.shape[0]
    out = np.empty((n, rows), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_matmul_q(_p(out), _p(xq), _p(_c(xd, np.float32)), _p(res),
                            _p(_c(w, np.uint8)), rows, cols, n, chain)
    assert rc == 0
    return out


def matmul_q_sample(w, xq, xd, rows, cols, n_batch, tok, row, residual=None, chain=CHAIN_AUTO):
    tok = _c(tok, np.int32)
    row = _c(row, np.int32)
    out = np.empty(tok.shape[0], np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_matmul_q_sample(_p(out), _p(_c(xq, np.int8)), _p(_c(xd, np.float32)), _p(res),
                                   _p(_c(w, np.uint8)), rows, cols, n_batch, chain, _p(tok),
                                   _p(row), tok.shape[0])
    assert rc == 0
    return out


def silu_mul(g, u):
    """vllm_silu_mul_worker over the flattened arrays (NEON form; last n % 4 scalar)."""
    g = _c(g, np.float32).copy()
    u = _c(u, np.float32)
    assert g.size == u.size
    lib().kqo_silu_mul_rows(_p(g), _p(u), g.size)
    return g


def matmul_silu(w, gate, up, rows, cols, residual=None, chain=CHAIN_AUTO):
    gate = _c(gate, np.float32).reshape(-1, cols)
    up = _c(up, np.float32).reshape(-1, cols)
    n = gate.shape[0]
    out = np.empty((n, rows), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_matmul_silu(_p(out), _p(gate), _p(up), _p(res), _p(_c(w, np.uint8)), rows,
                               cols, n, chain)
    assert rc == 0
    return out


def q8_tiles(wf, rows, cols, g=8):
    """Q8_0 tiles (g = 8: block_q8_0x8, VQF_FLAG_Q8_8X8; g = 4: block_q8_0x4) of fp32 weights."""
    wf = _c(wf, np.float32).reshape(rows, cols)
    legacy = np.empty(rows * cols // 32 * 34, np.uint8)
    lib().kqo_f32_to_q8_0(_p(legacy), _p(wf), rows * cols)
    tiles = np.empty_like(legacy)
    assert lib().kqo_repack_q8_0_tiled(_p(legacy), _p(tiles), g, rows, cols) == 0
    return tiles


def q8_matmul(w, x, rows, cols, residual=None, chain=CHAIN_AUTO, g=8):
    x = _c(x, np.float32).reshape(-1, cols)
    n = x.shape[0]
    out = np.empty((n, rows), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_q8_matmul(_p(out), _p(x), _p(res), _p(_c(w, np.uint8)), g, rows, cols, n,
                             chain)
    assert rc == 0
    return out


def q8_matmul_q(w, xq, xd, rows, cols, residual=None, chain=CHAIN_AUTO, g=8):
    xq = _c(xq, np.int8).reshape(-1, cols)
    n = xq.shape[0]
    out = np.empty((n, rows), np.float32)
    res = None if residual is None else _c(residual, np.float32)
    rc = lib().kqo_q8_matmul_q(_p(out), _p(xq), _p(_c(xd, np.float32)), _p(res),
                               _p(_c(w, np.uint8)), g, rows, cols, n, chain)
    assert rc == 0
    return out


def rms_norm(x, w, d, eps, chunked=True):
    x = _c(x, np.float32).reshape(-1, d)
    out = np.empty_like(x)
    lib().kqo_rms_norm(_p(out), _p(x), _p(_c(w, np.float32)), x.shape[0], d, eps, int(chunked))
    return out


def matmul_f64(w, xq, xd, rows, cols):
    xq = _c(xq, np.int8).reshape(-1, cols)
    n = xq.shape[0]
    out = np.empty((n, rows), np.float64)
    lib().kqo_matmul_f64(_p(out), _p(xq), _p(_c(xd, np.float32)), _p(_c(w, np.uint8)), rows,
                         cols, n)
    return out


def moe_route(logits, tk):
    logits = _c(logits, np.float32)
    T, ne = logits.shape
    sel = np.empty((T, tk), np.int32)
    pr = np.empty((T, tk), np.float32)
    for t in range(T):
        lib().kqo_moe_route(_p(logits[t]), ne, tk, _p(sel[t]), _p(pr[t]))
    return sel, pr


def router_logits(router, x, ne, d):
    x = _c(x, np.float32).reshape(-1, d)
    out = np.empty((x.shape[0], ne), np.float32)
    for t in range(x.shape[0]):
        lib().kqo_router_logits(_p(_c(router, np.float32)), _p(x[t]), ne, d, _p(out[t]))
    return out


def moe_ffn(X, sel, pr, G, U, D, ne, d, ef, av_in=None, stages=False):
    X = _c(X, np.float32).reshape(-1, d)
    T = X.shape[0]
    sel = _c(sel, np.int32)
    pr = _c(pr, np.float32)
    tk = sel.shape[1]
    Y = np.empty((T, d), np.float32)
    st = {}
    if stages:
        st = dict(gate=np.zeros((T * tk, ef), np.float32), up=np.zeros((T * tk, ef), np.float32),
                  av=np.zeros((T * tk, ef), np.float32), avq=np.zeros((T * tk, ef), np.int8),
                  avd=np.zeros((T * tk, ef // 32), np.float32),
                  P=np.zeros((T * tk, d), np.float32))
    rc = lib().kqo_moe_ffn(_p(Y), _p(X), _p(sel), _p(pr), T, tk, _p(_c(G, np.uint8)),
                           _p(_c(U, np.uint8)), _p(_c(D, np.uint8)), ne, d, ef,
                           _p(st.get("gate")), _p(st.get("up")), _p(st.get("av")),
                           _p(st.get("avq")), _p(st.get("avd")), _p(st.get("P")),
                           _p(None if av_in is None else _c(av_in, np.float32)))
    assert rc == 0
    return (Y, st) if stages else Y
