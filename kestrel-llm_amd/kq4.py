"""Python binding of libkq4.so (include/kq4.h) over ctypes.

Host side for tests and the benchmark: numpy arrays go through the host-pointer drop-in API
(1 = done on the GPU / 0 = not done, as the reference's NPU hook), device tensors (torch on ROCm,
used only as HBM allocations and streams) through the device-pointer API. There is no CPU path
here: if the library is missing or a call fails, the call raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkq4.so")

CHAIN_AUTO, CHAIN_CTILE, CHAIN_GEMV32, CHAIN_ASM, CHAIN_Q8GEMM = 0, 1, 2, 3, 4
MAX_MATS = 4

_P = ctypes.c_void_p
_I = ctypes.c_int
_U64 = ctypes.c_uint64

# (name, restype, argtypes) for every entry point include/kq4.h declares
SIGNATURES = [
    ("kq4_init", _I, [_I]),
    ("kq4_shutdown", None, []),
    ("kq4_last_error", ctypes.c_char_p, []),
    ("kq4_version", ctypes.c_char_p, []),
    ("kq4_set_option", _I, [ctypes.c_char_p, _I]),
    ("kq4_get_option", _I, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]),
    ("kq4_gemm_plan_info", _I, [_I, _I, _I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    ("kq4_weights_upload", _I, [_U64, _P, _I, _I]),
    ("kq4_weights_evict", _I, [_U64]),
    ("kq4_weights_clear", _I, []),
    ("kq4_matmul", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _U64]),
    ("kq4_matmul_multi", _I, [_I, _P, _P, _P, _P, _I, _P, _I, _I, _P]),
    ("kq4_matmul_silu", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _U64]),
    ("kq4_q8_matmul", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _U64]),
    ("kq4_q8_matmul_multi", _I, [_I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _P]),
    ("kq4_q8_weights_stream_bytes", ctypes.c_size_t, [_I, _I]),
    ("kq4_q8_weights_prepare_dev", _I, [_P, _P, _I, _I, _I, _P]),
    ("kq4_q8_weights_prepare_host", _I, [_P, _P, _I, _I, _I, _P]),
    ("kq4_q8_matmul_dev", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("kq4_q8_matmul_multi_dev", _I, [_I, _P, _P, _P, _P, _I, _P, _I, _I, _P]),
    ("kq4_moe_ffn", _I, [_P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I, _U64]),
    ("kq4_weights_stream_bytes", ctypes.c_size_t, [_I, _I]),
    ("kq4_matmul_workspace_bytes", ctypes.c_size_t, [_I, _I]),
    ("kq4_moe_workspace_bytes", ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    ("kq4_workspace_reserve", _I, [ctypes.c_size_t]),
    ("kq4_workspace_trim", _I, []),
    ("kq4_weights_prepare_dev", _I, [_P, _P, _I, _I, _P]),
    ("kq4_quantize_dev", _I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    ("kq4_matmul_dev", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("kq4_matmul_noalloc_dev", _I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("kq4_matmul_multi_dev", _I, [_I, _P, _P, _P, _P, _I, _P, _I, _I, _P]),
    ("kq4_matmul_silu_dev", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("kq4_silu_mul_dev", _I, [_P, _P, ctypes.c_long, _P]),
    ("kq4_rms_norm_dev", _I, [_P, _P, _P, _I, _I, ctypes.c_float, _I, _P]),
    ("kq4_rmsnorm_matmul_multi_dev", _I, [_I, _P, _P, _P, _P, _I, _P, _P, ctypes.c_float, _I,
                                          _P, _I, _I, _P]),
    ("kq4_matmul_q_dev", _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    ("kq4_matmul_multi_q_dev", _I, [_I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P]),
    ("kq4_block_sums_dev", _I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    ("kq4_moe_route_dev", _I, [_P, _P, _P, _I, _I, _I, _P]),
    ("kq4_moe_ffn_dev", _I, [_P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I, _P]),
    ("kq4_moe_router_logits_dev", _I, [_P, _P, _P, _I, _I, _I, _P]),
    ("kq4_moe_layer_dev", _I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    ("kq4_moe_ffn_stages_dev", _I,
     [_P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P]),
    # C11 op wrappers (include/kq4_ops.h)
    ("kq4_dyn_matvec_q4_q8", _I, [_P, _P, _P, _I, _I]),
    ("kq4_dyn_matvec_q4_q8_fused_gate_up", _I, [_P, _P, _P, _P, _P, _I, _I]),
    ("kq4_dyn_matvec_q4_q8_fused_qkv", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    ("kq4_dyn_matvec_q4_q8_fused_o_residual", _I, [_P, _P, _P, _P, _I, _I]),
    ("kq4_dyn_matvec_q4_q8_fused_down_residual", _I, [_P, _P, _P, _P, _I, _I]),
    ("kq4_silu_mul_down_residual", _I, [_P, _P, _P, _P, _P, _I, _I]),
    ("kq4_silu_mul_down_residual_batched", _I, [_P, _P, _P, _P, _P, _I, _I, _I]),
    ("kq4_dyn_matvec_q4_q8_fused_qkv_batched", _I,
     [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
    ("kq4_dyn_matvec_q4_q8_fused_o_residual_batched", _I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    ("kq4_dyn_matvec_q4_q8_fused_gate_up_batched", _I,
     [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P]),
    ("kq4_dyn_matvec_q4_q8_fused_down_residual_batched", _I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    ("kq4_dyn_matvec_q8", _I, [_P, _P, _P, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_qkv_batched", _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_o_residual_batched", _I, [_P, _P, _P, _P, _I, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_gate_up_batched", _I, [_P, _P, _P, _P, _P, _I, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_down_residual_batched", _I, [_P, _P, _P, _P, _I, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_o_residual", _I, [_P, _P, _P, _P, _I, _I]),
    ("kq4_dyn_matvec_q8_fused_down_residual", _I, [_P, _P, _P, _P, _I, _I]),
    ("kq4_st_moe_ffn_sparse_q4", _I, [_P, _P, _P]),
    ("kq4_st_moe_ffn_sparse_q4_batch", _I, [_P, _I, _P, _P]),
    # include/kq4_vqf.h
    ("kq4_weights_prepare_host", _I, [_P, _P, _I, _I, _P]),
    ("kq4_vqf_parse_header", _I, [_P, ctypes.c_size_t, _U64, _P]),
    ("kq4_vqf_open", _I, [ctypes.c_char_p, _I, ctypes.POINTER(_P)]),
    ("kq4_vqf_close", None, [_P]),
    ("kq4_vqf_get_info", _P, [_P]),
    ("kq4_vqf_entry", _I, [_P, _I, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                           ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                           ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    ("kq4_vqf_find", _I, [_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    ("kq4_vqf_q4_matrix", _I, [_P, _I, _I, ctypes.POINTER(_P), ctypes.POINTER(_I),
                               ctypes.POINTER(_I)]),
    ("kq4_vqf_prepare_dev", _I, [_P, _I, _I, _P, _P]),
    ("kq4_vqf_q8_matrix", _I, [_P, _I, _I, ctypes.POINTER(_P), ctypes.POINTER(_I),
                               ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    ("kq4_vqf_prepare_q8_dev", _I, [_P, _I, _I, _P, _P]),
    ("kq4_vqf_upload", _I, [_P, _I, _I, ctypes.POINTER(_U64)]),
]

PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN, PROJ_LM = range(8)


class VqfInfo(ctypes.Structure):
    """kq4_vqf_info (include/kq4_vqf.h)."""
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "version", "flags", "n_tensors", "dim", "n_layers", "n_heads", "n_kv_heads",
        "head_dim", "ffn_dim", "vocab_size")] + [
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float)] + [
        (n, ctypes.c_uint32) for n in ("n_experts", "moe_ffn", "top_k")] + [
        ("data_offset", _U64), ("file_len", _U64), ("legacy_header", _I)]


class KQ4Error(RuntimeError):
    pass


class MoeLayer(ctypes.Structure):
    """kq4_moe_layer (include/kq4_ops.h)."""
    _fields_ = [("router", _P), ("G", _P), ("U", _P), ("D", _P), ("n_experts", _I),
                ("top_k", _I), ("dim", _I), ("ef", _I)]


_lib = None


def lib():
    """Loads libkq4.so (built in-tree by `make -C kestrel-llm_amd`); raises if absent."""
    global _lib
    if _lib is None:
        # torch's wheel ships its own libamdhip64.so.7 (same soname as /opt/rocm's). Whichever
        # loads first serves the whole process, and torch cannot use the system one; so when
        # torch is installed, let it load first and libkq4 binds to the same runtime.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise KQ4Error(f"{LIB_PATH} is missing: build it with `make -C kestrel-llm_amd` "
                           "(or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error():
    return lib().kq4_last_error().decode(errors="replace")


def check(rc, what):
    """Device API: 0 = ok, negative = error."""
    if rc != 0:
        raise KQ4Error(f"{what} failed ({rc}): {last_error()}")


def check_done(rc, what):
    """Host drop-in API: 1 = done on the GPU, 0 = not done."""
    if rc != 1:
        raise KQ4Error(f"{what} not executed: {last_error()}")


def init(device=0):
    check(lib().kq4_init(device), "kq4_init")


def set_option(name, value):
    """A launch-planner option (include/kq4.h kq4_set_option); value < 0 restores its initial
    value (the KQ4_* environment variable, else the built-in default)."""
    check(lib().kq4_set_option(name.encode(), int(value)), f"kq4_set_option({name})")


def get_option(name):
    v = ctypes.c_int(0)
    check(lib().kq4_get_option(name.encode(), ctypes.byref(v)), f"kq4_get_option({name})")
    return v.value


def gemm_plan(n_batch, rows, cols, q8=False, chain=0, ncu=0):
    """(tile, K slices) of an n_batch-token matmul under the current options: (0, 0) for the
    decode GEMV, else the prefill GEMM's tile (1-4 as option gemm_tile) and slices (include/kq4.h
    kq4_gemm_plan_info; ncu 0 = the current device's CUs)."""
    t, k = ctypes.c_int(), ctypes.c_int()
    check(lib().kq4_gemm_plan_info(n_batch, rows, cols, int(q8), chain, ncu, ctypes.byref(t),
                                   ctypes.byref(k)), "kq4_gemm_plan_info")
    return t.value, k.value


class options:
    """Context manager setting planner options and restoring their initial values on exit."""

    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        for k, v in self.kv.items():
            set_option(k, v)
        return self

    def __exit__(self, *a):
        for k in self.kv:
            set_option(k, -1)


def _np_ptr(a):
    return a.ctypes.data if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr_array(ptrs):
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


# ---- host-pointer API (numpy) ---------------------------------------------------------------

def matmul(w, x, rows, cols, residual=None, chain=CHAIN_AUTO, wkey=0):
    """out[n_batch][rows] = [residual +] W.x through kq4_matmul (host pointers)."""
    x = _c(x, np.float32).reshape(-1, cols)
    w = _c(w, np.uint8)
    out = np.empty((x.shape[0], rows), np.float32)
    res = None if residual is None else _c(residual, np.float32).reshape(x.shape[0], rows)
    check_done(lib().kq4_matmul(_np_ptr(out), _np_ptr(x), _np_ptr(res), _np_ptr(w), rows, cols,
                                x.shape[0], chain, wkey), "kq4_matmul")
    return out


def matmul_silu(w, gate, up, rows, cols, residual=None, chain=CHAIN_AUTO, wkey=0):
    """out = [residual +] W.silu_mul(gate, up) through kq4_matmul_silu (host pointers)."""
    gate = _c(gate, np.float32).reshape(-1, cols)
    up = _c(up, np.float32).reshape(gate.shape)
    out = np.empty((gate.shape[0], rows), np.float32)
    res = None if residual is None else _c(residual, np.float32).reshape(gate.shape[0], rows)
    check_done(lib().kq4_matmul_silu(_np_ptr(out), _np_ptr(gate), _np_ptr(up), _np_ptr(res),
                                     _np_ptr(_c(w, np.uint8)), rows, cols, gate.shape[0], chain,
                                     wkey), "kq4_matmul_silu")
    return out


def q8_matmul(w, x, rows, cols, residual=None, chain=CHAIN_AUTO, wkey=0, g=8):
    """out = [residual +] W.x for Q8_0 tiles of g rows through kq4_q8_matmul (host pointers)."""
    x = _c(x, np.float32).reshape(-1, cols)
    out = np.empty((x.shape[0], rows), np.float32)
    res = None if residual is None else _c(residual, np.float32).reshape(x.shape[0], rows)
    check_done(lib().kq4_q8_matmul(_np_ptr(out), _np_ptr(x), _np_ptr(res),
                                   _np_ptr(_c(w, np.uint8)), g, rows, cols, x.shape[0], chain,
                                   wkey), "kq4_q8_matmul")
    return out


def matmul_multi(ws, rows, x, cols, residuals=None, chain=CHAIN_AUTO, wkeys=None):
    x = _c(x, np.float32).reshape(-1, cols)
    n = x.shape[0]
    ws = [_c(w, np.uint8) for w in ws]
    outs = [np.empty((n, r), np.float32) for r in rows]
    res = [None] * len(ws) if residuals is None else [
        None if r is None else _c(r, np.float32) for r in residuals]
    keys = None if wkeys is None else (ctypes.c_uint64 * len(ws))(*wkeys)
    rc = lib().kq4_matmul_multi(len(ws), _ptr_array([o.ctypes.data for o in outs]),
                                _ptr_array([_np_ptr(r) for r in res]),
                                _ptr_array([w.ctypes.data for w in ws]),
                                (ctypes.c_int * len(rows))(*rows), cols, _np_ptr(x), n, chain,
                                keys)
    check_done(rc, "kq4_matmul_multi")
    return outs


def moe_ffn(X, sel, pr, G, U, D, ne, d, ef, wkey=0):
    X = _c(X, np.float32).reshape(-1, d)
    T = X.shape[0]
    sel = _c(sel, np.int32).reshape(T, -1)
    pr = _c(pr, np.float32).reshape(T, -1)
    Y = np.empty((T, d), np.float32)
    check_done(lib().kq4_moe_ffn(_np_ptr(Y), _np_ptr(X), _np_ptr(sel), _np_ptr(pr), T,
                                 sel.shape[1], _np_ptr(_c(G, np.uint8)), _np_ptr(_c(U, np.uint8)),
                                 _np_ptr(_c(D, np.uint8)), ne, d, ef, wkey), "kq4_moe_ffn")
    return Y


# ---- device-pointer API (torch tensors as HBM buffers) ----------------------------------------

def _tp(t):
    return None if t is None else t.data_ptr()


def _need(t, name, dtype, numel, optional=False):
    """Raises unless t is a contiguous device tensor of `dtype` with at least `numel` elements
    (the library reads and writes raw pointers: a wrong view would be read out of bounds)."""
    import torch
    if t is None:
        if optional:
            return
        raise KQ4Error(f"{name}: missing")
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise KQ4Error(f"{name}: not a device tensor")
    if t.dtype != dtype:
        raise KQ4Error(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise KQ4Error(f"{name}: not contiguous")
    if t.numel() < numel:
        raise KQ4Error(f"{name}: {t.numel()} elements, needs {numel}")


def _act(x, cols, name="x"):
    """Token count of a [n][cols] fp32 activation tensor, checked."""
    import torch
    if x is None or x.dim() != 2 or x.shape[1] != cols:
        raise KQ4Error(f"{name}: expected shape [n, {cols}], got "
                       f"{None if x is None else tuple(x.shape)}")
    _need(x, name, torch.float32, x.shape[0] * cols)
    return x.shape[0]


def _mat(w, rows, cols, q8=False):
    import torch
    _need(w, "weights", torch.uint8, (q8_stream_bytes if q8 else stream_bytes)(rows, cols))


def _outs(outs, residuals, rows, n):
    import torch
    if len(outs) != len(rows) or (residuals is not None and len(residuals) != len(rows)):
        raise KQ4Error("one output (and residual) per matrix")
    for i, (o, r) in enumerate(zip(outs, rows)):
        _need(o, f"out[{i}]", torch.float32, n * r)
        if residuals is not None:
            _need(residuals[i], f"residual[{i}]", torch.float32, n * r, optional=True)


def _stream_ptr(stream):
    return None if stream is None else stream.cuda_stream


def matmul_workspace_bytes(n_batch, cols):
    return lib().kq4_matmul_workspace_bytes(n_batch, cols)


def moe_workspace_bytes(T, tk, ne, d, ef):
    return lib().kq4_moe_workspace_bytes(T, tk, ne, d, ef)


def workspace_reserve(nbytes):
    """Grows the device workspace before a HIP graph capture (see include/kq4.h)."""
    check(lib().kq4_workspace_reserve(nbytes), "kq4_workspace_reserve")


def workspace_trim():
    """Frees the outgrown workspaces once no graph captured before their growth is alive."""
    check(lib().kq4_workspace_trim(), "kq4_workspace_trim")


def stream_bytes(rows, cols):
    n = lib().kq4_weights_stream_bytes(rows, cols)
    if n == 0:
        raise KQ4Error(f"bad q4 matrix shape {rows}x{cols}")
    return n


def prepare_dev(w4x4, rows, cols, stream=None):
    """Stream-layout device copy (a new uint8 tensor) of the VQF 4x4 matrix w4x4, a device
    tensor or a host numpy array (copied to the device first); what every device-pointer call
    takes as its weights."""
    import torch
    if isinstance(w4x4, np.ndarray):
        w4x4 = torch.from_numpy(np.ascontiguousarray(w4x4, dtype=np.uint8)).cuda()
    dst = torch.empty(stream_bytes(rows, cols), dtype=torch.uint8, device=w4x4.device)
    check(lib().kq4_weights_prepare_dev(_tp(dst), _tp(w4x4), rows, cols, _stream_ptr(stream)),
          "kq4_weights_prepare_dev")
    return dst


def q8_stream_bytes(rows, cols):
    n = lib().kq4_q8_weights_stream_bytes(rows, cols)
    if n == 0:
        raise KQ4Error(f"bad q8 matrix shape {rows}x{cols}")
    return n


def q8_prepare_dev(tiles, rows, cols, g=8, stream=None):
    """q8 stream-layout device copy (a new uint8 tensor) of Q8_0 tiles of g rows (a device
    tensor, or a host numpy array)."""
    import torch
    dst = torch.empty(q8_stream_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    if isinstance(tiles, np.ndarray):
        t = np.ascontiguousarray(tiles, dtype=np.uint8)
        check(lib().kq4_q8_weights_prepare_host(_tp(dst), t.ctypes.data, g, rows, cols,
                                                _stream_ptr(stream)), "kq4_q8_weights_prepare_host")
    else:
        check(lib().kq4_q8_weights_prepare_dev(_tp(dst), _tp(tiles), g, rows, cols,
                                               _stream_ptr(stream)), "kq4_q8_weights_prepare_dev")
    return dst


def q8_matmul_dev(out, x, w, rows, cols, residual=None, chain=CHAIN_AUTO, stream=None):
    n = _act(x, cols)
    _mat(w, rows, cols, q8=True)
    _outs([out], [residual], [rows], n)
    check(lib().kq4_q8_matmul_dev(_tp(out), _tp(x), _tp(residual), _tp(w), rows, cols, n, chain,
                                  _stream_ptr(stream)), "kq4_q8_matmul_dev")


def q8_matmul_multi_dev(outs, x, ws, rows, cols, residuals=None, chain=CHAIN_AUTO, stream=None):
    n = _act(x, cols)
    for w, r in zip(ws, rows):
        _mat(w, r, cols, q8=True)
    _outs(outs, residuals, rows, n)
    res = [None] * len(ws) if residuals is None else residuals
    check(lib().kq4_q8_matmul_multi_dev(len(ws), _ptr_array([_tp(o) for o in outs]),
                                        _ptr_array([_tp(r) for r in res]),
                                        _ptr_array([_tp(w) for w in ws]),
                                        (ctypes.c_int * len(rows))(*rows), cols, _tp(x), n,
                                        chain, _stream_ptr(stream)), "kq4_q8_matmul_multi_dev")


def quantize_dev(x, xq, xd, xde=None, chain=CHAIN_AUTO, stream=None):
    import torch
    n, cols = x.shape
    _act(x, cols)
    _need(xq, "xq", torch.int8, n * cols)
    _need(xd, "xd", torch.float32, n * (cols // 32))
    _need(xde, "xde", torch.float32, n * (cols // 32), optional=True)
    check(lib().kq4_quantize_dev(_tp(xq), _tp(xd), _tp(xde), _tp(x), n, cols, chain,
                                 _stream_ptr(stream)), "kq4_quantize_dev")


def matmul_dev(out, x, w, rows, cols, residual=None, chain=CHAIN_AUTO, stream=None):
    n = _act(x, cols)
    _mat(w, rows, cols)
    _outs([out], [residual], [rows], n)
    check(lib().kq4_matmul_dev(_tp(out), _tp(x), _tp(residual), _tp(w), rows, cols, n, chain,
                               _stream_ptr(stream)), "kq4_matmul_dev")


NOALLOC_SCRATCH_BYTES = 64 << 20


def matmul_noalloc_dev(out, x, w, rows, cols, residual=None, chain=CHAIN_AUTO, stream=None):
    """kq4_matmul_dev without any device allocation (fixed per-device scratch)."""
    n = _act(x, cols)
    _mat(w, rows, cols)
    _outs([out], [residual], [rows], n)
    check(lib().kq4_matmul_noalloc_dev(_tp(out), _tp(x), _tp(residual), _tp(w), rows, cols, n,
                                       chain, _stream_ptr(stream)), "kq4_matmul_noalloc_dev")


def matmul_silu_dev(out, gate, up, w, rows, cols, residual=None, chain=CHAIN_AUTO, stream=None):
    n = _act(gate, cols, "gate")
    if _act(up, cols, "up") != n:
        raise KQ4Error("gate and up differ in tokens")
    _mat(w, rows, cols)
    _outs([out], [residual], [rows], n)
    check(lib().kq4_matmul_silu_dev(_tp(out), _tp(gate), _tp(up), _tp(residual), _tp(w), rows,
                                    cols, n, chain, _stream_ptr(stream)), "kq4_matmul_silu_dev")


RMS_CHUNKED, RMS_SERIAL = 0, 1


def rms_norm_dev(out, x, w, eps, order=RMS_CHUNKED, stream=None):
    import torch
    n, d = x.shape
    _act(x, d)
    _need(out, "out", torch.float32, n * d)
    _need(w, "w", torch.float32, d)
    check(lib().kq4_rms_norm_dev(_tp(out), _tp(x), _tp(w), n, d, eps, order,
                                 _stream_ptr(stream)), "kq4_rms_norm_dev")


def rmsnorm_matmul_multi_dev(outs, x, norm_w, eps, ws, rows, cols, residuals=None,
                             order=RMS_CHUNKED, normed=None, chain=CHAIN_AUTO, stream=None):
    import torch
    n = _act(x, cols)
    _need(norm_w, "norm_w", torch.float32, cols)
    _need(normed, "normed", torch.float32, n * cols, optional=True)
    for w, r in zip(ws, rows):
        _mat(w, r, cols)
    _outs(outs, residuals, rows, n)
    res = [None] * len(ws) if residuals is None else residuals
    check(lib().kq4_rmsnorm_matmul_multi_dev(
        len(ws), _ptr_array([_tp(o) for o in outs]), _ptr_array([_tp(r) for r in res]),
        _ptr_array([_tp(w) for w in ws]), (ctypes.c_int * len(rows))(*rows), cols, _tp(x),
        _tp(norm_w), eps, order, _tp(normed), n, chain, _stream_ptr(stream)),
        "kq4_rmsnorm_matmul_multi_dev")


def silu_mul_dev(gate, up, stream=None):
    """gate <- silu_mul(gate, up) in place (the reference worker's element rule)."""
    import torch
    _need(gate, "gate", torch.float32, up.numel())
    _need(up, "up", torch.float32, gate.numel())
    check(lib().kq4_silu_mul_dev(_tp(gate), _tp(up), gate.numel(), _stream_ptr(stream)),
          "kq4_silu_mul_dev")


def matmul_multi_dev(outs, x, ws, rows, cols, residuals=None, chain=CHAIN_AUTO, stream=None):
    n = _act(x, cols)
    for w, r in zip(ws, rows):
        _mat(w, r, cols)
    _outs(outs, residuals, rows, n)
    res = [None] * len(ws) if residuals is None else residuals
    check(lib().kq4_matmul_multi_dev(len(ws), _ptr_array([_tp(o) for o in outs]),
                                     _ptr_array([_tp(r) for r in res]),
                                     _ptr_array([_tp(w) for w in ws]),
                                     (ctypes.c_int * len(rows))(*rows), cols, _tp(x), n, chain,
                                     _stream_ptr(stream)), "kq4_matmul_multi_dev")


def _qact(xq, xd, cols, n):
    import torch
    _need(xq, "xq", torch.int8, n * cols)
    _need(xd, "xd", torch.float32, n * (cols // 32))


def matmul_q_dev(out, xq, xd, w, rows, cols, n, residual=None, chain=CHAIN_AUTO, stream=None):
    _qact(xq, xd, cols, n)
    _mat(w, rows, cols)
    _outs([out], [residual], [rows], n)
    check(lib().kq4_matmul_q_dev(_tp(out), _tp(xq), _tp(xd), _tp(residual), _tp(w), rows, cols,
                                 n, chain, _stream_ptr(stream)), "kq4_matmul_q_dev")


def matmul_multi_q_dev(outs, xq, xd, ws, rows, cols, n, residuals=None, chain=CHAIN_AUTO,
                       stream=None):
    _qact(xq, xd, cols, n)
    for w, r in zip(ws, rows):
        _mat(w, r, cols)
    _outs(outs, residuals, rows, n)
    res = [None] * len(ws) if residuals is None else residuals
    check(lib().kq4_matmul_multi_q_dev(len(ws), _ptr_array([_tp(o) for o in outs]),
                                       _ptr_array([_tp(r) for r in res]),
                                       _ptr_array([_tp(w) for w in ws]),
                                       (ctypes.c_int * len(rows))(*rows), cols, _tp(xq), _tp(xd),
                                       n, chain, _stream_ptr(stream)), "kq4_matmul_multi_q_dev")


def block_sums_dev(s_lo, s_hi, xq, w, rows, cols, n, stream=None):
    import torch
    _need(xq, "xq", torch.int8, n * cols)
    _mat(w, rows, cols)
    _need(s_lo, "s_lo", torch.int32, n * rows * (cols // 32))
    _need(s_hi, "s_hi", torch.int32, n * rows * (cols // 32))
    check(lib().kq4_block_sums_dev(_tp(s_lo), _tp(s_hi), _tp(xq), _tp(w), rows, cols, n,
                                   _stream_ptr(stream)), "kq4_block_sums_dev")


def moe_route_dev(sel, pr, logits, tk, stream=None):
    import torch
    T, ne = logits.shape
    _need(logits, "logits", torch.float32, T * ne)
    _need(sel, "sel", torch.int32, T * tk)
    _need(pr, "pr", torch.float32, T * tk)
    check(lib().kq4_moe_route_dev(_tp(sel), _tp(pr), _tp(logits), T, ne, tk,
                                  _stream_ptr(stream)), "kq4_moe_route_dev")


def moe_router_logits_dev(logits, router, X, stream=None):
    import torch
    T, d = X.shape
    ne = router.shape[0]
    _act(X, d, "X")
    _need(router, "router", torch.float32, ne * d)
    _need(logits, "logits", torch.float32, T * ne)
    check(lib().kq4_moe_router_logits_dev(_tp(logits), _tp(router), _tp(X), T, ne, d,
                                          _stream_ptr(stream)), "kq4_moe_router_logits_dev")


def _moe_args(Y, X, G, U, D, ne, d, ef):
    import torch
    T = _act(X, d, "X")
    _need(Y, "Y", torch.float32, T * d)
    _mat(G, ne * ef, d)
    _mat(U, ne * ef, d)
    _mat(D, d, ne * ef)
    return T


def moe_layer_dev(Y, X, router, G, U, D, ne, tk, d, ef, sel=None, pr=None, stream=None):
    import torch
    T = _moe_args(Y, X, G, U, D, ne, d, ef)
    _need(router, "router", torch.float32, ne * d)
    _need(sel, "sel", torch.int32, T * tk, optional=True)
    _need(pr, "pr", torch.float32, T * tk, optional=True)
    check(lib().kq4_moe_layer_dev(_tp(Y), _tp(X), _tp(router), _tp(G), _tp(U), _tp(D), T, ne, tk,
                                  d, ef, _tp(sel), _tp(pr), _stream_ptr(stream)),
          "kq4_moe_layer_dev")


def moe_ffn_dev(Y, X, sel, pr, G, U, D, ne, d, ef, stream=None):
    import torch
    T, tk = sel.shape
    if _moe_args(Y, X, G, U, D, ne, d, ef) != T:
        raise KQ4Error("X and sel differ in tokens")
    _need(sel, "sel", torch.int32, T * tk)
    _need(pr, "pr", torch.float32, T * tk)
    check(lib().kq4_moe_ffn_dev(_tp(Y), _tp(X), _tp(sel), _tp(pr), T, tk, _tp(G), _tp(U),
                                _tp(D), ne, d, ef, _stream_ptr(stream)), "kq4_moe_ffn_dev")


def moe_ffn_stages_dev(Y, X, sel, pr, G, U, D, ne, d, ef, gate=None, up=None, av=None,
                       av_in=None, stream=None):
    import torch
    T, tk = sel.shape
    if _moe_args(Y, X, G, U, D, ne, d, ef) != T:
        raise KQ4Error("X and sel differ in tokens")
    _need(sel, "sel", torch.int32, T * tk)
    _need(pr, "pr", torch.float32, T * tk)
    for name, t in (("gate", gate), ("up", up), ("av", av), ("av_in", av_in)):
        _need(t, name, torch.float32, T * tk * ef, optional=True)
    check(lib().kq4_moe_ffn_stages_dev(_tp(Y), _tp(X), _tp(sel), _tp(pr), T, tk, _tp(G), _tp(U),
                                       _tp(D), ne, d, ef, _tp(gate), _tp(up), _tp(av),
                                       _tp(av_in), _stream_ptr(stream)),
          "kq4_moe_ffn_stages_dev")


# ---- VQF files (include/kq4_vqf.h) -------------------------------------------------------------

def vqf_parse_header(buf, file_size):
    """Validates a header + directory held in buf (bytes) for a file of file_size bytes."""
    b = np.frombuffer(buf, np.uint8)
    info = VqfInfo()
    check(lib().kq4_vqf_parse_header(b.ctypes.data, b.size, file_size, ctypes.byref(info)),
          "kq4_vqf_parse_header")
    return info


class Vqf:
    """A mmap'd VQF file (kq4_vqf_open); close() or use as a context manager."""

    def __init__(self, path, verify_checksum=False):
        self._h = _P()
        check(lib().kq4_vqf_open(os.fsencode(path), int(verify_checksum), ctypes.byref(self._h)),
              "kq4_vqf_open")
        self.info = VqfInfo.from_address(lib().kq4_vqf_get_info(self._h))

    def close(self):
        if self._h:
            lib().kq4_vqf_close(self._h)
            self._h = _P()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def entries(self):
        out = []
        for i in range(self.info.n_tensors):
            name = ctypes.create_string_buffer(32)
            qt, r, c = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
            data, nbytes = _P(), _U64()
            check(lib().kq4_vqf_entry(self._h, i, name, ctypes.byref(qt), ctypes.byref(r),
                                      ctypes.byref(c), ctypes.byref(data), ctypes.byref(nbytes)),
                  "kq4_vqf_entry")
            out.append((name.value.decode(), qt.value, r.value, c.value, nbytes.value))
        return out

    def q4_matrix(self, proj, layer):
        """(numpy view of the layer's VQF 4x4 tile bytes, rows, cols)."""
        data, r, c = _P(), _I(), _I()
        check(lib().kq4_vqf_q4_matrix(self._h, proj, layer, ctypes.byref(data), ctypes.byref(r),
                                      ctypes.byref(c)), "kq4_vqf_q4_matrix")
        n = r.value // 4 * (c.value // 32) * 72
        arr = np.ctypeslib.as_array(ctypes.cast(data, ctypes.POINTER(ctypes.c_uint8)), (n,))
        return arr, r.value, c.value

    def q8_matrix(self, proj, layer):
        """(numpy view of the layer's Q8_0 tile bytes, rows, cols, tile rows g)."""
        data, r, c, g = _P(), _I(), _I(), _I()
        check(lib().kq4_vqf_q8_matrix(self._h, proj, layer, ctypes.byref(data), ctypes.byref(r),
                                      ctypes.byref(c), ctypes.byref(g)), "kq4_vqf_q8_matrix")
        n = r.value * (c.value // 32) * 34
        arr = np.ctypeslib.as_array(ctypes.cast(data, ctypes.POINTER(ctypes.c_uint8)), (n,))
        return arr, r.value, c.value, g.value

    def prepare_q8_dev(self, proj, layer, stream=None):
        """The layer's q8 stream-layout device copy (a new uint8 tensor), rows, cols."""
        import torch
        _, r, c, _g = self.q8_matrix(proj, layer)
        dst = torch.empty(q8_stream_bytes(r, c), dtype=torch.uint8, device="cuda")
        check(lib().kq4_vqf_prepare_q8_dev(self._h, proj, layer, _tp(dst), _stream_ptr(stream)),
              "kq4_vqf_prepare_q8_dev")
        return dst, r, c

    def prepare_dev(self, proj, layer, stream=None):
        """The layer's stream-layout device copy (a new uint8 tensor)."""
        import torch
        _, r, c = self.q4_matrix(proj, layer)
        dst = torch.empty(stream_bytes(r, c), dtype=torch.uint8, device="cuda")
        check(lib().kq4_vqf_prepare_dev(self._h, proj, layer, _tp(dst), _stream_ptr(stream)),
              "kq4_vqf_prepare_dev")
        return dst, r, c

    def upload(self, proj, layer):
        """Uploads into the host-pointer API's cache; returns the key (layer << 32 | proj)."""
        key = _U64()
        check(lib().kq4_vqf_upload(self._h, proj, layer, ctypes.byref(key)), "kq4_vqf_upload")
        return key.value
