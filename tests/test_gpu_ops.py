"""The C11 op wrappers (include/kq4_ops.h, reference argument lists) and the host-pointer
drop-in API on the GPU, against the oracle."""
import ctypes

import numpy as np
import pytest

import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
P = lambda a: a.ctypes.data  # noqa: E731


@pytest.fixture(autouse=True)
def fresh_cache(kq4):
    """The wrappers key cached weights by host pointer (the reference's weights are an mmap
    that lives as long as the process); test arrays do not, so drop the cache per test."""
    yield
    kq4.lib().kq4_weights_clear()


def test_reused_key_is_not_served_stale(kq4, orc):
    rows, cols = 32, 256
    w1 = synth.make_q4_weights(rows, cols, 61)
    w2 = synth.make_q4_weights(rows, cols, 62)
    x = synth.make_activations(1, cols, 63)
    a = kq4.matmul(w1, x, rows, cols, wkey=77)
    b = kq4.matmul(w2, x, rows, cols, wkey=77)     # same key, same size, different bytes
    assert rel_err(a, orc.matmul(w1, x, rows, cols))[0] <= TOL
    assert rel_err(b, orc.matmul(w2, x, rows, cols))[0] <= TOL


def test_weight_cache_and_host_api(kq4, orc):
    rows, cols, n = 64, 512, 3
    w = synth.make_q4_weights(rows, cols, 1)
    x = synth.make_activations(n, cols, 2)
    want = orc.matmul(w, x, rows, cols)
    assert kq4.lib().kq4_weights_upload(1234, P(w), rows, cols) == 1
    got = kq4.matmul(w, x, rows, cols, wkey=1234)
    assert rel_err(got, want)[0] <= TOL
    assert kq4.lib().kq4_weights_evict(1234) == 1
    assert kq4.lib().kq4_weights_evict(1234) == 0
    # bad shape -> 0 (caller falls back), with a message
    assert kq4.lib().kq4_matmul(P(got), P(x), None, P(w), 6, cols, n, 0, 0) == 0
    assert "rows" in kq4.last_error()


@pytest.mark.parametrize("n", [1, 4, 13])
def test_batched_wrappers(kq4, orc, n):
    lib = kq4.lib()
    cfg = synth.QWEN3VL_2B
    h, ffn = cfg["hidden"], 512
    qr, kvr = 256, 128
    wq, wk, wv = (synth.make_q4_weights(r, h, 10 + i) for i, r in enumerate((qr, kvr, kvr)))
    wg, wu = synth.make_q4_weights(ffn, h, 20), synth.make_q4_weights(ffn, h, 21)
    wo = synth.make_q4_weights(h, qr, 22)
    wd = synth.make_q4_weights(h, ffn, 23)
    x = synth.make_activations(n, h, 30)
    attn = synth.make_activations(n, qr, 31)
    act = synth.make_activations(n, ffn, 32)
    res = synth.make_activations(n, h, 33)

    q, k, v = (np.empty((n, r), np.float32) for r in (qr, kvr, kvr))
    assert lib.kq4_dyn_matvec_q4_q8_fused_qkv_batched(P(q), P(k), P(v), P(wq), P(wk), P(wv),
                                                      P(x), qr, kvr, h, n, None, None, None) == 1
    for got, w, r in ((q, wq, qr), (k, wk, kvr), (v, wv, kvr)):
        assert rel_err(got, orc.matmul(w, x, r, h))[0] <= TOL

    g, u = np.empty((n, ffn), np.float32), np.empty((n, ffn), np.float32)
    assert lib.kq4_dyn_matvec_q4_q8_fused_gate_up_batched(P(g), P(u), P(wg), P(wu), P(x), ffn, h,
                                                          n, None, None) == 1
    assert rel_err(g, orc.matmul(wg, x, ffn, h))[0] <= TOL
    assert rel_err(u, orc.matmul(wu, x, ffn, h))[0] <= TOL

    o = np.empty((n, h), np.float32)
    assert lib.kq4_dyn_matvec_q4_q8_fused_o_residual_batched(P(o), P(res), P(wo), P(attn), h, qr,
                                                             n, None) == 1
    assert rel_err(o, orc.matmul(wo, attn, h, qr, residual=res))[0] <= TOL

    dn = np.empty((n, h), np.float32)
    assert lib.kq4_dyn_matvec_q4_q8_fused_down_residual_batched(P(dn), P(res), P(wd), P(act), h,
                                                                ffn, n, None) == 1
    assert rel_err(dn, orc.matmul(wd, act, h, ffn, residual=res))[0] <= TOL


def test_single_token_wrappers_within_tolerance_of_m4f_chain(kq4, orc):
    """The single-token wrappers request the M4f chain (their NEON bodies call
    q4x4_dot1_group16_gemv, vllm_safetensors.c:6182-6560); the GEMV takes from it only the f32
    activation scale and sums in its own K split, so the bar is 1e-5, not bit identity."""
    lib = kq4.lib()
    rows, cols = 128, 1024
    w = synth.make_q4_weights(rows, cols, 40)
    w2 = synth.make_q4_weights(rows, cols, 41)
    x = synth.make_activations(1, cols, 42)
    res = synth.make_activations(1, rows, 43)
    out = np.empty(rows, np.float32)
    assert lib.kq4_dyn_matvec_q4_q8(P(out), P(w), P(x), rows, cols) == 1
    assert rel_err(out, orc.matmul(w, x, rows, cols, chain=2)[0])[0] <= TOL
    g, u = np.empty(rows, np.float32), np.empty(rows, np.float32)
    assert lib.kq4_dyn_matvec_q4_q8_fused_gate_up(P(g), P(u), P(w), P(w2), P(x), rows, cols) == 1
    assert rel_err(u, orc.matmul(w2, x, rows, cols, chain=2)[0])[0] <= TOL
    assert lib.kq4_dyn_matvec_q4_q8_fused_o_residual(P(out), P(res), P(w), P(x), rows, cols) == 1
    assert rel_err(out, orc.matmul(w, x, rows, cols, residual=res, chain=2)[0])[0] <= TOL


def test_moe_wrapper_routes_like_reference(kq4, orc):
    cfg = dict(hidden=256, experts=16, top_k=4, ef=64)
    d, ne, tk, ef = 256, 16, 4, 64
    G, U, D = synth.make_moe(cfg, 50)
    router = (np.random.default_rng(51).standard_normal((ne, d)) * 0.1).astype(np.float32)
    X = synth.make_activations(5, d, 52)
    layer = kq4.MoeLayer(router.ctypes.data, G.ctypes.data, U.ctypes.data, D.ctypes.data, ne, tk,
                         d, ef)
    Y = np.empty((5, d), np.float32)
    assert kq4.lib().kq4_st_moe_ffn_sparse_q4_batch(ctypes.byref(layer), 5, P(X), P(Y)) == 1
    sel, pr = orc.moe_route(orc.router_logits(router, X, ne, d), tk)
    Y_o = orc.moe_ffn(X, sel, pr, G, U, D, ne, d, ef)
    assert rel_err(Y, Y_o)[0] <= 1e-5
    y1 = np.empty(d, np.float32)
    x0 = np.ascontiguousarray(X[0])
    assert kq4.lib().kq4_st_moe_ffn_sparse_q4(ctypes.byref(layer), P(x0), P(y1)) == 1
    assert rel_err(y1, Y_o[0])[0] <= 1e-5
