/* kq4_ops.c - C11 host side: kestrel-llm's quantized-matmul op family on top of libkq4.
 * See include/kq4_ops.h for the contract; each wrapper cites the reference function it mirrors. */
#include "kq4_ops.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "kq4.h"

static uint64_t key_of(const void *p) { return (uint64_t)(uintptr_t)p; }

int kq4_dyn_matvec_q4_q8(float *out, const uint8_t *q4_w, const float *x, int rows, int cols) {
    return kq4_matmul(out, x, NULL, q4_w, rows, cols, 1, KQ4_CHAIN_GEMV32, key_of(q4_w));
}

int kq4_dyn_matvec_q4_q8_fused_gate_up(float *gate_out, float *up_out, const uint8_t *q4_gate,
                                       const uint8_t *q4_up, const float *x, int rows, int cols) {
    float *out[2] = {gate_out, up_out};
    const uint8_t *w[2] = {q4_gate, q4_up};
    const int r[2] = {rows, rows};
    const uint64_t k[2] = {key_of(q4_gate), key_of(q4_up)};
    return kq4_matmul_multi(2, out, NULL, w, r, cols, x, 1, KQ4_CHAIN_GEMV32, k);
}

int kq4_dyn_matvec_q4_q8_fused_qkv(float *q_out, float *k_out, float *v_out,
                                   const uint8_t *q4_q, const uint8_t *q4_k, const uint8_t *q4_v,
                                   const float *x, int q_rows, int kv_rows, int cols) {
    float *out[3] = {q_out, k_out, v_out};
    const uint8_t *w[3] = {q4_q, q4_k, q4_v};
    const int r[3] = {q_rows, kv_rows, kv_rows};
    const uint64_t k[3] = {key_of(q4_q), key_of(q4_k), key_of(q4_v)};
    return kq4_matmul_multi(3, out, NULL, w, r, cols, x, 1, KQ4_CHAIN_GEMV32, k);
}

int kq4_dyn_matvec_q4_q8_fused_o_residual(float *x, const float *residual, const uint8_t *q4_o,
                                          const float *attn_in, int rows, int cols) {
    return kq4_matmul(x, attn_in, residual, q4_o, rows, cols, 1, KQ4_CHAIN_GEMV32, key_of(q4_o));
}

int kq4_dyn_matvec_q4_q8_fused_down_residual(float *x, const float *residual,
                                             const uint8_t *q4_down, const float *activated,
                                             int hidden_dim, int ffn_dim) {
    return kq4_matmul(x, activated, residual, q4_down, hidden_dim, ffn_dim, 1, KQ4_CHAIN_GEMV32,
                      key_of(q4_down));
}

int kq4_silu_mul_down_residual(float *x, const float *residual, const uint8_t *q4_down,
                               const float *gate, const float *up, int hidden_dim, int ffn_dim) {
    /* the dense decode path follows the worker with the batched down wrapper at n_batch = 1
     * (:16761), whose dispatch gives the C-tile chain */
    return kq4_matmul_silu(x, gate, up, residual, q4_down, hidden_dim, ffn_dim, 1,
                           KQ4_CHAIN_AUTO, key_of(q4_down));
}

int kq4_silu_mul_down_residual_batched(float *x_batch, const float *residual_batch,
                                       const uint8_t *q4_down, const float *gate_batch,
                                       const float *up_batch, int hidden_dim, int ffn_dim,
                                       int n_batch) {
    return kq4_matmul_silu(x_batch, gate_batch, up_batch, residual_batch, q4_down, hidden_dim,
                           ffn_dim, n_batch, KQ4_CHAIN_AUTO, key_of(q4_down));
}

/* Tile rows of the reference's Q8_0 repack for a matrix of `rows` rows (q8_8x8_enabled
 * vllm_safetensors.c:3971-3979 and the rows % 8 gate of q8_vdot_dispatch :5283-5290). */
static int q8_tile_rows(int rows) {
    const char *e = getenv("VLLM_Q8_8X8");
    const int on = !(e && e[0] == '0');
    return (on && rows % 8 == 0) ? 8 : 4;
}

int kq4_dyn_matvec_q8(float *out, const uint8_t *q8_w, const float *x, int rows, int cols) {
    return kq4_q8_matmul(out, x, NULL, q8_w, q8_tile_rows(rows), rows, cols, 1, KQ4_CHAIN_AUTO,
                         key_of(q8_w));
}

int kq4_dyn_matvec_q8_fused_qkv_batched(float *q_out, float *k_out, float *v_out,
                                        const uint8_t *q8_q, const uint8_t *q8_k,
                                        const uint8_t *q8_v, const float *x_batch, int q_rows,
                                        int kv_rows, int cols, int n_batch) {
    /* one tile layout per call: the q and kv matrices share it when both row counts allow */
    const int g = (q8_tile_rows(q_rows) == 8 && q8_tile_rows(kv_rows) == 8) ? 8 : 4;
    float *out[3] = {q_out, k_out, v_out};
    const uint8_t *w[3] = {q8_q, q8_k, q8_v};
    const int r[3] = {q_rows, kv_rows, kv_rows};
    const uint64_t k[3] = {key_of(q8_q), key_of(q8_k), key_of(q8_v)};
    return kq4_q8_matmul_multi(3, out, NULL, w, g, r, cols, x_batch, n_batch, KQ4_CHAIN_AUTO, k);
}

int kq4_dyn_matvec_q8_fused_o_residual_batched(float *x_batch, const float *residual_batch,
                                               const uint8_t *q8_o, const float *attn_batch,
                                               int rows, int cols, int n_batch) {
    return kq4_q8_matmul(x_batch, attn_batch, residual_batch, q8_o, q8_tile_rows(rows), rows,
                         cols, n_batch, KQ4_CHAIN_AUTO, key_of(q8_o));
}

int kq4_dyn_matvec_q8_fused_gate_up_batched(float *gate_out, float *up_out,
                                            const uint8_t *q8_gate, const uint8_t *q8_up,
                                            const float *x_batch, int rows, int cols,
                                            int n_batch) {
    float *out[2] = {gate_out, up_out};
    const uint8_t *w[2] = {q8_gate, q8_up};
    const int r[2] = {rows, rows};
    const uint64_t k[2] = {key_of(q8_gate), key_of(q8_up)};
    return kq4_q8_matmul_multi(2, out, NULL, w, q8_tile_rows(rows), r, cols, x_batch, n_batch,
                               KQ4_CHAIN_AUTO, k);
}

int kq4_dyn_matvec_q8_fused_down_residual_batched(float *x_batch, const float *residual_batch,
                                                  const uint8_t *q8_down,
                                                  const float *activated_batch, int hidden_dim,
                                                  int ffn_dim, int n_batch) {
    return kq4_q8_matmul(x_batch, activated_batch, residual_batch, q8_down,
                         q8_tile_rows(hidden_dim), hidden_dim, ffn_dim, n_batch, KQ4_CHAIN_AUTO,
                         key_of(q8_down));
}

int kq4_dyn_matvec_q8_fused_o_residual(float *x, const float *residual, const uint8_t *q8_o,
                                       const float *attn_in, int rows, int cols) {
    return kq4_dyn_matvec_q8_fused_o_residual_batched(x, residual, q8_o, attn_in, rows, cols, 1);
}

int kq4_dyn_matvec_q8_fused_down_residual(float *x, const float *residual,
                                          const uint8_t *q8_down, const float *activated,
                                          int hidden_dim, int ffn_dim) {
    return kq4_dyn_matvec_q8_fused_down_residual_batched(x, residual, q8_down, activated,
                                                         hidden_dim, ffn_dim, 1);
}

int kq4_dyn_matvec_q4_q8_fused_qkv_batched(float *q_out, float *k_out, float *v_out,
                                           const uint8_t *q4_q, const uint8_t *q4_k,
                                           const uint8_t *q4_v, const float *x_batch, int q_rows,
                                           int kv_rows, int cols, int n_batch,
                                           const uint8_t *x8_q, const uint8_t *x8_k,
                                           const uint8_t *x8_v) {
    (void)x8_q; (void)x8_k; (void)x8_v;
    float *out[3] = {q_out, k_out, v_out};
    const uint8_t *w[3] = {q4_q, q4_k, q4_v};
    const int r[3] = {q_rows, kv_rows, kv_rows};
    const uint64_t k[3] = {key_of(q4_q), key_of(q4_k), key_of(q4_v)};
    return kq4_matmul_multi(3, out, NULL, w, r, cols, x_batch, n_batch, KQ4_CHAIN_AUTO, k);
}

int kq4_dyn_matvec_q4_q8_fused_o_residual_batched(float *x_batch, const float *residual_batch,
                                                  const uint8_t *q4_o, const float *attn_batch,
                                                  int rows, int cols, int n_batch,
                                                  const uint8_t *x8_o) {
    (void)x8_o;
    return kq4_matmul(x_batch, attn_batch, residual_batch, q4_o, rows, cols, n_batch,
                      KQ4_CHAIN_AUTO, key_of(q4_o));
}

int kq4_dyn_matvec_q4_q8_fused_gate_up_batched(float *gate_out, float *up_out,
                                               const uint8_t *q4_gate, const uint8_t *q4_up,
                                               const float *x_batch, int rows, int cols,
                                               int n_batch, const uint8_t *x8_gate,
                                               const uint8_t *x8_up) {
    (void)x8_gate; (void)x8_up;
    float *out[2] = {gate_out, up_out};
    const uint8_t *w[2] = {q4_gate, q4_up};
    const int r[2] = {rows, rows};
    const uint64_t k[2] = {key_of(q4_gate), key_of(q4_up)};
    return kq4_matmul_multi(2, out, NULL, w, r, cols, x_batch, n_batch, KQ4_CHAIN_AUTO, k);
}

int kq4_dyn_matvec_q4_q8_fused_down_residual_batched(float *x_batch, const float *residual_batch,
                                                     const uint8_t *q4_down,
                                                     const float *activated_batch, int hidden_dim,
                                                     int ffn_dim, int n_batch,
                                                     const uint8_t *x8_down) {
    (void)x8_down;
    return kq4_matmul(x_batch, activated_batch, residual_batch, q4_down, hidden_dim, ffn_dim,
                      n_batch, KQ4_CHAIN_AUTO, key_of(q4_down));
}

/* Router logits (serial fp32 dot, i ascending) and deterministic top-k + softmax over the k
 * selected, as st_moe_ffn_sparse_q4 computes them on the host (vllm_safetensors.c:12959-12985;
 * batched router :14931-14989 computes the same per-token values). */
static int route_token(const kq4_moe_layer *w, const float *x, int *sel, float *pr) {
    const int ne = w->n_experts, tk = w->top_k, d = w->dim;
    float sv[64];
    if (tk < 1 || tk > 64) return 0;
    for (int k = 0; k < tk; k++) { sel[k] = -1; sv[k] = -INFINITY; }
    for (int e = 0; e < ne; e++) {
        const float *rw = w->router + (size_t)e * d;
        float s = 0.0f;
        for (int i = 0; i < d; i++) s += rw[i] * x[i];
        for (int k = 0; k < tk; k++) {
            if (s > sv[k] || (s == sv[k] && (sel[k] < 0 || e < sel[k]))) {
                for (int j = tk - 1; j > k; j--) { sel[j] = sel[j - 1]; sv[j] = sv[j - 1]; }
                sel[k] = e;
                sv[k] = s;
                break;
            }
        }
    }
    float mx = -INFINITY;
    for (int k = 0; k < tk; k++) if (sv[k] > mx) mx = sv[k];
    float sum = 0.0f;
    for (int k = 0; k < tk; k++) { pr[k] = expf(sv[k] - mx); sum += pr[k]; }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int k = 0; k < tk; k++) pr[k] *= inv;
    return 1;
}

int kq4_st_moe_ffn_sparse_q4_batch(const kq4_moe_layer *w, int nb, const float *X, float *Y) {
    if (!w || !X || !Y || nb < 1 || w->top_k < 1 || w->top_k > 32) return 0;
    const int tk = w->top_k, d = w->dim;
    int *sel = (int *)malloc((size_t)nb * tk * sizeof(int));
    float *pr = (float *)malloc((size_t)nb * tk * sizeof(float));
    int ok = sel && pr;
    for (int t = 0; ok && t < nb; t++)
        ok = route_token(w, X + (size_t)t * d, sel + (size_t)t * tk, pr + (size_t)t * tk);
    if (ok)
        ok = kq4_moe_ffn(Y, X, sel, pr, nb, tk, w->G, w->U, w->D, w->n_experts, d, w->ef,
                         key_of(w->G));
    free(sel);
    free(pr);
    return ok;
}

int kq4_st_moe_ffn_sparse_q4(const kq4_moe_layer *w, const float *x_ffn, float *y) {
    return kq4_st_moe_ffn_sparse_q4_batch(w, 1, x_ffn, y);
}
