/* ref_harness.c - reaches the reference's own x86-64 code from /root/reference so tests can
 * pin the oracle against it and bench.py can time it as the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target `ref`) into oracle/_ref/ from the
 * reference sources where they lie; nothing here is copied into this repository and nothing
 * in the product links it.
 *
 * Like the reference's own probe tools/bench/attn_pv_probe.c:2, this file #includes
 * src/model/vllm_safetensors.c so the `static` kernels become callable. Only the x86-64 build
 * of that file is possible here (no aarch64 toolchain), so:
 *   - quantize_row_q8_0_act, f16_to_f32_bits, f32_to_f16_bits are the same scalar code the
 *     NEON build restates bit-for-bit (vllm_safetensors.c:7893-7920 comment);
 *   - the MoE int8 track (VLLM_ACTQ=1, VLLM_ACTQ16=0) is the x86 twin of the ARM int8 track
 *     (same integer sums and fp32 chain: :11279-11299 vs :11861-11924);
 *   - the dense wrappers run the x86 arithmetic (fp32 / int16 activations) and are used only
 *     as the CPU timing baseline, never as a parity reference.
 */
#include "vllm_safetensors.c"

/* src/main.c:504 defines this global; main.c itself is not part of the harness build. */
int g_bench_seqlen = 0;

/* vqf_convert/src/quant_kernels.c and qk_repack.c (linked from their own objects). */
void f32_to_q4_0(uint8_t *q4_out, const float *f32_in, int n_elements);
int repack_q4_0_4x4_inplace(uint8_t *buf, int rows, int cols);

int kref_init(int threads) {
    g_st_q4_repack = 1;   /* VQF files carry VQF_FLAG_Q4_4X4 (vqf.c:386-399) */
    return vllm_tp_init(threads);
}

uint32_t kref_f16_to_f32_bits(uint16_t h) { return f16_to_f32_bits(h); }
uint16_t kref_f32_to_f16_bits(float x) { return f32_to_f16_bits(x); }
float kref_vq_f16(uint16_t h) { return vq_f16(h); }

void kref_quantize_row(const float *x, int8_t *q, float *d, int cols) {
    quantize_row_q8_0_act(x, q, d, cols);
}

void kref_f32_to_q4_0(uint8_t *out, const float *in, int n) { f32_to_q4_0(out, in, n); }
int kref_repack_q4_0_4x4(uint8_t *buf, int rows, int cols) {
    return repack_q4_0_4x4_inplace(buf, rows, cols);
}

/* Builds a one-layer MoE STModelWeights around caller buffers and runs the reference MoE FFN.
 * T == 1 -> st_moe_ffn_sparse_q4 (router included); T >= 2 -> st_moe_ffn_sparse_q4_batch. */
int kref_moe_ffn(float *Y, const float *X, int T, const float *router, const uint8_t *G,
                 const uint8_t *U, const uint8_t *D, int ne, int tk, int d, int ef) {
    static STModelWeights w;
    memset(&w, 0, sizeof(w));
    w.cfg.dim = d;
    w.cfg.ffn_dim = ne * ef;
    w.cfg.n_experts = ne;
    w.cfg.top_k = tk;
    w.cfg.is_moe = 1;
    w.cfg.n_layers = 1;
    w.n_layers_allocated = 1;
    w.moe_router = (float *)router;
    w.q4_gate_weight = (uint8_t *)G;
    w.q4_up_weight = (uint8_t *)U;
    w.q4_down_weight = (uint8_t *)D;
    if (T == 1) {
        st_moe_ffn_sparse_q4(&w, 0, X, Y);
        return 1;
    }
    return st_moe_ffn_sparse_q4_batch(&w, 0, T, X, Y);
}

/* Dense op wrappers (x86 arithmetic; CPU baseline only). */
void kref_gate_up_batched(float *gate, float *up, const uint8_t *wg, const uint8_t *wu,
                          const float *x, int rows, int cols, int n_batch) {
    dyn_matvec_q4_q8_fused_gate_up_batched(gate, up, wg, wu, x, rows, cols, n_batch, NULL, NULL);
}
void kref_qkv_batched(float *q, float *k, float *v, const uint8_t *wq, const uint8_t *wk,
                      const uint8_t *wv, const float *x, int q_rows, int kv_rows, int cols,
                      int n_batch) {
    dyn_matvec_q4_q8_fused_qkv_batched(q, k, v, wq, wk, wv, x, q_rows, kv_rows, cols, n_batch,
                                       NULL, NULL, NULL);
}
void kref_o_residual_batched(float *x, const float *res, const uint8_t *wo, const float *attn,
                             int rows, int cols, int n_batch) {
    dyn_matvec_q4_q8_fused_o_residual_batched(x, res, wo, attn, rows, cols, n_batch, NULL);
}
void kref_down_residual_batched(float *x, const float *res, const uint8_t *wd, const float *act,
                                int hidden, int ffn, int n_batch) {
    dyn_matvec_q4_q8_fused_down_residual_batched(x, res, wd, act, hidden, ffn, n_batch, NULL);
}
/* q4g_gemm_mat (vllm_safetensors.c:1130-1187): the x86 q4 GEMM over int16 activations that the
 * batched wrappers take for n_batch > 1 (:1583-1588, :1699-1702, :1649, :1754); 0 = done. */
int kref_gemm_mat(float *out, const float *resid, const uint8_t *w, const float *x, int rows,
                  int cols, int nb) {
    return q4g_gemm_mat(out, resid, w, x, rows, cols, nb);
}
/* The reference's logical-CPU count (include/common/vllm_platform.h:354-357) and its pool size. */
long kref_num_cpus(void) { return st_num_cpus(); }
int kref_threads(void) { return vllm_tp_threads(); }
void kref_matvec(float *out, const uint8_t *w, const float *x, int rows, int cols) {
    dyn_matvec_q4_q8(out, w, x, rows, cols);
}

/* The reference's SiLU-multiply over n elements in place, run as its callers run it
 * (vllm_tp_parfor over 16-element tasks, :16735 / :17233). On x86-64 the worker takes its
 * non-NEON body, fast_silu(g) * u with this host's expf (:10955-10957). */
void kref_silu_mul(float *g, const float *u, int n) {
    vllm_silu_mul_ctx c = {g, (float *)u, n};
    vllm_tp_parfor(0, (n + 15) / 16, vllm_silu_mul_worker, &c);
}

/* The reference's RMSNorms: single-token dyn_rms_norm (chunked sum of squares, :8811-8827)
 * and the batched dyn_rms_norm_batch (per-token worker, serial sum unless VLLM_SPEC_VNORM=1,
 * :8849-8873). */
void kref_rms_norm(float *out, const float *x, const float *w, int d, float eps) {
    dyn_rms_norm(out, x, w, d, eps);
}
void kref_rms_norm_batch(float *out, const float *x, const float *w, int nb, int d, float eps) {
    dyn_rms_norm_batch(out, x, w, nb, d, eps);
}

/* The reference converter's Q8_0 encoder and tile repacks (vqf_convert/src/quant_kernels.c:64,
 * qk_repack.c:51, :78; linked from their own objects). */
void f32_to_q8_0(uint8_t *q8_out, const float *f32_in, int n_elements);
int repack_q8_0_8x8_inplace(uint8_t *buf, int rows, int cols);
int repack_q8_0_4x4_inplace(uint8_t *buf, int rows, int cols);
void kref_f32_to_q8_0(uint8_t *out, const float *in, int n) { f32_to_q8_0(out, in, n); }
int kref_repack_q8_0_8x8(uint8_t *buf, int rows, int cols) {
    return repack_q8_0_8x8_inplace(buf, rows, cols);
}
int kref_repack_q8_0_4x4(uint8_t *buf, int rows, int cols) {
    return repack_q8_0_4x4_inplace(buf, rows, cols);
}
