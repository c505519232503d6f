/* kq4_ops.h - kestrel-llm's quantized-matmul op family, argument list for argument list, on top
 * of libkq4 (include/kq4.h).
 *
 * Each function mirrors the `static` C11 wrapper of the same name (prefixed kq4_) in
 * src/model/vllm_safetensors.c and computes the same op on the GPU; the only difference is the
 * return value: 1 = done on the GPU, 0 = not done (kq4_last_error() says why) and the caller
 * runs its CPU body, exactly the contract of the reference's NPU hook
 * (st_npu_try_gemm_batched_q4 vllm_safetensors.c:3371-3506). Weight pointers are read-only
 * pointers into the mmap'd VQF (vllm_safetensors.h:215-219); they double as weight-cache keys,
 * so each matrix is uploaded to HBM once. The x8_* arguments are the reference's unused prefill
 * copies and are ignored here as there.
 *
 * Chains: the single-token fused wrappers run the M4f chain (KQ4_CHAIN_GEMV32, their NEON bodies
 * call q4x4_dot1_group16_gemv :6182-6560); the batched wrappers run the reference's batched
 * dispatch (KQ4_CHAIN_AUTO, q4x4_gemm_batched :4593-4631).
 */
#ifndef KQ4_OPS_H
#define KQ4_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dyn_matvec_q4_q8 (vllm_safetensors.c:8628): lm_head-style single-token matvec. */
int kq4_dyn_matvec_q4_q8(float *out, const uint8_t *q4_w, const float *x, int rows, int cols);

/* dyn_matvec_q4_q8_fused_gate_up (:8634) */
int kq4_dyn_matvec_q4_q8_fused_gate_up(float *gate_out, float *up_out, const uint8_t *q4_gate,
                                       const uint8_t *q4_up, const float *x, int rows, int cols);

/* dyn_matvec_q4_q8_fused_qkv (:8643) */
int kq4_dyn_matvec_q4_q8_fused_qkv(float *q_out, float *k_out, float *v_out,
                                   const uint8_t *q4_q, const uint8_t *q4_k, const uint8_t *q4_v,
                                   const float *x, int q_rows, int kv_rows, int cols);

/* dyn_matvec_q4_q8_fused_o_residual (:8653): x = residual + O.attn_in */
int kq4_dyn_matvec_q4_q8_fused_o_residual(float *x, const float *residual, const uint8_t *q4_o,
                                          const float *attn_in, int rows, int cols);

/* dyn_matvec_q4_q8_fused_down_residual (:8663): x = residual + down.activated */
int kq4_dyn_matvec_q4_q8_fused_down_residual(float *x, const float *residual,
                                             const uint8_t *q4_down, const float *activated,
                                             int hidden_dim, int ffn_dim);

/* vllm_silu_mul_worker's parfor (:10932-10958, called over ffn_dim elements at :16735) followed
 * by dyn_matvec_q4_q8_fused_down_residual (:8663): x = residual + down.silu_mul(gate, up). */
int kq4_silu_mul_down_residual(float *x, const float *residual, const uint8_t *q4_down,
                               const float *gate, const float *up, int hidden_dim, int ffn_dim);

/* dyn_matvec_q4_q8_fused_qkv_batched (:8684) */
int kq4_dyn_matvec_q4_q8_fused_qkv_batched(float *q_out, float *k_out, float *v_out,
                                           const uint8_t *q4_q, const uint8_t *q4_k,
                                           const uint8_t *q4_v, const float *x_batch, int q_rows,
                                           int kv_rows, int cols, int n_batch,
                                           const uint8_t *x8_q, const uint8_t *x8_k,
                                           const uint8_t *x8_v);

/* dyn_matvec_q4_q8_fused_o_residual_batched (:8713) */
int kq4_dyn_matvec_q4_q8_fused_o_residual_batched(float *x_batch, const float *residual_batch,
                                                  const uint8_t *q4_o, const float *attn_batch,
                                                  int rows, int cols, int n_batch,
                                                  const uint8_t *x8_o);

/* dyn_matvec_q4_q8_fused_gate_up_batched (:8738) */
int kq4_dyn_matvec_q4_q8_fused_gate_up_batched(float *gate_out, float *up_out,
                                               const uint8_t *q4_gate, const uint8_t *q4_up,
                                               const float *x_batch, int rows, int cols,
                                               int n_batch, const uint8_t *x8_gate,
                                               const uint8_t *x8_up);

/* dyn_matvec_q4_q8_fused_down_residual_batched (:8762) */
int kq4_dyn_matvec_q4_q8_fused_down_residual_batched(float *x_batch, const float *residual_batch,
                                                     const uint8_t *q4_down,
                                                     const float *activated_batch, int hidden_dim,
                                                     int ffn_dim, int n_batch,
                                                     const uint8_t *x8_down);

/* The batched twin: the parfor over n_batch * ffn_dim elements (:17232-17233) followed by
 * dyn_matvec_q4_q8_fused_down_residual_batched (:8762). */
int kq4_silu_mul_down_residual_batched(float *x_batch, const float *residual_batch,
                                       const uint8_t *q4_down, const float *gate_batch,
                                       const float *up_batch, int hidden_dim, int ffn_dim,
                                       int n_batch);

/* ---- Q8_0 op family (dyn_matvec_q8_* vllm_safetensors.c:8509-8610): weights in the tiled
 * Q8_0 layout the reference repacks to - 8x8 (block_q8_0x8) unless VLLM_Q8_8X8=0 or rows % 8 != 0,
 * then 4x4 - as q8x8_enabled / q8_vdot_dispatch choose it (:3971-3979, :5283-5290). */

/* dyn_matvec_q8 (single-token matvec, :1236 / :5400-5440) */
int kq4_dyn_matvec_q8(float *out, const uint8_t *q8_w, const float *x, int rows, int cols);

/* dyn_matvec_q8_fused_qkv_batched (:8509) */
int kq4_dyn_matvec_q8_fused_qkv_batched(float *q_out, float *k_out, float *v_out,
                                        const uint8_t *q8_q, const uint8_t *q8_k,
                                        const uint8_t *q8_v, const float *x_batch, int q_rows,
                                        int kv_rows, int cols, int n_batch);

/* dyn_matvec_q8_fused_o_residual_batched (:8529) */
int kq4_dyn_matvec_q8_fused_o_residual_batched(float *x_batch, const float *residual_batch,
                                               const uint8_t *q8_o, const float *attn_batch,
                                               int rows, int cols, int n_batch);

/* dyn_matvec_q8_fused_gate_up_batched (:8547) */
int kq4_dyn_matvec_q8_fused_gate_up_batched(float *gate_out, float *up_out,
                                            const uint8_t *q8_gate, const uint8_t *q8_up,
                                            const float *x_batch, int rows, int cols,
                                            int n_batch);

/* dyn_matvec_q8_fused_down_residual_batched (:8563) */
int kq4_dyn_matvec_q8_fused_down_residual_batched(float *x_batch, const float *residual_batch,
                                                  const uint8_t *q8_down,
                                                  const float *activated_batch, int hidden_dim,
                                                  int ffn_dim, int n_batch);

/* dyn_matvec_q8_fused_o_residual (:8583) and _down_residual (:8595), single token */
int kq4_dyn_matvec_q8_fused_o_residual(float *x, const float *residual, const uint8_t *q8_o,
                                       const float *attn_in, int rows, int cols);
int kq4_dyn_matvec_q8_fused_down_residual(float *x, const float *residual,
                                          const uint8_t *q8_down, const float *activated,
                                          int hidden_dim, int ffn_dim);

/* One MoE layer as st_moe_ffn_sparse_q4 reads it from STModelWeights (:12937-12952): fp32 router
 * [ne][d], q4 4x4 G/U [ne*ef][d] and D [d][ne*ef]. */
typedef struct {
    const float *router;
    const uint8_t *G, *U, *D;
    int n_experts, top_k, dim, ef;
} kq4_moe_layer;

/* st_moe_ffn_sparse_q4 (:12921), int8 track: router logits and top-k/softmax on the host in the
 * reference's order (:12959-12985), expert FFN on the GPU. */
int kq4_st_moe_ffn_sparse_q4(const kq4_moe_layer *w, const float *x_ffn, float *y);

/* st_moe_ffn_sparse_q4_batch[_arm] (:14426/:14894): nb tokens at once; returns 1 handled /
 * 0 not handled (the reference then falls back to per-token calls). */
int kq4_st_moe_ffn_sparse_q4_batch(const kq4_moe_layer *w, int nb, const float *X, float *Y);

#ifdef __cplusplus
}
#endif
#endif /* KQ4_OPS_H */
