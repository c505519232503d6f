/* kq4_oracle.h - scalar CPU restatement of kestrel-llm's Q4_0 x int8 matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as
 * the checker or the CPU baseline - never as a product fallback. The product library
 * (libkq4.so) neither links nor loads it.
 *
 * Every function restates one piece of the reference (citations are paths under the
 * kestrel-llm tree). Pinning (how each function is checked beyond "retyping the formula")
 * is listed per function; see tests/test_oracle_*.py for the checks themselves.
 *
 * Conventions (same as the reference op family):
 *   - weights: VQF 4x4 tiles, [rows/4 groups][cols/32 blocks][72 B]
 *   - activations / outputs: fp32 token-major [n_batch][cols] / [n_batch][rows]
 *   - quantized activations: int8 [n_batch][cols] + f32 scales [n_batch][cols/32]
 */
#ifndef KQ4_ORACLE_H
#define KQ4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 accumulation chains of the reference int8 path (see kq4_oracle.c header). */
enum {
    KQO_CHAIN_AUTO = 0,   /* reference dispatch: M<=3 -> CTILE; M>=4 -> ASM on 4*floor(M/4) + CTILE tail */
    KQO_CHAIN_CTILE = 1,  /* V1: lo/hi accumulators, f32 activation scale */
    KQO_CHAIN_GEMV32 = 2, /* V2: single accumulator, f32 activation scale */
    KQO_CHAIN_ASM = 3,    /* V3: single accumulator, activation scale rounded to f16 (RNE) */
    KQO_CHAIN_Q8GEMM = 4  /* Q8_0 batched GEMM: fl(acc + fl(fl(wd * f16r(xd)) * S)) */
};

uint32_t kqo_f16_to_f32_bits(uint16_t h);
float kqo_f16_to_f32(uint16_t h);
uint16_t kqo_f32_to_f16_bits(float x);

/* legacy Q4_0 encoder (18 B blocks) and the legacy -> 4x4 tile repack */
void kqo_f32_to_q4_0(uint8_t *q4_out, const float *f32_in, int n_elements);
int kqo_repack_q4_0_4x4(const uint8_t *legacy, uint8_t *tiles, int rows, int cols);
int kqo_unpack_4x4_to_q4_0(const uint8_t *tiles, uint8_t *legacy, int rows, int cols);
int kqo_tile_weight(const uint8_t *tile, int r, int e);   /* signed nibble value (n-8) */

void kqo_quantize_row_q8_0_act(const float *x, int8_t *q, float *d, int cols);
void kqo_quantize_rows(const float *x, int8_t *q, float *d, int n_batch, int cols);

/* Integer block sums S_lo/S_hi, layout [n_batch][rows][nb] (int32, exact). */
void kqo_block_sums(const uint8_t *w, const int8_t *xq, int rows, int cols, int n_batch,
                    int32_t *s_lo, int32_t *s_hi);

/* Full op: quantize x, then the chain selected by `chain` (KQO_CHAIN_*). residual may be NULL.
 * Returns 0, or -1 on bad shapes. */
int kqo_matmul(float *out, const float *x, const float *residual, const uint8_t *w,
               int rows, int cols, int n_batch, int chain);
/* Same, from already-quantized activations. */
int kqo_matmul_q(float *out, const int8_t *xq, const float *xd, const float *residual,
                 const uint8_t *w, int rows, int cols, int n_batch, int chain);
/* Selected outputs only: out[i] = output (token tok[i], row row[i]) of the full op with
 * n_batch tokens (the chain of a token depends on its index and n_batch). */
int kqo_matmul_q_sample(float *out, const int8_t *xq, const float *xd, const float *residual,
                        const uint8_t *w, int rows, int cols, int n_batch, int chain,
                        const int *tok, const int *row, int n_sample);

/* ---- dense SiLU * up (AArch64 NEON form of vllm_silu_mul_worker) ---- */
float kqo_exp_neon(float x);
float kqo_frecpe(float x);                     /* positive normal x < 2^126, else NaN */
float kqo_silu_mul_neon(float g, float u);
float kqo_fast_silu(float x);
void kqo_silu_mul_rows(float *g, const float *u, long n);   /* in place, n elements */
/* out = [residual +] W . silu_mul(gate, up), both [n_batch][cols]. */
int kqo_matmul_silu(float *out, const float *gate, const float *up, const float *residual,
                    const uint8_t *w, int rows, int cols, int n_batch, int chain);

/* ---- Q8_0 weights: legacy 34-B blocks, tiled 8x8 (272 B) / 4x4 (136 B), matmul chains ---- */
void kqo_f32_to_q8_0(uint8_t *q8_out, const float *f32_in, int n_elements);
int kqo_repack_q8_0_tiled(const uint8_t *legacy, uint8_t *tiles, int g, int rows, int cols);
/* chain: KQO_CHAIN_AUTO (n_batch 1 -> VDOT, >= 2 -> GEMM), KQO_CHAIN_GEMV32 (VDOT),
 * KQO_CHAIN_Q8GEMM (GEMM); g = tile rows (8 or 4) */
int kqo_q8_matmul_q(float *out, const int8_t *xq, const float *xd, const float *residual,
                    const uint8_t *w, int g, int rows, int cols, int n_batch, int chain);
int kqo_q8_matmul(float *out, const float *x, const float *residual, const uint8_t *w, int g,
                  int rows, int cols, int n_batch, int chain);

/* ---- RMSNorm (dyn_rms_norm chunked order / dyn_rms_norm_batch serial order) ---- */
void kqo_rms_norm(float *out, const float *x, const float *w, int n_batch, int d, float eps,
                  int chunked);

/* float64 brute-force sum_b wd*xd*S (error-budget reference, not a chain). */
void kqo_matmul_f64(double *out, const int8_t *xq, const float *xd, const uint8_t *w,
                    int rows, int cols, int n_batch);

/* ---- MoE (int8 track) ---- */
void kqo_moe_route(const float *logits, int ne, int tk, int *sel, float *pr);
void kqo_router_logits(const float *router, const float *x, int ne, int d, float *logits);
float kqo_silu_mul(float g, float u);
/* Expert-grouped MoE FFN for T tokens with given routing. Optional stage outputs
 * (any may be NULL): gate/up [T][tk][ef], av [T][tk][ef], avq [T][tk][ef], avd [T][tk][ef/32],
 * P (unweighted down partials) [T][tk][d]. If av_in != NULL the down stage consumes av_in
 * ([T][tk][ef]) instead of the computed av (stage-wise pinning). */
int kqo_moe_ffn(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                float *gate_o, float *up_o, float *av_o, int8_t *avq_o, float *avd_o,
                float *P_o, const float *av_in);

#ifdef __cplusplus
}
#endif
#endif
