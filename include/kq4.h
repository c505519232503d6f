/* kq4.h - C ABI of libkq4.so, the MI355X (gfx950) Q4_0 x int8 block-quantized matmul.
 *
 * This is the drop-in boundary for kestrel-llm's quantized-matmul op family. The reference
 * runs the op inside src/model/vllm_safetensors.c as `static` C11 functions; its only
 * accelerator boundary is the NPU hook, which returns 1 = executed / 0 = run the CPU path and
 * keys a persistent device weight cache by `wkey = layer<<32 | proj`
 * (st_npu_try_gemm_batched_q4 vllm_safetensors.c:3371-3506, vllm_npu_gemm_gw
 * include/npu/vllm_npu.h:135-159). The host-pointer entry points below follow that contract;
 * the device-pointer entry points are the same ops for callers whose tensors already live in
 * HBM. Plain C types only (no HIP/torch types): a HIP stream is passed as `void *`
 * (NULL = the default stream).
 *
 * Data formats (identical to the reference's):
 *   weights   VQF 4x4 tiles: [rows/4 groups][cols/32 blocks] x 72 B; a tile holds 4 f16 row
 *             scales then 64 nibble bytes, byte 8+16k+4r+i = legacy qs byte 4k+i of row r,
 *             XOR 0x88 (vqf_convert/src/qk_repack.c:19-46, VQF_FLAG_Q4_4X4
 *             include/model/vqf_format.h:32). The host-pointer API takes them as stored. The
 *             device-pointer API takes the device copy kq4_weights_prepare_dev makes of them
 *             once (the "stream layout": the same tiles, regrouped so the GEMV reads each
 *             kernel lane's tiles with full-width coalesced loads), as the reference's NPU path
 *             converts weights once into its device cache (st_npu_gw_build
 *             vllm_safetensors.c:2790-3040).
 *   x / out   fp32 token-major [n_batch][cols] / [n_batch][rows]
 *   residual  fp32 [n_batch][rows]; out = residual + W.x (fused O / down projections)
 * Preconditions (as the reference's 4x4 path): rows % 4 == 0, cols % 32 == 0.
 *
 * Threading: like the reference op (called only from the single inference thread,
 * vllm_safetensors.c:4670-4672), the library keeps one workspace per device; calls that
 * overlap on one device (different host threads or different streams) race on it.
 *
 * HIP graphs: the device-pointer calls may be captured. A captured call keeps the workspace it
 * was recorded with; the library never frees a workspace before kq4_shutdown (growing it
 * allocates a new one and keeps the old one for the graphs that use it), so a graph stays valid
 * whatever calls run after its capture. The workspace cannot grow while a stream is being
 * captured (that needs hipMalloc): such a call returns KQ4_EINVAL and launches nothing. Size it
 * before capturing with kq4_workspace_reserve (kq4_matmul_workspace_bytes,
 * kq4_moe_workspace_bytes), or by running the same calls once eagerly. kq4_workspace_trim frees
 * the outgrown workspaces once the graphs captured before the growth are destroyed. Only the
 * call's own stream is asked whether it is capturing: a call that grows the workspace on
 * another stream while some stream captures in hipStreamCaptureModeGlobal fails in hipMalloc
 * (KQ4_ENOMEM) and invalidates that capture, so reserve first in that mode too.
 *
 * Error convention: device-pointer calls return KQ4_OK (0) or a negative KQ4_E* code;
 * host-pointer drop-in calls return 1 (done on the GPU) or 0 (not done: the caller runs its
 * CPU path). kq4_last_error() describes the last failure of the calling thread.
 */
#ifndef KQ4_H
#define KQ4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KQ4_OK 0
#define KQ4_EINVAL (-1)   /* bad shape / argument */
#define KQ4_EHIP (-2)     /* HIP runtime error */
#define KQ4_ENOMEM (-3)   /* device allocation failed */
#define KQ4_ENODEV (-4)   /* no usable gfx950 device */
#define KQ4_EIO (-5)      /* file cannot be read or fails validation (kq4_vqf.h) */

/* fp32 accumulation chain (how per-block products are summed; integer block sums are the
 * same in all of them). AUTO is the reference's dispatch (q4x4_gemm_batched
 * vllm_safetensors.c:4593-4631): n_batch <= 3 -> CTILE; n_batch > 3 -> ASM on the first
 * n_batch & ~3 tokens and CTILE on the rest.
 * The prefill GEMM (n_batch > 16; option gemv_chunk_max) replays the selected chain per output
 * bit for bit, except where
 * the planner splits K (launches that leave CUs idle: fewer 128x128 tiles than CUs with K >= 256
 * blocks, K >= 128 blocks with fewer 64-token tiles than three per CU, or K of 64-127 blocks
 * with at most one 64x64 tile per two CUs; never the CTILE chain; option gemm_split, 1 keeps
 * every output the single chain): each K slice then runs the chain from zero and the slices' outputs are
 * added in slice order, within 1e-5 of the single chain. The decode
 * GEMV (n_batch <= 8; q4 9..16 in one 16-token launch; and the GEMM's 1..3-token AUTO tail)
 * takes from the chain only its activation
 * scale (f16-rounded for ASM tokens, f32 otherwise): it splits K over waves and sums each
 * wave's terms in block order (one token: a lo and a hi chain per half block, as CTILE; two or
 * more: one term per block, as GEMV32), then adds the waves' sums in a fixed order. So CTILE and
 * GEMV32 run the same GEMV, whose outputs match either reference chain within 1e-5 of the
 * output's magnitude, not bit for bit. */
#define KQ4_CHAIN_AUTO 0
#define KQ4_CHAIN_CTILE 1   /* q4x4_dot1_group16, vllm_safetensors.c:4180-4216 */
#define KQ4_CHAIN_GEMV32 2  /* q4x4_dot1_group16_gemv (M4f), :4229-4251 */
#define KQ4_CHAIN_ASM 3     /* llama 4x4 asm GEMM, f16-rounded activation scale, :4328-4368 */
/* Q8_0 weights (kq4_q8_*): AUTO = 1 token -> GEMV32 (the VDOT chain of q8x8_dot_rows
 * :5178-5225), >= 2 tokens -> Q8GEMM for every token (gemm_q8_0_8x8_neon :4973-5050:
 * acc = fl(acc + fl(fl(wd * f16r(xd)) * S)), unfused). */
#define KQ4_CHAIN_Q8GEMM 4

/* Summation order of an RMSNorm's sum of squares (both are the reference's, one binary32
 * rounding per step): CHUNKED = dyn_rms_norm (vllm_safetensors.c:8811-8827, decode; also the
 * batch worker under VLLM_SPEC_VNORM=1): 8-element chunks, each reduced as
 * ((q0+q4)+(q1+q5))+((q2+q6)+(q3+q7)), summed in order; SERIAL = dyn_rms_norm_batch's default
 * worker (:8849-8867, prefill): the squares summed in order. */
#define KQ4_RMS_CHUNKED 0
#define KQ4_RMS_SERIAL 1

/* Most weight matrices one fused call may take (QKV = 3, gate/up = 2). */
#define KQ4_MAX_MATS 4

/* ---- lifetime ---------------------------------------------------------------------------- */

/* Selects `device` (a gfx950 GPU) for the calling thread and prepares its workspace.
 * Replaces the NPU open/probe step (vllm_npu_available include/npu/vllm_npu.h:88-100). */
int kq4_init(int device);
/* Frees every device buffer the library owns (workspaces, weight cache). */
void kq4_shutdown(void);
const char *kq4_last_error(void);
/* Library version string. */
const char *kq4_version(void);

/* Sets one of the launch planner's options, for measurement and tests (no counterpart in the
 * reference): gemv_kind (0 v_dot4 / 1 MFMA dots), gemv_mfma_from, gemv_hs (0 whole 32-row sets,
 * 1 halves, 2 quarters per workgroup), gemv_rps (row sets per workgroup, 1..3), gemv_waves,
 * gemv_wpcu, gemv_maxw, gemv_fq (0 / 1: activations quantized by a separate launch / in the
 * GEMV), gemv_fq_work, gemv_silu_fq_work, gemv_chunk_max (the largest q4 batch the decode GEMV
 * takes, 9..16 tokens in one launch of its 16-token kernel, 16 by default; 8 or less: every batch beyond 8 tokens
 * on the prefill GEMM; Q8_0 batches beyond 8 tokens always take the GEMM), gemm_kind (0: the prefill GEMM on int8 MFMA, the
 * default; 1: on fp8 operands; the same outputs), gemm_tile (0: the planner's choice; 1 / 2 / 3 /
 * 4: 128x128 / 64x128 / 64x64 / 128x64 token x row tiles; the same outputs), gemm_split (K slices
 * of the int8 GEMM: 0 or 1 none, every output the single chain bit for bit; 2..8 that many;
 * -1 the planner's choice, the default), gemm_prio (the pipelined int8 GEMM's issue priority
 * falling with progress through K, so the workgroups sharing a CU end together: 0 off, 1 on,
 * -1 the planner's choice: on for 128x128 launches of whole rounds of two workgroups per CU and
 * for every 64x128 launch; the same outputs). The initial value
 * of each comes from the environment variable KQ4_ + its upper-case name, else the built-in
 * default (for most, the planner's own choice); value < 0 restores that initial value. Takes
 * effect for launches planned after it returns. */
int kq4_set_option(const char *name, int value);
/* The option's current value in *value (-1: the planner's choice). */
int kq4_get_option(const char *name, int *value);
/* How the current options and planner would run an n_batch-token matmul of rows x cols (q8: Q8_0
 * weights; chain as for kq4_matmul; ncu: the CUs to plan for, 0 = the current device's):
 * *tile = 0 and *ksplit = 0 for the decode GEMV (up to 8 tokens; q4 up to gemv_chunk_max), else the prefill
 * GEMM's tile (1 / 2 / 3 / 4: 128x128 / 64x128 / 64x64 / 128x64 tokens x rows) and its K
 * slices (1 = unsplit: the single chain, bit for bit); the int8 GEMM's plan (the fp8-operand
 * form of gemm_kind 1 picks its tile apart and never splits K). For tests and measurement; no
 * counterpart in the reference. */
int kq4_gemm_plan_info(int n_batch, int rows, int cols, int q8, int chain, int ncu, int *tile,
                       int *ksplit);

/* ---- host-pointer drop-in API (synchronous; 1 = done, 0 = caller falls back) -------------- */

/* Uploads 4x4 q4 weights once and keeps them under `wkey` (layer<<32 | proj), as the NPU
 * weight cache does (st_npu_gw_get/build vllm_safetensors.c:2780-3040). */
int kq4_weights_upload(uint64_t wkey, const uint8_t *w4x4, int rows, int cols);
int kq4_weights_evict(uint64_t wkey);
/* Drops every cached weight matrix of the current device; returns how many were dropped.
 * A cached entry is also re-uploaded when its host bytes no longer match (sampled
 * fingerprint), so a key reused for different weights is never served stale. */
int kq4_weights_clear(void);

/* out = [residual +] W.x for n_batch tokens; replaces q4x4_gemm_batched / dyn_matvec_q4_q8*
 * (vllm_safetensors.c:4593-4631, 6147-6174, 8628-8786) behind st_npu_try_gemm_batched_q4's
 * 1/0 contract (:3371-3506). wkey != 0 uses (or fills) the weight cache; wkey == 0 copies the
 * weights for this call only. */
int kq4_matmul(float *out, const float *x, const float *residual, const uint8_t *w4x4, int rows,
               int cols, int n_batch, int chain, uint64_t wkey);

/* The dense FFN's SiLU-multiply and down projection in one call:
 * out = [residual +] W.silu_mul(gate, up), gate/up [n_batch][cols]. silu_mul is the reference's
 * AArch64 vllm_silu_mul_worker element rule (vllm_safetensors.c:10932-10958: exp_neon4 :4041,
 * FRECPE and two FRECPS Newton steps), bit for bit; it replaces the worker's parfor plus
 * dyn_matvec_q4_q8_fused_down_residual[_batched] (:8663, :8762; dense decode :16756-16767,
 * batched :17232-17247). The product is quantized without being written to memory. */
int kq4_matmul_silu(float *out, const float *gate, const float *up, const float *residual,
                    const uint8_t *w4x4, int rows, int cols, int n_batch, int chain,
                    uint64_t wkey);

/* Up to KQ4_MAX_MATS matrices sharing one activation (fused QKV / gate+up wrappers); wkeys may
 * be NULL (no caching) or hold one key per matrix (0 = no caching for that matrix). */
int kq4_matmul_multi(int n_mats, float *const *out, const float *const *residual,
                     const uint8_t *const *w4x4, const int *rows, int cols, const float *x,
                     int n_batch, int chain, const uint64_t *wkeys);

/* Q8_0 weights (the reference's prefill format of dual VQF files, vllm_safetensors.c:2453-2460,
 * and its q8 mode): tiles of g = 8 rows (block_q8_0x8, 272 B per 8 rows x 32 cols,
 * VQF_FLAG_Q8_8X8, the reference's default) or g = 4 rows (block_q8_0x4, 136 B): g f16 row
 * scales, then qs[k*4g + m*4 + i] = row m's element 4k+i (vqf_convert/src/qk_repack.c:51-103).
 * out = [residual +] W.x with the reference's Q8 chains (KQ4_CHAIN_AUTO / GEMV32 / Q8GEMM).
 * wkey as kq4_matmul (the q8 copy of a key is kept apart from its q4 copy). */
int kq4_q8_matmul(float *out, const float *x, const float *residual, const uint8_t *w_tiles,
                  int g, int rows, int cols, int n_batch, int chain, uint64_t wkey);
int kq4_q8_matmul_multi(int n_mats, float *const *out, const float *const *residual,
                        const uint8_t *const *w_tiles, int g, const int *rows, int cols,
                        const float *x, int n_batch, int chain, const uint64_t *wkeys);

/* MoE FFN of T tokens with top-k routing given as expert ids `sel` [T][tk] and weights `pr`
 * [T][tk]; int8 activation track (VLLM_ACTQ=1) of st_moe_ffn_sparse_q4 / _batch_arm
 * (vllm_safetensors.c:12921-13398, 14894-15064). G/U: [ne*ef rows][d cols], D: [d rows]
 * [ne*ef cols], all 4x4 tiles. wkey != 0 caches G/U/D under wkey, wkey+1, wkey+2. */
int kq4_moe_ffn(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                uint64_t wkey);

/* ---- device-pointer API (stream-ordered, asynchronous) ----------------------------------- */

/* Workspace bytes the device-pointer matmuls (kq4_matmul_dev, _multi_dev, _silu_dev,
 * kq4_rmsnorm_matmul_multi_dev and the q8 twins) need for n_batch tokens of cols columns, and
 * the MoE calls (kq4_moe_ffn_dev, kq4_moe_ffn_stages_dev, kq4_moe_layer_dev) for T tokens; 0 for
 * a bad shape. The workspace is shared: reserve the largest any call will need. Beyond 8 tokens
 * the matmul figure includes up to 24 MiB for the partial sums of a K-split GEMM (the planner's
 * splits never need more; a split forced through gemm_split may). No counterpart in the
 * reference (its scratch grows inside the op, xq_scratch_ensure vllm_safetensors.c:4670-4695);
 * for callers that capture HIP graphs. */
size_t kq4_matmul_workspace_bytes(int n_batch, int cols);
size_t kq4_moe_workspace_bytes(int T, int tk, int ne, int d, int ef);
/* Grows the current device's workspace to at least `bytes` now (not while the calling thread's
 * stream is being captured). */
int kq4_workspace_reserve(size_t bytes);
/* Frees the current device's outgrown workspaces (kept since they grew, for graphs captured
 * before the growth) after waiting for the device to go idle. Call it only once every graph
 * captured before the last growth has been destroyed (a replay would read freed memory), and
 * not while a stream captures. No counterpart in the reference. */
int kq4_workspace_trim(void);

/* Size in bytes of the stream-layout copy of a rows x cols q4 matrix (0 for a bad shape):
 * 9216 B per (32-row set, 16-block stage), rows rounded up to 32, blocks up to 16. */
size_t kq4_weights_stream_bytes(int rows, int cols);

/* Writes the stream-layout copy of the VQF 4x4 matrix w4x4 (device memory, as stored) to dst
 * (device memory, 16-byte aligned, kq4_weights_stream_bytes(rows, cols) bytes; w4x4 8-byte
 * aligned). Stacked
 * matrices of equal shape can be prepared as one matrix of their summed rows when rows % 32 == 0
 * (MoE G/U: ne*ef rows). Replaces the upload/convert step of the NPU weight cache
 * (st_npu_gw_build vllm_safetensors.c:2790-3040). Every `w` / `G` / `U` / `D` of the calls
 * below is such a copy. */
int kq4_weights_prepare_dev(uint8_t *dst, const uint8_t *w4x4, int rows, int cols,
                            void *stream);

/* kq4_weights_prepare_dev from VQF 4x4 tiles in host memory (e.g. the mmap'd VQF file): the
 * tiles are copied to the device and repacked into dst; returns once the host bytes have been
 * read. */
int kq4_weights_prepare_host(uint8_t *dst, const uint8_t *w4x4_host, int rows, int cols,
                             void *stream);

/* Q8_0 weights on the device: the q8 stream layout (8704 B per 32-row set and 8-block stage)
 * made once from the reference's tiles (device or host memory), and the matmuls over it
 * (decode GEMV up to 8 tokens, int8-MFMA GEMM beyond). g = 8 or 4 tile rows, rows % g == 0. */
size_t kq4_q8_weights_stream_bytes(int rows, int cols);
int kq4_q8_weights_prepare_dev(uint8_t *dst, const uint8_t *w_tiles, int g, int rows, int cols,
                               void *stream);
int kq4_q8_weights_prepare_host(uint8_t *dst, const uint8_t *w_tiles_host, int g, int rows,
                                int cols, void *stream);
int kq4_q8_matmul_dev(float *out, const float *x, const float *residual, const uint8_t *w,
                      int rows, int cols, int n_batch, int chain, void *stream);
int kq4_q8_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                            const uint8_t *const *w, const int *rows, int cols, const float *x,
                            int n_batch, int chain, void *stream);

/* Activation quantizer (quantize_row_q8_0_act vllm_safetensors.c:7893-7920) for n_batch rows:
 * xq int8 [n_batch][cols], xd f32 [n_batch][cols/32]. xde (may be NULL) receives the scale
 * each token's chain multiplies by: f32(f16_rne(xd)) for ASM-chain tokens, xd otherwise.
 * Device buffers of this API: x and xq 16-byte aligned (xq 8-byte here), scales 4-byte. */
int kq4_quantize_dev(int8_t *xq, float *xd, float *xde, const float *x, int n_batch, int cols,
                     int chain, void *stream);

/* Quantize x once, then out = [residual +] W.x. */
int kq4_matmul_dev(float *out, const float *x, const float *residual, const uint8_t *w,
                   int rows, int cols, int n_batch, int chain, void *stream);

/* kq4_matmul_dev that allocates nothing, for callers that cannot call hipMalloc (code under HIP
 * graph capture, serving loops and harnesses that forbid allocation). No counterpart in the
 * reference. Same arguments, kernels and results as kq4_matmul_dev; the quantized activations go
 * to a fixed per-device scratch array of KQ4_NOALLOC_SCRATCH_BYTES (held by each GPU the library
 * runs on until the process ends) instead of the growable workspace. Beyond 8 tokens the
 * prefill GEMM's operands, n_batch * cols * 17/8 bytes (rounded up to 256-byte pieces), must
 * fit in it (2048 x 12288 does; the int8 operands and the planner's K-split partial sums then
 * fit too), else KQ4_EINVAL. Every call on a GPU
 * shares that GPU's scratch: calls that overlap on one GPU (other streams or threads) race. */
#define KQ4_NOALLOC_SCRATCH_BYTES (64u << 20)
int kq4_matmul_noalloc_dev(float *out, const float *x, const float *residual, const uint8_t *w,
                           int rows, int cols, int n_batch, int chain, void *stream);

/* kq4_matmul_silu on device buffers (gate, up 16-byte aligned): up to 4 tokens in one launch
 * (the GEMV forms the product while quantizing), else the quantizer forms it. */
int kq4_matmul_silu_dev(float *out, const float *gate, const float *up, const float *residual,
                        const uint8_t *w, int rows, int cols, int n_batch, int chain,
                        void *stream);

/* RMSNorm of n_batch rows of d floats, bit for bit the reference's: out = fl(fl(x*rms)*w),
 * rms = 1/sqrtf(ss/d + eps) with ss in `order` (KQ4_RMS_*). Replaces dyn_rms_norm (:8811) and
 * dyn_rms_norm_batch (:8869). d % 8 == 0, d <= 16384; out, x, w 16-byte aligned; out may be
 * x. */
int kq4_rms_norm_dev(float *out, const float *x, const float *w, int n_batch, int d, float eps,
                     int order, void *stream);

/* RMSNorm and the matmuls it feeds in one call: the layer input x [n_batch][cols] is normalised
 * (norm_w [cols], eps, order as kq4_rms_norm_dev) and quantized in the same pass, then
 * out[i] = [residual[i] +] W[i].normed as kq4_matmul_multi_dev. It replaces the reference's
 * dyn_rms_norm / dyn_rms_norm_batch followed by the QKV or gate/up wrapper (decode
 * :16413-16436 and :16705-16753; prefill :17096-17120 and :17191-17224). normed (may be NULL,
 * 16-byte aligned) receives the fp32 normalised input. */
int kq4_rmsnorm_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                                 const uint8_t *const *w, const int *rows, int cols,
                                 const float *x, const float *norm_w, float eps, int order,
                                 float *normed, int n_batch, int chain, void *stream);

/* vllm_silu_mul_worker over n elements in place (vllm_safetensors.c:10932-10958):
 * gate[i] = silu_mul(gate[i], up[i]) in the NEON form for i < (n & ~3), bit for bit; the last
 * n % 4 elements take the worker's scalar tail fast_silu(g) * u (:3685-3696), here with a
 * correctly rounded exp (the reference's libm expf may differ in the last bit). gate and up
 * 16-byte aligned. */
int kq4_silu_mul_dev(float *gate, const float *up, long n, void *stream);

/* Up to KQ4_MAX_MATS weight matrices sharing one activation (one quantization, one launch):
 * fused QKV (dyn_matvec_q4_q8_fused_qkv_batched :8684) and gate/up (:8738). residual[i] may
 * be NULL. */
int kq4_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                         const uint8_t *const *w, const int *rows, int cols, const float *x,
                         int n_batch, int chain, void *stream);

/* Same op from already-quantized activations (xq/xd as kq4_quantize_dev writes them). */
int kq4_matmul_q_dev(float *out, const int8_t *xq, const float *xd, const float *residual,
                     const uint8_t *w, int rows, int cols, int n_batch, int chain, void *stream);

/* Several matrices from one already-quantized activation: the reference's batched wrappers
 * quantize once and run q/k/v or gate/up from the same xq/xd (:6670-6706, :6846-6870). */
int kq4_matmul_multi_q_dev(int n_mats, float *const *out, const float *const *residual,
                           const uint8_t *const *w, const int *rows, int cols, const int8_t *xq,
                           const float *xd, int n_batch, int chain, void *stream);

/* Debug/verification: the exact integer block sums S_lo / S_hi [n_batch][rows][cols/32]
 * computed by the same device dot-product routine the matmul kernels use. */
int kq4_block_sums_dev(int32_t *s_lo, int32_t *s_hi, const int8_t *xq, const uint8_t *w,
                       int rows, int cols, int n_batch, void *stream);

/* MoE routing on the device: deterministic top-k (ties -> smaller id) + softmax over the k
 * selected (vllm_safetensors.c:12968-12984). logits [T][ne] -> sel [T][tk], pr [T][tk]. */
int kq4_moe_route_dev(int *sel, float *pr, const float *logits, int T, int ne, int tk,
                      void *stream);

/* MoE router logits on the device: logits [T][ne] = router [ne][d] . X [T][d] in fp32, each
 * (token, expert) the reference's serial chain s += rw[i] * x[i], i ascending
 * (st_moe_ffn_sparse_q4 vllm_safetensors.c:12961-12966, batched :14937-14962), bit for bit.
 * d % 32 == 0; router and X 16-byte aligned. */
int kq4_moe_router_logits_dev(float *logits, const float *router, const float *X, int T, int ne,
                              int d, void *stream);

/* A whole MoE FFN layer on the device, as st_moe_ffn_sparse_q4 / _batch_arm run it
 * (:12921-13398, :14894-15064): router logits, top-k + softmax (kq4_moe_route_dev), and the
 * expert FFN (kq4_moe_ffn_dev). sel_out [T][tk] / pr_out [T][tk] receive the routing when not
 * NULL. */
int kq4_moe_layer_dev(float *Y, const float *X, const float *router, const uint8_t *G,
                      const uint8_t *U, const uint8_t *D, int T, int ne, int tk, int d, int ef,
                      int *sel_out, float *pr_out, void *stream);

/* MoE FFN on device buffers (see kq4_moe_ffn); G and U prepared as [ne*ef rows][d cols], D as
 * [d rows][ne*ef cols]. */
int kq4_moe_ffn_dev(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                    const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                    void *stream);

/* Verification variant of kq4_moe_ffn_dev exposing the stages the reference's own A/B checks
 * compare (VLLM_MOE_2B_VERIFY, vllm_safetensors.c:14604-14625): gate_out/up_out/av_out
 * [T*tk][ef] (each may be NULL; gate_out and up_out together), and av_in [T*tk][ef] which, when
 * not NULL, replaces the computed SiLU product as the input of the down projection. */
int kq4_moe_ffn_stages_dev(float *Y, const float *X, const int *sel, const float *pr, int T,
                           int tk, const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne,
                           int d, int ef, float *gate_out, float *up_out, float *av_out,
                           const float *av_in, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KQ4_H */
