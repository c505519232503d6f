// kq4_internal.h - launch interfaces shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

// Raises kernel fn's dynamic LDS limit to `bytes` on the current device once per (kernel,
// device): `done`, one per kernel, holds a bit per device id below 64 (devices beyond make the
// call every time). Thread-safe: threads that race both make the idempotent call.
inline hipError_t kq4_lds_limit_once(const void *fn, int bytes,
                                     std::atomic<unsigned long long> &done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const unsigned long long bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

#define KQ4_GEMV_MAX_M 8
#define KQ4_GEMV_WIDE_M 16   // q4 batches of 9-16 tokens: one launch of the 16-token kernel
#define KQ4_MAXMAT 4

// Every kernel reads q4 weights in the stream layout (kq4_common.h): a VQF 4x4 matrix repacked
// once by kq4_launch_repack into kq4_stream_bytes(rows, cols) bytes.
size_t kq4_stream_bytes(int rows, int cols);
int kq4_launch_repack(uint8_t *dst, const uint8_t *src, int rows, int cols, hipStream_t stream);
// Q8_0 weights: the reference's tiles (g = 8 rows: block_q8_0x8, 4: block_q8_0x4) repacked into
// the q8 stream layout (kq4_common.h), kq8_stream_bytes(rows, cols) bytes.
size_t kq8_stream_bytes(int rows, int cols);
int kq8_launch_repack(uint8_t *dst, const uint8_t *src, int g, int rows, int cols,
                      hipStream_t stream);

// One weight matrix of a (possibly fused) GEMV launch. All matrices share the activation.
struct KQ4GemvMat {
  const uint8_t *w;     // stream layout
  float *out;           // [M][rows]
  const float *res;     // [M][rows] or nullptr
  int rows;
  int wg_begin;         // first group (R row sets, or a half / quarter set) of this matrix
};

struct KQ4GemvArgs {
  KQ4GemvMat mat[KQ4_MAXMAT];
  int nmat;
  const float *xf;      // fp32 activations [M][cols] when the kernel quantizes them itself
  const float *xu;      // with xf: the dense FFN's up output; the activation is silu_mul(xf, xu)
  const int8_t *xq;     // [M][cols] (pre-quantized path)
  const float *xd;      // [M][nb] activation scales (pre-quantized path)
  int asm_tokens;       // tokens [0, asm_tokens) multiply by f32(f16_rne(xd)) (ASM chain)
  int wf;               // weights: 0 q4 (kq4 stream layout); q8 (q8 stream layout) with the
                        // 1 fused VDOT or 2 unfused GEMM chain
  int cols;
  int nb;
  int nw;               // waves per workgroup
  int ntok;             // tokens of the 16-token kernel (9-16; the rows past it are padding)
};

// up != nullptr: quantizes silu_mul(x, up) instead of x (the dense FFN's down input).
int kq4_launch_quantize(const float *x, int8_t *xq, float *xd, float *xde, int n_batch, int cols,
                        int asm_tokens, hipStream_t stream, int block_major = 0,
                        const float *up = nullptr);
// g[i] = silu_mul(g[i], u[i]) in place, the reference worker's element rule (g, u 16-B aligned).
int kq4_launch_silu_mul(float *g, const float *u, long n, hipStream_t stream);
// RMSNorm of n_batch rows of d (d % 8 == 0, d <= 16384; 16-B aligned rows), serial = 0 the chunked order of
// dyn_rms_norm, 1 the serial order of dyn_rms_norm_batch; out (may be null) the fp32 result,
// xq/xd (may be null; d % 32 == 0) its int8 quantization, token-major. LDS: kq4_rms_norm_lds.
size_t kq4_rms_norm_lds(int d, int serial);
int kq4_launch_rms_norm(const float *x, const float *w, float *out, int8_t *xq, float *xd,
                        int n_batch, int d, float eps, int serial, hipStream_t stream);

// One GEMV launch (kq4_gemv_impl.h): n_batch in [1, KQ4_GEMV_MAX_M]; kind 0 = per-lane v_dot4
// dots (n_batch <= KQ4_GEMV_DOT4_MAX_M), 1 = v_mfma dots; half_sets 0 (whole 32-row sets, rps of
// them per group), 1 (16-row halves) or 2 (8-row quarters, rps = 1); grid = groups workgroups
// of args.nw (1..16) waves. args.xf (in-kernel quantization) for every n_batch.
#define KQ4_GEMV_DOT4_MAX_M 4
#define KQ4_GEMV_MAX_RPS 3
#define KQ4_GEMV_RPS_MAX_WAVES 8   // waves per workgroup when it takes several row sets
int kq4_launch_gemv(const KQ4GemvArgs &args, int n_batch, int kind, int half_sets, int rps,
                    int grid, hipStream_t stream);
int kq4_gemv_slab_bytes(int n_batch);

int kq4_launch_block_sums(int32_t *s_lo, int32_t *s_hi, const int8_t *xq, const uint8_t *w,
                          int rows, int cols, int n_batch, hipStream_t stream);

// Prefill GEMM (int8 MFMA) with the exact reference chain `chain` (ASM, GEMV32 or CTILE) for
// tokens [0, n_tok). Activation (token t, block b) is at xq + t*q_ts + b*q_bs (bytes) and its
// scale at xd + t*d_ts + b*d_bs; the layout must be token-major (q_ts >= (nb-1)*q_bs + 32 and
// d_ts >= (nb-1)*d_bs + 1), which the launcher checks.
struct KQ4GemmAct {
  const int8_t *xq;
  long q_ts, q_bs;
  const float *xd;
  long d_ts, d_bs;
};
// wf = 1: Q8_0 weights in the q8 stream layout, chain KQ4_CHAIN_Q8GEMM or KQ4_CHAIN_GEMV32.
// tile: 1 / 2 / 3 / 4 = 128x128 / 64x128 / 64x64 / 128x64 (tokens x rows; the C-tile chain is
// capped at 64x128), 0 the planner's choice (kq4_gemm_plan).
// ksplit > 1: K in that many slices, each its own chain from zero, added in slice order by a
// second launch; part = (ksplit - 1) * n_tok * rows floats of workspace (16-byte aligned) for
// slices 1 .. ksplit - 1. Within 1e-5 of the single chain, not bit-identical to it.
// prio: the 128x128 form's issue priority by progress through K (kq4_prio_by_progress): 0 off,
// 1 on, -1 on for launches of whole rounds (a multiple of two workgroups per CU). Outputs do
// not depend on it.
#define KQ4_GEMM_SPLIT_MAX 8
#define KQ4_SPLIT_PART_MAX (24u << 20)   // partial-sum bytes of the planner's splits, at most
// The planner's tile and K slices of one prefill GEMM launch; force_tile / force_split are the
// planner options gemm_tile and gemm_split (-1: the planner's choice).
struct KQ4GemmPlan {
  int tile, ksplit;
};
KQ4GemmPlan kq4_gemm_plan(int n_tok, int rows, int cols, int wf, int chain, int ncu,
                          int force_tile, int force_split);
int kq4_launch_gemm(float *out, const float *res, const uint8_t *w, const KQ4GemmAct &act,
                    int rows, int cols, int n_tok, int chain, int ncu, hipStream_t stream,
                    int wf = 0, int tile = 0, int ksplit = 1, float *part = nullptr,
                    int prio = -1);

// Prefill GEMM on fp8 matrix-core operands (ASM or GEMV32 chain, q4 weights, bit-identical to
// kq4_launch_gemm): xp = the activations' e4m3 operand pairs [n_tok][cols/32][64] (the
// quantizer's block_major = 2 output), xd their f32 scales [n_tok][cols/32].
int kq4_launch_gemm_f8(float *out, const float *res, const uint8_t *w, const uint8_t *xp,
                       const float *xd, int rows, int cols, int n_tok, int chain, int ncu,
                       hipStream_t stream, int tile = 0);

// MoE
int kq4_launch_moe_route(int *sel, float *pr, const float *logits, int T, int ne, int tk,
                         hipStream_t stream);
// fp32 router logits [T][ne] = router [ne][d] . X [T][d], the reference's serial chain per
// (token, expert); d % 32 == 0, rows 16-byte aligned.
int kq4_launch_moe_logits(float *logits, const float *router, const float *X, int T, int ne,
                          int d, hipStream_t stream);
#define KQ4_MOE_REC 16     // ints per slot record (3 header + 12 pair ids + 1 spare)
#define KQ4_MOE_RECP 12    // pair ids a slot record holds
struct KQ4MoeWs {
  int *ex_off;   // [ne+1]
  int *ex_pair;  // [T*tk] (t*tk+j) grouped by expert
  int *rec;      // [ne][KQ4_MOE_REC] slot records (active experts in id order): expert (-1 past
                 // them), offset of its pairs in ex_pair, pair count, its first pair ids
  int8_t *xq;    // [T][d]
  float *xd;     // [T][d/32]
  int8_t *avq;   // [T*tk][ef]
  float *avd;    // [T*tk][ef/32]
  float *P;      // [T*tk][d]
  int ncu;       // compute units of the device (sizes the down projection's workgroups)
};
// Shapes the MoE kernels take: d, ef multiples of 32, d <= 4096, ef <= 3840.
int kq4_moe_shape_ok(int d, int ef);
int kq4_launch_moe_dbg(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                       const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d,
                       int ef, const KQ4MoeWs &ws, float *g_out, float *u_out, float *av_out,
                       const float *av_in, hipStream_t s);
int kq4_launch_moe(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                   const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                   const KQ4MoeWs &ws, hipStream_t stream);
