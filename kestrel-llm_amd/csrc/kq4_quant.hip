// kq4_quant.hip - activation quantizer (fp32 -> int8 + per-32-block f32 scale) for gfx950.
//
// Restates quantize_row_q8_0_act (kestrel-llm src/model/vllm_safetensors.c:7893-7920) bit for
// bit: amax = max(1e-10f, max|x|); d = amax / 127.0f (IEEE division); q = (int)(x/d + 0.5f)
// (truncation toward zero), clamped to [-127, 127]; every x/d is a true IEEE division.
// With `up` given it quantizes silu_mul(x, up) (kq4_silu_mul), the input of the dense FFN's down
// projection, without writing that product to memory.
#include "kq4_common.h"
#include "kq4_internal.h"

#include <stdlib.h>

// A lane quad per (token, block): each lane reads 8 consecutive floats (two 16-B loads), the
// quad's maximum takes two DPP quad permutes (an integer maximum: amax is non-negative and never
// NaN), and each lane writes its 8 codes as one 8-byte store. Each x/d is the Markstein-corrected
// quotient q = RN(x*y), q = RN(q + RN(x - q*d)*y) with y = RN(1/d): two IEEE divisions per lane
// (d and 1/d) instead of nine. It equals the IEEE quotient for every pair of float32
// significands (all 2^46, kestrel-llm_amd/probe/kq4_div_probe.hip), hence for all operands here
// whose residual stays normal; where it would not (|x| < 2^-102, while d >= 1e-10/127), |x/d| is
// below 2^-61 and both give code 0.
// Token-major output: a wave's 16 quads take 16 consecutive blocks of a token. Block-major
// output ([b][m][32]): a wave's 16 quads take 4 tokens x 4 blocks, so each block's 128 B of
// codes for the 4 tokens is written whole by one store instruction (one quad per block in
// token-major order would leave each 128-B line to four workgroups, on different XCDs).
__global__ __launch_bounds__(256) void kq4_quantize_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ up,
                                                           int8_t *__restrict__ xq,
                                                           float *__restrict__ xd,
                                                           float *__restrict__ xde, int n_batch,
                                                           int cols, int nb, int asm_tokens,
                                                           int block_major) {
  const int qq = threadIdx.x & 3;
  const long gq = (long)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
  int m, b;
  if (block_major == 1) {
    const long g = gq >> 4;
    const int qi = (int)(gq & 15), nbg = (nb + 3) >> 2;
    m = (int)(g / nbg) * 4 + (qi & 3);
    b = (int)(g % nbg) * 4 + (qi >> 2);
    if (m >= n_batch || b >= nb) return;   // whole quads exit together
  } else {
    if (gq >= (long)n_batch * nb) return;
    m = (int)(gq / nb);
    b = (int)(gq - (long)m * nb);
  }
  const long blk = (long)m * nb + b;
  const size_t off = (size_t)m * cols + (size_t)b * 32 + 8 * qq;
  const float4 v0 = *reinterpret_cast<const float4 *>(x + off);
  const float4 v1 = *reinterpret_cast<const float4 *>(x + off + 4);
  float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  if (up) {
    const float4 u0 = *reinterpret_cast<const float4 *>(up + off);
    const float4 u1 = *reinterpret_cast<const float4 *>(up + off + 4);
    const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = kq4_silu_mul(v[i], u[i]);
  }
  float a = 1e-10f;
#pragma unroll
  for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
  a = kq4_quad_max_pos(a);
  const float d = a / 127.0f;
  const float y = 1.0f / d;
  int c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q = v[i] * y;
    const float e = fmaf(-q, d, v[i]);
    q = fmaf(e, y, q);
    c[i] = (int)(q + 0.5f);
    c[i] = c[i] > 127 ? 127 : (c[i] < -127 ? -127 : c[i]);
  }
  // low bytes of c[0..3], c[4..7] into one dword each: two byte selects and an or
  uint32_t pk[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    pk[k] = __builtin_amdgcn_perm((uint32_t)c[4 * k + 1], (uint32_t)c[4 * k], 0x0c0c0400u) |
            __builtin_amdgcn_perm((uint32_t)c[4 * k + 3], (uint32_t)c[4 * k + 2], 0x04000c0cu);
  // token-major [m][cols] / [m][nb], block-major [b][m][32] / [b][m], or (block_major = 2) the
  // fp8 GEMM's operand pairs [m][nb][64]: the e4m3 bytes of 16*(q >> 4) for the block's 32
  // elements, then those of q & 15 (kq4_e4m3_hi / _lo), scales token-major
  const size_t so = block_major == 1 ? (size_t)b * n_batch + m : (size_t)blk;
  if (block_major == 2) {
    uint32_t hi[2] = {0, 0}, lo[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = (int)(int8_t)(pk[i >> 2] >> (8 * (i & 3)));
      hi[i >> 2] |= kq4_e4m3_hi(q) << (8 * (i & 3));
      lo[i >> 2] |= kq4_e4m3_lo(q) << (8 * (i & 3));
    }
    uint8_t *pair = reinterpret_cast<uint8_t *>(xq) + (size_t)blk * 64 + 8 * qq;
    *reinterpret_cast<uint2 *>(pair) = make_uint2(hi[0], hi[1]);
    *reinterpret_cast<uint2 *>(pair + 32) = make_uint2(lo[0], lo[1]);
  } else {
    const size_t qo = block_major ? ((size_t)b * n_batch + m) * 32 + 8 * qq : off;
    *reinterpret_cast<uint2 *>(xq + qo) = make_uint2(pk[0], pk[1]);
  }
  if (qq == 0) {
    xd[so] = d;
    if (xde) xde[so] = (m < asm_tokens) ? kq4_f16_round(d) : d;
  }
}

int kq4_launch_quantize(const float *x, int8_t *xq, float *xd, float *xde, int n_batch, int cols,
                        int asm_tokens, hipStream_t stream, int block_major, const float *up) {
  const int nb = cols / 32;
  const long nblk = (long)n_batch * nb;
  if (nblk <= 0) return 0;
  const int per_wg = 256 / 4;
  // block-major: whole groups of 4 tokens x 4 blocks
  const long quads = block_major == 1 ? (long)((n_batch + 3) / 4) * ((nb + 3) / 4) * 16 : nblk;
  const long grid = (quads + per_wg - 1) / per_wg;
  hipLaunchKernelGGL(kq4_quantize_kernel, dim3((unsigned)grid), dim3(256), 0, stream, x, up, xq, xd,
                     xde, n_batch, cols, nb, asm_tokens, block_major);
  return (int)hipGetLastError();
}

// ---- SiLU * up in place ------------------------------------------------------------------------
// vllm_silu_mul_worker (vllm_safetensors.c:10932-10958) over n elements: g[i] = silu_mul(g[i],
// u[i]) in the NEON form for i < (n & ~3); the last n % 4 elements take the worker's scalar tail,
// fast_silu(g) * u (:3685-3696), with exp evaluated in double and rounded once (the correctly
// rounded expf; the reference's libm expf may differ from it in the last bit).
KQ4_DEV float kq4_fast_silu(float x) {
  if (x <= 0.0f) {
    if (x < -20.0f) return 0.0f;
    const float ex = (float)exp((double)x);
    return x * ex / (1.0f + ex);
  }
  if (x > 20.0f) return x;
  return x / (1.0f + (float)exp((double)-x));
}

__global__ __launch_bounds__(256) void kq4_silu_mul_kernel(float *__restrict__ g,
                                                           const float *__restrict__ u, long n) {
  const long i4 = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 + 4 <= n) {
    float4 a = *reinterpret_cast<const float4 *>(g + i4);
    const float4 b = *reinterpret_cast<const float4 *>(u + i4);
    a.x = kq4_silu_mul(a.x, b.x);
    a.y = kq4_silu_mul(a.y, b.y);
    a.z = kq4_silu_mul(a.z, b.z);
    a.w = kq4_silu_mul(a.w, b.w);
    *reinterpret_cast<float4 *>(g + i4) = a;
  } else {
    for (long i = i4; i < n; ++i) g[i] = kq4_fast_silu(g[i]) * u[i];
  }
}

int kq4_launch_silu_mul(float *g, const float *u, long n, hipStream_t stream) {
  if (n <= 0) return 0;
  const long grid = (n + 1023) / 1024;
  hipLaunchKernelGGL(kq4_silu_mul_kernel, dim3((unsigned)grid), dim3(256), 0, stream, g, u, n);
  return (int)hipGetLastError();
}

// ---- RMSNorm, optionally quantized in the same pass -------------------------------------------
// dyn_rms_norm (vllm_safetensors.c:8811-8827) and dyn_rms_norm_batch's worker (:8849-8867), one
// workgroup per token: out = fl(fl(x * rms) * w), rms = fl(1 / fl(sqrt(fl(fl(ss / d) + eps)))).
// The sum of squares ss is the reference's serial chain, in one of its two orders:
//   chunked (dyn_rms_norm; the batch worker under VLLM_SPEC_VNORM=1): the workgroup's threads
//     form every 8-element chunk's hsum8 of squares, ((q0+q4)+(q1+q5)) + ((q2+q6)+(q3+q7)), into
//     LDS, then one lane adds the d/8 chunk sums in order;
//   serial (dyn_rms_norm_batch's default): the threads square every element into LDS, one lane
//     adds the d squares in order.
// Thread i takes chunks i, i+256, .. (CPT of them). HOLD = 1 (a few tokens: the latency of one
// token is what counts) keeps them and w's in registers from the start, so the only global-memory
// wait is the first; HOLD = 0 (many tokens: the workgroups resident at once are what count) reads
// them again after the sum, so a wave needs about 40 registers and a CU holds 8 workgroups.
// The serial lane reads its terms from LDS 32 at a time. Then each thread normalises its
// chunks and, when xq is given, quantizes them as kq4_quantize_kernel does (a lane quad per
// 32-block, quantize_row_q8_0_act :7893-7920).
// d % 8 == 0 (d % 32 == 0 to quantize), d <= 2048 * CPT; rows 16-byte aligned. out may be x (in
// place, as the reference calls it at :19607): every workgroup reads its own row before the
// barrier that precedes its writes, and re-reads (HOLD = 0) only that row.
#define KQ4_RMS_THREADS 256
#define KQ4_RMS_HOLD_MAX 256   // tokens up to which x and w stay in registers
#define KQ4_RMS_BATCH 32   // terms the serial lane reads from LDS at once

template <int CPT, int HOLD>
__global__ __launch_bounds__(KQ4_RMS_THREADS) void kq4_rms_norm_kernel(
    const float *x, const float *__restrict__ w, float *out, int8_t *__restrict__ xq,
    float *__restrict__ xd, int d, float eps, int serial) {
  extern __shared__ __align__(16) float kq4_rms_lds[];   // d/8 chunk sums, or d squares
  __shared__ float rms_s;
  const int t = blockIdx.x;
  const float *xr = x + (size_t)t * d;
  const int nc = d >> 3;
  auto load8 = [&](const float *p, int c, float *o) {
    float4 a = make_float4(0, 0, 0, 0), b = a;
    if (c < nc) {
      a = *reinterpret_cast<const float4 *>(p + 8 * c);
      b = *reinterpret_cast<const float4 *>(p + 8 * c + 4);
    }
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  };
  float v[HOLD ? CPT : 1][8], wv[HOLD ? CPT : 1][8];
  if (HOLD) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = threadIdx.x + KQ4_RMS_THREADS * j;
      load8(xr, c, v[HOLD ? j : 0]);
      load8(w, c, wv[HOLD ? j : 0]);
    }
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = threadIdx.x + KQ4_RMS_THREADS * j;
    float vj[8];
    if (HOLD) {
#pragma unroll
      for (int k = 0; k < 8; ++k) vj[k] = v[HOLD ? j : 0][k];
    } else {
      load8(xr, c, vj);
    }
    if (c < nc) {
      float q[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = vj[k] * vj[k];
      if (serial) {
        *reinterpret_cast<float4 *>(kq4_rms_lds + 8 * c) = make_float4(q[0], q[1], q[2], q[3]);
        *reinterpret_cast<float4 *>(kq4_rms_lds + 8 * c + 4) = make_float4(q[4], q[5], q[6], q[7]);
      } else {
        kq4_rms_lds[c] = ((q[0] + q[4]) + (q[1] + q[5])) + ((q[2] + q[6]) + (q[3] + q[7]));
      }
    }
  }
  // zero padding to whole batches: adding +0 to the non-negative sum is exact
  const int n = serial ? d : nc;
  const int npad = (n + KQ4_RMS_BATCH - 1) & ~(KQ4_RMS_BATCH - 1);
  for (int i = n + threadIdx.x; i < npad; i += KQ4_RMS_THREADS) kq4_rms_lds[i] = 0.0f;
  __syncthreads();
  // the chain lane: lane 0 of wave (t % 4), so that the chains of a CU's workgroups spread over
  // its four SIMDs
  if (threadIdx.x == 64 * (t & 3)) {
    // one dependent add per term, KQ4_RMS_BATCH terms read at a time (each consumed as it lands)
    float ss = 0.0f;
    for (int i = 0; i < npad; i += KQ4_RMS_BATCH) {
      float4 b[KQ4_RMS_BATCH / 4];
#pragma unroll
      for (int k = 0; k < KQ4_RMS_BATCH / 4; ++k)
        b[k] = *reinterpret_cast<const float4 *>(kq4_rms_lds + i + 4 * k);
#pragma unroll
      for (int k = 0; k < KQ4_RMS_BATCH / 4; ++k) {
        ss += b[k].x;
        ss += b[k].y;
        ss += b[k].z;
        ss += b[k].w;
      }
    }
    rms_s = 1.0f / sqrtf(ss / (float)d + eps);
  }
  __syncthreads();
  const float rms = rms_s;
  float *orow = out ? out + (size_t)t * d : nullptr;
  const int nb = d >> 5;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = threadIdx.x + KQ4_RMS_THREADS * j;
    const bool live = c < nc;
    float vj[8], wj[8];
    if (HOLD) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        vj[k] = v[HOLD ? j : 0][k];
        wj[k] = wv[HOLD ? j : 0][k];
      }
    } else {
      load8(xr, c, vj);
      load8(w, c, wj);
    }
    float o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = vj[k] * rms * wj[k];
    if (live && orow) {
      *reinterpret_cast<float4 *>(orow + 8 * c) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4 *>(orow + 8 * c + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (xq) {   // uniform; nc % 4 == 0 here, so a lane quad is live or dead as a whole
      float a = 1e-10f;
#pragma unroll
      for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(o[i]));
      a = kq4_quad_max(a);
      const float dq = a / 127.0f;
      uint32_t pk[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int q = (int)(o[i] / dq + 0.5f);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        pk[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
      }
      if (live) {
        *reinterpret_cast<uint2 *>(xq + (size_t)t * d + 8 * c) = make_uint2(pk[0], pk[1]);
        if ((c & 3) == 0) xd[(size_t)t * nb + (c >> 2)] = dq;
      }
    }
  }
}

size_t kq4_rms_norm_lds(int d, int serial) {
  const int n = serial ? d : d / 8;
  return (size_t)((n + KQ4_RMS_BATCH - 1) & ~(KQ4_RMS_BATCH - 1)) * sizeof(float);
}

template <int CPT, int HOLD>
static hipError_t rms_launch_h(const float *x, const float *w, float *out, int8_t *xq, float *xd,
                               int n_batch, int d, float eps, int serial, hipStream_t s) {
  // the serial order keeps d squares in LDS (64 KB at d = 16384); the kernel's static LDS (the
  // broadcast rms) comes off the 160 KB a workgroup may hold
  static std::atomic<unsigned long long> attr{0};
  hipError_t e = kq4_lds_limit_once(
      reinterpret_cast<const void *>(&kq4_rms_norm_kernel<CPT, HOLD>), 160 * 1024 - 1024, attr);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((kq4_rms_norm_kernel<CPT, HOLD>), dim3(n_batch), dim3(KQ4_RMS_THREADS),
                     kq4_rms_norm_lds(d, serial), s, x, w, out, xq, xd, d, eps, serial);
  return hipGetLastError();
}

// Registers held (HOLD = 1) up to KQ4_RMS_HOLD_MAX tokens, re-read beyond (KQ4_RMS_HOLD_MAX in the
// environment overrides it, for measurement).
template <int CPT>
static hipError_t rms_launch(const float *x, const float *w, float *out, int8_t *xq, float *xd,
                             int n_batch, int d, float eps, int serial, hipStream_t s) {
  static const int hold_max = [] {
    const char *e = getenv("KQ4_RMS_HOLD_MAX");
    return e ? atoi(e) : KQ4_RMS_HOLD_MAX;
  }();
  if (n_batch <= hold_max)
    return rms_launch_h<CPT, 1>(x, w, out, xq, xd, n_batch, d, eps, serial, s);
  return rms_launch_h<CPT, 0>(x, w, out, xq, xd, n_batch, d, eps, serial, s);
}

int kq4_launch_rms_norm(const float *x, const float *w, float *out, int8_t *xq, float *xd,
                        int n_batch, int d, float eps, int serial, hipStream_t stream) {
  if (n_batch <= 0) return 0;
  const int cpt = (d / 8 + KQ4_RMS_THREADS - 1) / KQ4_RMS_THREADS;
  if (d % 8 || cpt > 8 || (xq && d % 32)) return (int)hipErrorInvalidValue;
  if (cpt <= 1) return (int)rms_launch<1>(x, w, out, xq, xd, n_batch, d, eps, serial, stream);
  if (cpt <= 2) return (int)rms_launch<2>(x, w, out, xq, xd, n_batch, d, eps, serial, stream);
  if (cpt <= 4) return (int)rms_launch<4>(x, w, out, xq, xd, n_batch, d, eps, serial, stream);
  return (int)rms_launch<8>(x, w, out, xq, xd, n_batch, d, eps, serial, stream);
}
