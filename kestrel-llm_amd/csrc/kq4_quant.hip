// kq4_quant.hip - activation quantizer (fp32 -> int8 + per-32-block f32 scale) for gfx950.
//
// Restates quantize_row_q8_0_act (kestrel-llm src/model/vllm_safetensors.c:7893-7920) bit for
// bit: amax = max(1e-10f, max|x|); d = amax / 127.0f (IEEE division); q = (int)(x/d + 0.5f)
// (truncation toward zero), clamped to [-127, 127]; every x/d is a true IEEE division.
// With `up` given it quantizes silu_mul(x, up) (kq4_silu_mul), the input of the dense FFN's down
// projection, without writing that product to memory.
#include "kq4_common.h"
#include "kq4_internal.h"

// A lane quad per block: each lane reads 8 consecutive floats (two 16-B loads; a wave's load
// instruction covers 16 blocks = 1 KB), the quad's max takes two shuffles, and each lane writes its
// 8 codes as one 8-byte store.
__global__ __launch_bounds__(256) void kq4_quantize_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ up,
                                                           int8_t *__restrict__ xq,
                                                           float *__restrict__ xd,
                                                           float *__restrict__ xde, int n_batch,
                                                           int cols, int nb, int asm_tokens,
                                                           int block_major) {
  const int qq = threadIdx.x & 3;
  const long blk = (long)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
  if (blk >= (long)n_batch * nb) return;  // whole quads exit together
  const int m = (int)(blk / nb);
  const int b = (int)(blk - (long)m * nb);
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
  a = fmaxf(a, __shfl_xor(a, 1));
  a = fmaxf(a, __shfl_xor(a, 2));
  const float d = a / 127.0f;
  uint32_t pk[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int q = (int)(v[i] / d + 0.5f);
    q = q > 127 ? 127 : (q < -127 ? -127 : q);
    pk[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
  }
  // token-major [m][cols] / [m][nb], or block-major [b][m][32] / [b][m] for the GEMM
  const size_t qo = block_major ? ((size_t)b * n_batch + m) * 32 + 8 * qq : off;
  const size_t so = block_major ? (size_t)b * n_batch + m : (size_t)blk;
  *reinterpret_cast<uint2 *>(xq + qo) = make_uint2(pk[0], pk[1]);
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
  const long grid = (nblk + per_wg - 1) / per_wg;
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
