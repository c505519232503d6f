// kq4_quant.hip - activation quantizer (fp32 -> int8 + per-32-block f32 scale) for gfx950.
//
// Restates quantize_row_q8_0_act (kestrel-llm src/model/vllm_safetensors.c:7893-7920) bit for
// bit: amax = max(1e-10f, max|x|); d = amax / 127.0f (IEEE division); q = (int)(x/d + 0.5f)
// (truncation toward zero), clamped to [-127, 127]; every x/d is a true IEEE division.
#include "kq4_common.h"
#include "kq4_internal.h"

// A lane quad per block: each lane reads 8 consecutive floats (two 16-B loads; a wave's load
// instruction covers 16 blocks = 1 KB), the quad's max takes two shuffles, and each lane writes its
// 8 codes as one 8-byte store.
__global__ __launch_bounds__(256) void kq4_quantize_kernel(const float *__restrict__ x,
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
  const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
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
                        int asm_tokens, hipStream_t stream, int block_major) {
  const int nb = cols / 32;
  const long nblk = (long)n_batch * nb;
  if (nblk <= 0) return 0;
  const int per_wg = 256 / 4;
  const long grid = (nblk + per_wg - 1) / per_wg;
  hipLaunchKernelGGL(kq4_quantize_kernel, dim3((unsigned)grid), dim3(256), 0, stream, x, xq, xd,
                     xde, n_batch, cols, nb, asm_tokens, block_major);
  return (int)hipGetLastError();
}
