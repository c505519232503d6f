// kq4_quant.hip - activation quantizer (fp32 -> int8 + per-32-block f32 scale) for gfx950.
//
// Restates quantize_row_q8_0_act (kestrel-llm src/model/vllm_safetensors.c:7893-7920) bit for
// bit: amax = max(1e-10f, max|x|); d = amax / 127.0f (IEEE division); q = (int)(x/d + 0.5f)
// (truncation toward zero), clamped to [-127, 127]. Each half-wave (32 lanes) owns one 32-element
// block: one coalesced 128-byte read, a 5-step xor-shuffle max, one divide per lane.
#include "kq4_common.h"
#include "kq4_internal.h"

__global__ __launch_bounds__(256) void kq4_quantize_kernel(const float *__restrict__ x,
                                                           int8_t *__restrict__ xq,
                                                           float *__restrict__ xd,
                                                           float *__restrict__ xde, int n_batch,
                                                           int cols, int nb, int asm_tokens,
                                                           int block_major) {
  const int lane = threadIdx.x & 31;
  const long blk = (long)blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5);
  if (blk >= (long)n_batch * nb) return;  // whole 32-lane halves exit together
  const int m = (int)(blk / nb);
  const int b = (int)(blk - (long)m * nb);
  const size_t off = (size_t)m * cols + (size_t)b * 32 + lane;
  const float v = x[off];
  // token-major [m][cols] / [m][nb], or block-major [b][m][32] / [b][m] for the GEMM
  const size_t qo = block_major ? ((size_t)b * n_batch + m) * 32 + lane : off;
  const size_t so = block_major ? (size_t)b * n_batch + m : (size_t)blk;
  float a = fmaxf(fabsf(v), 1e-10f);
#pragma unroll
  for (int s = 16; s > 0; s >>= 1) a = fmaxf(a, __shfl_xor(a, s, 32));
  const float d = a / 127.0f;
  int q = (int)(v / d + 0.5f);
  q = q > 127 ? 127 : (q < -127 ? -127 : q);
  xq[qo] = (int8_t)q;
  if (lane == 0) {
    xd[so] = d;
    if (xde) xde[so] = (m < asm_tokens) ? kq4_f16_round(d) : d;
  }
}

int kq4_launch_quantize(const float *x, int8_t *xq, float *xd, float *xde, int n_batch, int cols,
                        int asm_tokens, hipStream_t stream, int block_major) {
  const int nb = cols / 32;
  const long nblk = (long)n_batch * nb;
  if (nblk <= 0) return 0;
  const int per_wg = 256 / 32;
  const long grid = (nblk + per_wg - 1) / per_wg;
  hipLaunchKernelGGL(kq4_quantize_kernel, dim3((unsigned)grid), dim3(256), 0, stream, x, xq, xd,
                     xde, n_batch, cols, nb, asm_tokens, block_major);
  return (int)hipGetLastError();
}
