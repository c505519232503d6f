// kq4_gemv.hip - decode GEMV (1..8 tokens) over VQF 4x4 q4 tiles x int8 activations, gfx950.
//
// Computes out[m][n] = sum_b fl(wd[n,b] * xs[m,b]) * S[m,n,b], where S is the exact integer
// dot of row n's 32 nibble weights (n-8) with the token's int8 block and xs is the token's
// block scale (f16-rounded for ASM-chain tokens, as the reference's asm path; the op of
// q4x4_gemm_batched / dyn_matvec_q4_q8, kestrel-llm src/model/vllm_safetensors.c:4593-4631,
// 6147-6174). The integer sums are exact (v_dot4_i32_i8 on 16*(n-8) bytes, |16 S| < 2^20);
// the per-block products are summed in a split-K tree rather than the reference's serial
// chain, so fp32 outputs agree to a few ulp of the row magnitude, not bit for bit.
//
// Work decomposition (HBM-bound: the weight stream is the whole cost):
//   workgroup = a 16-row slab (4 tile groups) over the whole K, split into chunks of 32*PPL
//   blocks handed to its 1..8 waves; lane (g = lane/16, j = lane%16) of a wave owns tile pairs
//   (2 consecutive blocks, 144 B = 9 x 16 B loads) p = j + 16 i of its chunk, so the 16 lanes
//   of a group read 16 consecutive pairs (2304 B contiguous) per load instruction, and every
//   lane issues all loads of a chunk before computing. Per-lane partial sums (4 rows x M
//   tokens) are all-reduced across the 16 lanes with DPP, then the wave partials are added in
//   wave order through LDS: deterministic, one launch, no cross-workgroup synchronisation.
#include "kq4_common.h"
#include "kq4_internal.h"

// Integer sums of one tile row against one int8 block (qa[0..7] = 32 activations):
// returns 16*S_lo and 16*S_hi. Shared by the GEMV and the block-sum verification kernel.
KQ4_DEV void kq4_row_dot16(const uint32_t *tile, int r, const uint32_t *qa, int &lo16,
                           int &hi16) {
  int lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = tile[2 + 4 * k + r];
    lo = kq4_dot4(kq4_lo16(w), qa[k], lo);
    hi = kq4_dot4(kq4_hi16(w), qa[4 + k], hi);
  }
  lo16 = lo;
  hi16 = hi;
}

// Weight-stream load (plain cached load; switchable to a non-temporal hint for measurement).
#ifndef KQ4_WLOAD
#define KQ4_WLOAD(p) (*(p))
#endif

template <bool A16>
KQ4_DEV void kq4_load_pair(uint32_t *dst, const uint8_t *src, bool second) {
  if (A16) {
    // even block count: every pair is complete and 16-byte aligned (144 B = 9 x 16 B; chunk 4
    // straddles the two tiles)
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const uint4 v = KQ4_WLOAD(s + i);
      dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
  } else {
    const uint2 *s = reinterpret_cast<const uint2 *>(src);
    const int n8 = second ? 18 : 9;
#pragma unroll
    for (int i = 0; i < 18; ++i) {
      if (i < n8) {
        const uint2 v = KQ4_WLOAD(s + i);
        dst[2 * i] = v.x; dst[2 * i + 1] = v.y;
      }
    }
  }
}

// Quantizes the activation blocks [bbase, bbase + 32) of M tokens into this wave's LDS slice
// (quantize_row_q8_0_act vllm_safetensors.c:7893-7920): lane pair (2 bl, 2 bl + 1) owns block
// bl, 16 elements each. d = amax / 127 is a true division; x / d is computed as the
// Markstein-corrected quotient q = x*y, q += fma(-q, d, x) * y with y = RN(1/d), which is the
// correctly rounded x / d for normal operands (d >= 1e-10/127 here), so the codes are the
// reference's bit for bit.
template <int M>
KQ4_DEV void kq4_quantize_chunk(const float *__restrict__ xf, int cols, int nb, int bbase,
                                int lane, int8_t *sq, float *sx) {
  const int bl = lane >> 1, h = lane & 1;
  const int b = bbase + bl;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v[16];
    if (b < nb) {
      const float4 *src = reinterpret_cast<const float4 *>(xf + (size_t)m * cols + (size_t)b * 32 + 16 * h);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 f = src[i];
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = 0.0f;
    }
    float amax = 1e-10f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    const float d = amax / 127.0f;
    const float y = 1.0f / d;
    uint32_t pk[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float q = v[i] * y;
      const float e = fmaf(-q, d, v[i]);
      q = fmaf(e, y, q);
      int c = (int)(q + 0.5f);
      c = c > 127 ? 127 : (c < -127 ? -127 : c);
      pk[i >> 2] |= ((uint32_t)c & 0xFFu) << (8 * (i & 3));
    }
    *reinterpret_cast<uint4 *>(sq + m * 1024 + bl * 32 + 16 * h) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    if (h == 0) sx[m * 32 + bl] = d;
  }
}

template <int M, int PPL, bool A16, bool FQ>
__global__ __launch_bounds__(64 * KQ4_GEMV_MAXW) void kq4_gemv_kernel(const KQ4GemvArgs a) {
  __shared__ float sred[KQ4_GEMV_MAXW][16 * KQ4_GEMV_MAX_M];
  // fused quantization (FQ): per-wave int8 codes and scales of the current K chunk
  __shared__ __align__(16) int8_t sq[FQ ? KQ4_GEMV_MAXW : 1][FQ ? M * 1024 : 16];
  __shared__ float sx[FQ ? KQ4_GEMV_MAXW : 1][FQ ? M * 32 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwave = blockDim.x >> 6;
  const int wg = blockIdx.x;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < KQ4_MAXMAT; ++i)
    if (i < a.nmat && wg >= a.mat[i].wg_begin) mi = i;
  const uint8_t *__restrict__ w = a.mat[mi].w;
  const int rows = a.mat[mi].rows;
  const int slab = wg - a.mat[mi].wg_begin;
  const int gl = lane >> 4, j = lane & 15;
  const int g = slab * 4 + gl;
  const int nb = a.nb, cols = a.cols;
  const bool gvalid = g < (rows >> 2);
  const int bpw = 32 * PPL;

  float acc[4][M];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  // wave `wave` takes K chunks wave, wave + nwave, ...; all loads of a chunk are in flight
  // before its arithmetic starts
  for (int bbase = wave * bpw; bbase < nb; bbase += nwave * bpw) {
    uint32_t t[PPL][36];
    bool valid[PPL], second[PPL];
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
      const int b0 = bbase + 2 * (p * 16 + j);
      valid[p] = gvalid && b0 < nb;
      second[p] = b0 + 1 < nb;
      if (valid[p]) kq4_load_pair<A16>(t[p], w + ((size_t)g * nb + b0) * 72, second[p]);
    }
    if (FQ) {   // weight loads are in flight; quantize this chunk's activations meanwhile
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // previous chunk's LDS reads done
      kq4_quantize_chunk<M>(a.xf, cols, nb, bbase, lane, &sq[wave][0], &sx[wave][0]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // codes visible to the whole wave
    }
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
      if (!valid[p]) continue;
      const int b0 = bbase + 2 * (p * 16 + j);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (tt == 1 && !second[p]) break;
        const int b = b0 + tt;
        const uint32_t *tile = &t[p][18 * tt];
        float wd[4];
        wd[0] = kq4_h2f(tile[0]) * 0.0625f;
        wd[1] = kq4_h2f(tile[0] >> 16) * 0.0625f;
        wd[2] = kq4_h2f(tile[1]) * 0.0625f;
        wd[3] = kq4_h2f(tile[1] >> 16) * 0.0625f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4 *qp =
              FQ ? reinterpret_cast<const uint4 *>(&sq[wave][m * 1024 + (b - bbase) * 32])
                 : reinterpret_cast<const uint4 *>(a.xq + (size_t)m * cols + (size_t)b * 32);
          const uint4 q0 = qp[0], q1 = qp[1];
          const uint32_t qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
          const float xr = FQ ? sx[wave][m * 32 + (b - bbase)] : a.xd[(size_t)m * nb + b];
          const float xs = (m < a.asm_tokens) ? kq4_f16_round(xr) : xr;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int lo16, hi16;
            kq4_row_dot16(tile, r, qa, lo16, hi16);
            // 16*S times fl(wd*xs)/16 == S * fl(wd*xs) exactly (power-of-two scaling).
            acc[r][m] = fmaf((float)(lo16 + hi16), wd[r] * xs, acc[r][m]);
          }
        }
      }
    }
  }

  // all-reduce each (row, token) partial over the 16 lanes of the group
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = kq4_row16_sum(acc[r][m]);

  float *__restrict__ out = a.mat[mi].out;
  const float *__restrict__ res = a.mat[mi].res;
  if (nwave == 1) {
    if (gvalid) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (((r * M + m) & 15) == j) {
            const size_t o = (size_t)m * rows + (size_t)g * 4 + r;
            out[o] = res ? res[o] + acc[r][m] : acc[r][m];
          }
    }
    return;
  }
  // K chunks of the slab were split over the waves: add the wave partials in wave order
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (((r * M + m) & 15) == j) sred[wave][(gl * 4 + r) * M + m] = acc[r][m];
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * M; idx += blockDim.x) {
    const int rr = idx / M, m = idx - rr * M;
    const int n = slab * 16 + rr;
    float s = sred[0][idx];
    for (int v = 1; v < nwave; ++v) s += sred[v][idx];
    if (n < rows) {
      const size_t o = (size_t)m * rows + n;
      out[o] = res ? res[o] + s : s;
    }
  }
}

template <int M, int PPL, bool FQ>
static void launch_m(const KQ4GemvArgs &a, int total_wg, bool a16, hipStream_t s) {
  const dim3 block(64 * a.nwave);
  if (a16)
    hipLaunchKernelGGL((kq4_gemv_kernel<M, PPL, true, FQ>), dim3(total_wg), block, 0, s, a);
  else
    hipLaunchKernelGGL((kq4_gemv_kernel<M, PPL, false, FQ>), dim3(total_wg), block, 0, s, a);
}

template <int PPL>
static void launch_ppl(const KQ4GemvArgs &a, int n_batch, int total_wg, bool a16, hipStream_t s) {
  switch (n_batch) {
    case 1: launch_m<1, PPL, false>(a, total_wg, a16, s); break;
    case 2: launch_m<2, PPL, false>(a, total_wg, a16, s); break;
    case 3: launch_m<3, PPL, false>(a, total_wg, a16, s); break;
    case 4: launch_m<4, PPL, false>(a, total_wg, a16, s); break;
    case 5: launch_m<5, PPL, false>(a, total_wg, a16, s); break;
    case 6: launch_m<6, PPL, false>(a, total_wg, a16, s); break;
    case 7: launch_m<7, PPL, false>(a, total_wg, a16, s); break;
    default: launch_m<8, PPL, false>(a, total_wg, a16, s); break;
  }
}

int kq4_launch_gemv(const KQ4GemvArgs &a, int n_batch, int ppl, int total_wg, hipStream_t s) {
  if (n_batch < 1 || n_batch > KQ4_GEMV_MAX_M || total_wg <= 0) return (int)hipErrorInvalidValue;
  bool a16 = (a.nb % 2) == 0;
  for (int i = 0; i < a.nmat; ++i) a16 = a16 && ((uintptr_t)a.mat[i].w % 16) == 0;
  if (a.xf) {   // fused activation quantization: one pair per lane per 32-block chunk
    if (n_batch > KQ4_GEMV_FQ_MAX_M) return (int)hipErrorInvalidValue;
    switch (n_batch) {
      case 1: launch_m<1, 1, true>(a, total_wg, a16, s); break;
      case 2: launch_m<2, 1, true>(a, total_wg, a16, s); break;
      case 3: launch_m<3, 1, true>(a, total_wg, a16, s); break;
      default: launch_m<4, 1, true>(a, total_wg, a16, s); break;
    }
  } else if (ppl == 2) {
    launch_ppl<2>(a, n_batch, total_wg, a16, s);
  } else {
    launch_ppl<1>(a, n_batch, total_wg, a16, s);
  }
  return (int)hipGetLastError();
}

// ---- verification: exact per-block integer sums through kq4_row_dot16 ---------------------
__global__ __launch_bounds__(256) void kq4_block_sums_kernel(int32_t *__restrict__ s_lo,
                                                             int32_t *__restrict__ s_hi,
                                                             const int8_t *__restrict__ xq,
                                                             const uint8_t *__restrict__ w,
                                                             int rows, int cols, int n_batch) {
  const int nb = cols / 32;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)n_batch * rows * nb;
  if (idx >= total) return;
  const int b = (int)(idx % nb);
  const long mn = idx / nb;
  const int n = (int)(mn % rows);
  const int m = (int)(mn / rows);
  const uint2 *tp = reinterpret_cast<const uint2 *>(w + ((size_t)(n >> 2) * nb + b) * 72);
  uint32_t tile[18];
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const uint2 v = tp[i];
    tile[2 * i] = v.x;
    tile[2 * i + 1] = v.y;
  }
  const uint4 *qp = reinterpret_cast<const uint4 *>(xq + (size_t)m * cols + (size_t)b * 32);
  const uint4 q0 = qp[0], q1 = qp[1];
  const uint32_t qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  int lo16, hi16;
  kq4_row_dot16(tile, n & 3, qa, lo16, hi16);
  s_lo[idx] = lo16 >> 4;   // exact: both are multiples of 16
  s_hi[idx] = hi16 >> 4;
}

int kq4_launch_block_sums(int32_t *s_lo, int32_t *s_hi, const int8_t *xq, const uint8_t *w,
                          int rows, int cols, int n_batch, hipStream_t s) {
  const long total = (long)n_batch * rows * (cols / 32);
  if (total <= 0) return 0;
  hipLaunchKernelGGL(kq4_block_sums_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     s, s_lo, s_hi, xq, w, rows, cols, n_batch);
  return (int)hipGetLastError();
}
