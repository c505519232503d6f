// kq4_gemv.hip - the decode GEMV's dispatch over its per-token-count instantiations
// (kq4_gemv_m<M>.hip, kernel in kq4_gemv_impl.h), the repack from the VQF 4x4 layout into the
// stream layout the kernels read, and the verification kernel of the exact block sums.
#include "kq4_gemv_impl.h"

template <int M>
hipError_t kq4_gv_launch_m(const KQ4GemvArgs &a, int kind, int fq, int hs, int rps, int grid,
                           hipStream_t s);
extern template hipError_t kq4_gv_launch_m<1>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<2>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<3>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<4>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<5>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<6>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<7>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
extern template hipError_t kq4_gv_launch_m<8>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
hipError_t kq4_gv_launch_wide(const KQ4GemvArgs &a, int fq, int hs, int rps, int grid,
                              hipStream_t s);

// a wave's LDS slab: the 16-token kernel (9-16 tokens) holds 16 token rows and 16-wide scales
int kq4_gemv_slab_bytes(int n_batch) {
  return n_batch > KQ4_GEMV_MAX_M ? kq4_gv_slab<KQ4_GEMV_WIDE_M>() : n_batch * KQ4_GV_QTS + KQ4_GV_XS;
}

int kq4_launch_gemv(const KQ4GemvArgs &a, int n_batch, int kind, int half_sets, int rps,
                    int grid, hipStream_t s) {
  const int nw = a.nw;
  const bool wide = n_batch > KQ4_GEMV_MAX_M;   // the 16-token kernel: q4, MFMA, single sets
  if (wide && (n_batch > KQ4_GEMV_WIDE_M || a.ntok != n_batch || a.wf || kind != 1 ||
               half_sets > 1 || (a.xu != nullptr)))
    return (int)hipErrorInvalidValue;
  if (n_batch < 1 || n_batch > KQ4_GEMV_WIDE_M || grid <= 0 || nw < 1 || nw > 16 || kind < 0 ||
      kind > 1 || (kind == 0 && n_batch > KQ4_GEMV_DOT4_MAX_M) || half_sets < 0 ||
      half_sets > 2 || rps < 1 || rps > KQ4_GEMV_MAX_RPS || (half_sets && rps != 1) ||
      (rps > 1 && nw > KQ4_GEMV_RPS_MAX_WAVES) ||
      (size_t)nw * kq4_gemv_slab_bytes(n_batch) > 160 * 1024 - 64)
    return (int)hipErrorInvalidValue;
  for (int i = 0; i < a.nmat; ++i)
    if ((uintptr_t)a.mat[i].w % 16) return (int)hipErrorInvalidValue;
  if (a.xu && !a.xf) return (int)hipErrorInvalidValue;
  const int fq = a.xf ? (a.xu ? 2 : 1) : 0;
  const int hs = half_sets;
  hipError_t e;
  if (wide) return (int)kq4_gv_launch_wide(a, fq, hs, rps, grid, s);
  switch (n_batch) {
    case 1: e = kq4_gv_launch_m<1>(a, kind, fq, hs, rps, grid, s); break;
    case 2: e = kq4_gv_launch_m<2>(a, kind, fq, hs, rps, grid, s); break;
    case 3: e = kq4_gv_launch_m<3>(a, kind, fq, hs, rps, grid, s); break;
    case 4: e = kq4_gv_launch_m<4>(a, kind, fq, hs, rps, grid, s); break;
    case 5: e = kq4_gv_launch_m<5>(a, kind, fq, hs, rps, grid, s); break;
    case 6: e = kq4_gv_launch_m<6>(a, kind, fq, hs, rps, grid, s); break;
    case 7: e = kq4_gv_launch_m<7>(a, kind, fq, hs, rps, grid, s); break;
    default: e = kq4_gv_launch_m<8>(a, kind, fq, hs, rps, grid, s); break;
  }
  return (int)e;
}

// ---- VQF 4x4 -> stream layout ------------------------------------------------------------------
// One thread per 8-byte piece of the stream buffer. Piece o (byte offset in its chunk):
//   o < 8192: unit i = o/1024, lane l = (o/16)%64, block 16*stage + 2i + (o/8)%2 of row
//             32*set + l%32, half h = l/32. From the VQF tile the row's 16 code bytes are the
//             dwords Q[k] at 8 + 16k + 4r (r = row%4; byte j of the row = element j in the low
//             nibble, element j+16 in the high one), so half h's dword d is
//             ((Q[2d] >> 4h) & 0x0F0F0F0F) | ((Q[2d+1] >> 4h) & 0x0F0F0F0F) << 4.
//   o >= 8192: lane l = (o-8192)/16: the f16 scales of row 32*set + l%32, blocks
//             16*stage + 8*(l/32) + 4*((o/8)%2) + 0..3 (tile byte 2r of each block's tile).
// Rows or blocks past the matrix give zeros.
__global__ __launch_bounds__(256) void kq4_repack_kernel(uint8_t *__restrict__ dst,
                                                         const uint8_t *__restrict__ src,
                                                         int rows, int nb, int nst, long total) {
  const long k = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= total) return;
  const long chunk = k / (KQ4_GV_CHUNK / 8);
  const int o = 8 * (int)(k - chunk * (KQ4_GV_CHUNK / 8));
  const int set = (int)(chunk / nst), stage = (int)(chunk - (long)set * nst);
  uint2 v = make_uint2(0, 0);
  if (o < 8192) {
    const int i = o >> 10, l = (o >> 4) & 63, hb = (o >> 3) & 1;
    const int row = 32 * set + (l & 31), h = l >> 5;
    const int b = 16 * stage + 2 * i + hb;
    if (row < rows && b < nb) {
      const uint8_t *tile = src + ((size_t)(row >> 2) * nb + b) * 72 + 8 + 4 * (row & 3);
      uint32_t Q[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) Q[q] = *reinterpret_cast<const uint32_t *>(tile + 16 * q);
      const int sh = 4 * h;
      v.x = ((Q[0] >> sh) & 0x0F0F0F0Fu) | (((Q[1] >> sh) & 0x0F0F0F0Fu) << 4);
      v.y = ((Q[2] >> sh) & 0x0F0F0F0Fu) | (((Q[3] >> sh) & 0x0F0F0F0Fu) << 4);
    }
  } else {
    const int l = (o - 8192) >> 4, hb = (o >> 3) & 1;
    const int row = 32 * set + (l & 31);
    const int b0 = 16 * stage + 8 * (l >> 5) + 4 * hb;
    uint32_t f[4] = {0, 0, 0, 0};
    if (row < rows) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (b0 + u < nb)
          f[u] = *reinterpret_cast<const uint16_t *>(
              src + ((size_t)(row >> 2) * nb + b0 + u) * 72 + 2 * (row & 3));
    }
    v.x = f[0] | (f[1] << 16);
    v.y = f[2] | (f[3] << 16);
  }
  *reinterpret_cast<uint2 *>(dst + chunk * KQ4_GV_CHUNK + o) = v;
}

size_t kq4_stream_bytes(int rows, int cols) {
  const size_t sets = ((size_t)rows + 31) / 32;
  const size_t nst = ((size_t)cols / 32 + KQ4_GV_CB - 1) / KQ4_GV_CB;
  return sets * nst * KQ4_GV_CHUNK;
}

int kq4_launch_repack(uint8_t *dst, const uint8_t *src, int rows, int cols, hipStream_t s) {
  const int nb = cols / 32;
  const int nst = (nb + KQ4_GV_CB - 1) / KQ4_GV_CB;
  const long total = (long)kq4_stream_bytes(rows, cols) / 8;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(kq4_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     dst, src, rows, nb, nst, total);
  return (int)hipGetLastError();
}

// ---- tiled Q8_0 -> q8 stream layout ---------------------------------------------------------------
// One thread per 16-byte piece of the stream buffer. The source is the reference's tiled Q8_0
// (g = 8: block_q8_0x8, 272 B per 8 rows x 32 cols; g = 4: block_q8_0x4, 136 B): g f16 row scales,
// then qs[k*4g + m*4 + i] = row m's element 4k+i. Piece o (byte offset in its chunk):
//   o < 8192: block i = o/1024 of the stage, lane l = (o/16)%64: row 32*set + l%32, half h = l/32,
//             i.e. the 4 dwords k = 4h .. 4h+3 of that row in the tile;
//   o >= 8192: row 32*set + (o-8192)/16: its 8 scales (blocks 8*stage + 0..7).
// Rows or blocks past the matrix give zeros.
__global__ __launch_bounds__(256) void kq8_repack_kernel(uint8_t *__restrict__ dst,
                                                         const uint8_t *__restrict__ src, int g,
                                                         int rows, int nb, int nst, long total) {
  const long k = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= total) return;
  const long chunk = k / (KQ8_STREAM_CHUNK / 16);
  const int o = 16 * (int)(k - chunk * (KQ8_STREAM_CHUNK / 16));
  const int set = (int)(chunk / nst), stage = (int)(chunk - (long)set * nst);
  const size_t tb = (size_t)34 * g;   // bytes per tile
  uint4 v = make_uint4(0, 0, 0, 0);
  if (o < 8192) {
    const int i = o >> 10, l = (o >> 4) & 63;
    const int row = 32 * set + (l & 31), h = l >> 5;
    const int b = KQ8_STREAM_CB * stage + i;
    if (row < rows && b < nb) {
      const uint8_t *q = src + ((size_t)(row / g) * nb + b) * tb + 2 * g + 4 * (row % g);
      v.x = *reinterpret_cast<const uint32_t *>(q + (4 * h + 0) * 4 * g);
      v.y = *reinterpret_cast<const uint32_t *>(q + (4 * h + 1) * 4 * g);
      v.z = *reinterpret_cast<const uint32_t *>(q + (4 * h + 2) * 4 * g);
      v.w = *reinterpret_cast<const uint32_t *>(q + (4 * h + 3) * 4 * g);
    }
  } else {
    const int row = 32 * set + ((o - 8192) >> 4);
    uint32_t f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row < rows) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int b = KQ8_STREAM_CB * stage + u;
        if (b < nb)
          f[u] = *reinterpret_cast<const uint16_t *>(src + ((size_t)(row / g) * nb + b) * tb +
                                                     2 * (row % g));
      }
    }
    v = make_uint4(f[0] | (f[1] << 16), f[2] | (f[3] << 16), f[4] | (f[5] << 16),
                   f[6] | (f[7] << 16));
  }
  *reinterpret_cast<uint4 *>(dst + chunk * KQ8_STREAM_CHUNK + o) = v;
}

size_t kq8_stream_bytes(int rows, int cols) {
  const size_t sets = ((size_t)rows + 31) / 32;
  const size_t nst = ((size_t)cols / 32 + KQ8_STREAM_CB - 1) / KQ8_STREAM_CB;
  return sets * nst * KQ8_STREAM_CHUNK;
}

int kq8_launch_repack(uint8_t *dst, const uint8_t *src, int g, int rows, int cols,
                      hipStream_t s) {
  const int nb = cols / 32;
  const int nst = (nb + KQ8_STREAM_CB - 1) / KQ8_STREAM_CB;
  const long total = (long)kq8_stream_bytes(rows, cols) / 16;
  if (total <= 0) return 0;
  if (g != 8 && g != 4) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kq8_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     dst, src, g, rows, nb, nst, total);
  return (int)hipGetLastError();
}

// ---- verification: exact per-block integer sums through the GEMV's integer dots --------------
// One wave per (32-row set, block, 32-token set), reading the weights in the stream layout.
// S_lo / S_hi come from the MFMA kind's operands and v_mfma (zeroing the B lanes of one K half),
// and are checked against the DOT4 kind's kq4_dot4 sums of the same half-rows (the lane's row,
// first token of the set); a mismatch is written as INT32_MIN so the test fails.
__global__ __launch_bounds__(64) void kq4_block_sums_kernel(int32_t *__restrict__ s_lo,
                                                            int32_t *__restrict__ s_hi,
                                                            const int8_t *__restrict__ xq,
                                                            const uint8_t *__restrict__ w,
                                                            int rows, int cols, int n_batch) {
  const int nb = cols / 32;
  const int nst = (nb + KQ4_GV_CB - 1) / KQ4_GV_CB;
  const int lane = threadIdx.x;
  const int j = lane & 31, h = lane >> 5;
  const int row0 = blockIdx.x * 32, b = blockIdx.y, t0 = blockIdx.z * 32;
  const int rw = row0 + j < rows ? row0 + j : rows - 1;
  const uint2 wv = *reinterpret_cast<const uint2 *>(w + kq4_stream_nib(rw, b, h, nst));
  uint32_t o[4];
  kq4_unpack_half(wv.x, wv.y, o);
  const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
  const kq4_v4i Z = {0, 0, 0, 0};
  int t = t0 + j;
  t = t < n_batch ? t : n_batch - 1;
  const kq4_v4i A = *reinterpret_cast<const kq4_v4i *>(xq + (size_t)t * cols + (size_t)b * 32 + 16 * h);
  const kq4_v16i Clo = kq4_gv_mfma(A, h == 0 ? B : Z);
  const kq4_v16i Chi = kq4_gv_mfma(A, h == 1 ? B : Z);
  // the DOT4 kind's sum of this lane's half-row against token t0, and the other half's
  const uint32_t *q = reinterpret_cast<const uint32_t *>(xq + (size_t)t0 * cols + (size_t)b * 32);
  int dh = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) dh = kq4_dot4(o[k], q[4 * h + k], dh);
  const int dx = __shfl_xor(dh, 32);
  const int dlo = h == 0 ? dh : dx, dhi = h == 0 ? dx : dh;
  const int row = row0 + j;
  if (row >= rows) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int m = t0 + 8 * (v >> 2) + 4 * h + (v & 3);
    if (m >= n_batch) continue;
    const size_t oo = ((size_t)m * rows + row) * nb + b;
    int lo = Clo[v] >> 4, hi = Chi[v] >> 4;   // exact: multiples of 16
    if (m == t0 && (lo != (dlo >> 4) || hi != (dhi >> 4))) lo = hi = INT32_MIN;
    s_lo[oo] = lo;
    s_hi[oo] = hi;
  }
}

int kq4_launch_block_sums(int32_t *s_lo, int32_t *s_hi, const int8_t *xq, const uint8_t *w,
                          int rows, int cols, int n_batch, hipStream_t s) {
  if (n_batch <= 0 || rows <= 0) return 0;
  const dim3 grid((unsigned)((rows + 31) / 32), (unsigned)(cols / 32),
                  (unsigned)((n_batch + 31) / 32));
  hipLaunchKernelGGL(kq4_block_sums_kernel, grid, dim3(64), 0, s, s_lo, s_hi, xq, w, rows, cols,
                     n_batch);
  return (int)hipGetLastError();
}
