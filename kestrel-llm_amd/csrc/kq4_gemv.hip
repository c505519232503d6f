// kq4_gemv.hip - decode GEMV (1..8 tokens) over VQF 4x4 q4 tiles x int8 activations, gfx950.
//
// Computes out[m][n] = [res +] sum_b S[m,n,b] * fl(wd[n,b] * xs[m,b]), the op of
// q4x4_gemm_batched / dyn_matvec_q4_q8 (kestrel-llm src/model/vllm_safetensors.c:4593-4631,
// 6147-6174): S is the exact integer dot of row n's 32 nibble weights (n-8) with the token's
// int8 block, xs the token's block scale (f16-rounded for ASM-chain tokens, as the reference's
// asm path multiplies by the f16 scale it repacks, :4104-4105). Every per-block term is the
// reference's; the blocks of one output are summed serially within a slice of K and the slices
// are then added in a fixed order, so outputs agree with the reference's single serial chain to a
// few ulp of the row magnitude.
//
// Work decomposition (the weight stream is the whole cost):
//   * a workgroup = one 32-row set (8 tile groups) over the whole K, W waves (1..8); wave w
//     takes the 16-block stages w, w + W, ... . A stage is 8 x 16 x 72 B = 9216 B, loaded as
//     9 x 16 B per lane so that every load instruction reads 1 KB of contiguous bytes (a
//     group's 16 tiles are 1152 contiguous bytes), then laid out per group in the wave's own LDS
//     slab. Up to two stages per wave are in flight, each issued as (activations, weights).
//   * each wave also stages its own activations (int8 codes + per-block scales) in its slab,
//     quantizing them from fp32 itself (FQ, M <= 2) or copying a pre-quantized buffer, so the
//     stage loop has no workgroup barrier.
//   * the integer dot, two kinds:
//       DOT4: lane (g, j) owns the tile pair (2j, 2j+1) of group g; v_dot4_i32_i8 on the
//             nibbles shifted into the high half of each byte (16*(n-8)), the 8 lanes' partial
//             rows all-reduced with DPP. Fewest instructions per byte at small M.
//       MFMA: one v_mfma_i32_32x32x32_i8 per block: A = activations (32 token rows, M <= 8
//             used), B = the 32 weight rows as 16*(n-8) bytes, K = the block's 32 elements; the
//             result 16*S sits in lanes (row = lane%32, token = 4*(lane/32)+v). Its cost does not
//             grow with M.
//   * at the end the waves' partial sums are added in wave order through LDS: deterministic,
//     one launch, no cross-workgroup communication.
#include "kq4_common.h"
#include "kq4_internal.h"

// A stage is G8 groups x CB blocks = 128 tiles = 9216 B: a 32-row set (G8 = 8, CB = 16) or a
// 16-row set (G8 = 4, CB = 32, DOT4 only).
template <int G8>
constexpr int kq4_gv_cb() { return 128 / G8; }
// LDS bytes per token row of a stage's int8 codes (block pairs at an 80-B pitch, see qpos).
template <int G8>
constexpr int kq4_gv_qts() { return G8 == 8 ? 672 : 1312; }

typedef int kq4_v4i __attribute__((ext_vector_type(4)));
typedef int kq4_v16i __attribute__((ext_vector_type(16)));

// LDS pitch of one group's CB tiles: DOT4 reads 144-B tile pairs (the unpadded pitch is
// conflict-free for them); MFMA reads one dword per lane of 8 groups at once, which needs a 16-B
// pad to spread the groups over the banks.
template <int KIND, int G8>
constexpr int kq4_gv_pitch() { return kq4_gv_cb<G8>() * 72 + (KIND == 0 ? 0 : 16); }

template <int M, int KIND, int G8>
constexpr int kq4_gv_slab() {
  return G8 * kq4_gv_pitch<KIND, G8>() + M * kq4_gv_qts<G8>() + kq4_gv_cb<G8>() * 8 * 4;
}

// Byte offset of block blk's 32 codes in a token row: block pairs at an 80-B pitch (16-B pad),
// which spreads both readers' 16-B accesses over the banks.
KQ4_DEV int kq4_gv_qpos(int blk) { return (blk >> 1) * 80 + (blk & 1) * 32; }

// B operand of one block for weight row (lane%32) from its tile's 4 nibble dwords: lanes
// 0..31 carry elements 0..15 (low nibbles), lanes 32..63 elements 16..31 (high nibbles), each
// as 16*(n-8) int8 lanes in element order.
KQ4_DEV kq4_v4i kq4_gv_bop(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int sh) {
  kq4_v4i b;
  b.x = (int)((w0 << sh) & 0xF0F0F0F0u);
  b.y = (int)((w1 << sh) & 0xF0F0F0F0u);
  b.z = (int)((w2 << sh) & 0xF0F0F0F0u);
  b.w = (int)((w3 << sh) & 0xF0F0F0F0u);
  return b;
}

KQ4_DEV kq4_v16i kq4_gv_mfma(kq4_v4i a, kq4_v4i b) {
  const kq4_v16i z = {0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

// ---- weight stage: 9216 B = 36 dwords per lane ----------------------------------------------

template <int UNIT>
struct KQ4GvStage {
  uint32_t d[36];
};

// Per-lane byte offsets of the lane's units within a stage, relative to the stage's first block
// in group g0: unit u = 64 i + lane is group gi = u / UPG at byte (u % UPG)*UNIT of that group's
// CB tiles (UPG = CB*72/UNIT units per group). Groups past the matrix end read group G-1 (in
// bounds; unused).
template <int UNIT, int G8>
struct KQ4GvOff {
  uint32_t o[9216 / UNIT / 64];
};

template <int UNIT, int G8>
KQ4_DEV void kq4_gv_offsets(KQ4GvOff<UNIT, G8> &f, int g0, int G, int nb, int lane) {
  constexpr int UPG = kq4_gv_cb<G8>() * 72 / UNIT;
  constexpr int NL = 9216 / UNIT / 64;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int u = 64 * i + lane;
    const int gi = u / UPG;
    int g = g0 + gi;
    g = g < G ? g : G - 1;
    f.o[i] = (uint32_t)g * (uint32_t)nb * 72u + (uint32_t)((u - gi * UPG) * UNIT);
  }
}

// Loads stage st. In a partial last stage, bytes past the matrix's last block read the stage's
// first block instead (in bounds; unused).
template <int UNIT, int G8>
KQ4_DEV void kq4_gv_load(KQ4GvStage<UNIT> &s, const uint8_t *__restrict__ w,
                         const KQ4GvOff<UNIT, G8> &f, int nb, int st, int lane) {
  constexpr int CB = kq4_gv_cb<G8>();
  constexpr int UPG = CB * 72 / UNIT;
  constexpr int NL = 9216 / UNIT / 64;
  const int kb = st * CB;
  const uint8_t *base = w + (size_t)kb * 72;
  const bool partial = nb - kb < CB;
  const uint32_t valid = (uint32_t)(nb - kb) * 72u;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    uint32_t off = f.o[i];
    if (partial) {
      const int u = 64 * i + lane;
      const uint32_t in = (uint32_t)((u - (u / UPG) * UPG) * UNIT);
      off = in >= valid ? off - in : off;
    }
    const uint8_t *p = base + off;
    if (UNIT == 16) {
      const uint4 v = *reinterpret_cast<const uint4 *>(p);
      s.d[4 * i] = v.x; s.d[4 * i + 1] = v.y; s.d[4 * i + 2] = v.z; s.d[4 * i + 3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2 *>(p);
      s.d[2 * i] = v.x; s.d[2 * i + 1] = v.y;
    }
  }
}

template <int UNIT, int KIND, int G8>
KQ4_DEV void kq4_gv_store(const KQ4GvStage<UNIT> &s, uint8_t *sw, int lane) {
  constexpr int UPG = kq4_gv_cb<G8>() * 72 / UNIT;
  constexpr int NL = 9216 / UNIT / 64;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int u = 64 * i + lane;
    uint8_t *p;
    if (KIND == 0) {
      p = sw + u * UNIT;                       // unpadded pitch: the stage bytes as loaded
    } else {
      const int gi = u / UPG;
      p = sw + gi * kq4_gv_pitch<KIND, G8>() + (u - gi * UPG) * UNIT;
    }
    if (UNIT == 16)
      *reinterpret_cast<uint4 *>(p) = make_uint4(s.d[4 * i], s.d[4 * i + 1], s.d[4 * i + 2], s.d[4 * i + 3]);
    else
      *reinterpret_cast<uint2 *>(p) = make_uint2(s.d[2 * i], s.d[2 * i + 1]);
  }
}

// ---- activations of a stage -------------------------------------------------------------------
// Loaded into registers together with (just before) the stage's weights, then written to the
// wave's slab as int8 codes (token row m at m*qts, block at kq4_gv_qpos) and the effective
// per-block scale sx[blk][m] = xs/16 (xs = f16-rounded xd for ASM-chain tokens; the /16 undoes the
// 16*(n-8) weight scaling exactly). Issuing them before the weights keeps the in-order load
// counter from making the quantization wait for the weights.
//
// FQ (M <= KQ4_GEMV_FQ_MAX_M): lane quad (4q .. 4q+3) owns block q (+16 per pass) for one token
// per pass, 8 fp32 each; the quantization restates quantize_row_q8_0_act
// (vllm_safetensors.c:7893-7920): d = amax/127 is a true division, x/d the Markstein-corrected
// quotient q = x*y, q += fma(-q, d, x)*y with y = RN(1/d), which is the correctly rounded x/d for
// these normal operands, so the codes are the reference's bit for bit.
// Pre-quantized: lane i copies 16-B units i, i+64, .. of the stage's codes and scales i, i+64.
template <int M, bool FQ, int G8>
struct KQ4GvAct {
  static constexpr int CB = kq4_gv_cb<G8>();
  static constexpr int NP = FQ ? M * CB / 16 : 1;              // quantization passes
  static constexpr int NQ = FQ ? 1 : (2 * CB * M + 63) / 64;   // uint4 per lane
  static constexpr int NX = FQ ? 1 : (CB * M + 63) / 64;       // scales per lane
  float4 f[FQ ? 2 * NP : 1];
  uint4 q[NQ];
  float x[NX];
};

template <int M, bool FQ, int G8>
KQ4_DEV void kq4_gv_act_load(KQ4GvAct<M, FQ, G8> &r, const KQ4GemvArgs &a, int st, int lane) {
  constexpr int CB = kq4_gv_cb<G8>();
  const int nb = a.nb, cols = a.cols;
  const int kb = st * CB;
  if (FQ) {
    const int qq = lane & 3;
#pragma unroll
    for (int p = 0; p < KQ4GvAct<M, FQ, G8>::NP; ++p) {
      const int item = (lane >> 2) + 16 * p;           // (token, block) = (item / CB, item % CB)
      const int m = item / CB, b = kb + (item - m * CB);
      if (b < nb) {
        const float4 *src =
            reinterpret_cast<const float4 *>(a.xf + (size_t)m * cols + (size_t)b * 32 + 8 * qq);
        r.f[2 * p] = src[0];
        r.f[2 * p + 1] = src[1];
      } else {
        r.f[2 * p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        r.f[2 * p + 1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, G8>::NQ; ++c) {
      const int i = lane + 64 * c;
      const int m = i / (2 * CB), u = i - m * 2 * CB, b = kb + (u >> 1), hh = u & 1;
      r.q[c] = make_uint4(0, 0, 0, 0);
      if (m < M && b < nb)
        r.q[c] = *reinterpret_cast<const uint4 *>(a.xq + (size_t)m * cols + (size_t)b * 32 + 16 * hh);
    }
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, G8>::NX; ++c) {
      const int i = lane + 64 * c;
      const int m = i / CB, b = kb + (i - m * CB);
      r.x[c] = (m < M && b < nb) ? a.xd[(size_t)m * nb + b] : 0.0f;
    }
  }
}

template <int M, bool FQ, int G8>
KQ4_DEV void kq4_gv_act_put(const KQ4GvAct<M, FQ, G8> &r, const KQ4GemvArgs &a, int lane,
                            uint8_t *sq, float (*sx)[8]) {
  constexpr int CB = kq4_gv_cb<G8>();
  constexpr int QTS = kq4_gv_qts<G8>();
  if (FQ) {
    const int qq = lane & 3;
#pragma unroll
    for (int p = 0; p < KQ4GvAct<M, FQ, G8>::NP; ++p) {
      const int item = (lane >> 2) + 16 * p;
      const int m = item / CB, blk = item - m * CB;
      const float v[8] = {r.f[2 * p].x, r.f[2 * p].y, r.f[2 * p].z, r.f[2 * p].w,
                          r.f[2 * p + 1].x, r.f[2 * p + 1].y, r.f[2 * p + 1].z, r.f[2 * p + 1].w};
      float amax = 1e-10f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      const float d = amax / 127.0f;
      const float y = 1.0f / d;
      uint32_t pk[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = v[i] * y;
        const float e = fmaf(-q, d, v[i]);
        q = fmaf(e, y, q);
        int c = (int)(q + 0.5f);
        c = c > 127 ? 127 : (c < -127 ? -127 : c);
        pk[i >> 2] |= ((uint32_t)c & 0xFFu) << (8 * (i & 3));
      }
      *reinterpret_cast<uint2 *>(sq + m * QTS + kq4_gv_qpos(blk) + 8 * qq) = make_uint2(pk[0], pk[1]);
      if (qq == 0) sx[blk][m] = ((m < a.asm_tokens) ? kq4_f16_round(d) : d) * 0.0625f;
    }
  } else {
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, G8>::NQ; ++c) {
      const int i = lane + 64 * c;
      const int m = i / (2 * CB), u = i - m * 2 * CB;
      if (m < M)
        *reinterpret_cast<uint4 *>(sq + m * QTS + kq4_gv_qpos(u >> 1) + 16 * (u & 1)) = r.q[c];
    }
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, G8>::NX; ++c) {
      const int i = lane + 64 * c;
      const int m = i / CB, blk = i - m * CB;
      if (m < M) sx[blk][m] = ((m < a.asm_tokens) ? kq4_f16_round(r.x[c]) : r.x[c]) * 0.0625f;
    }
  }
}

// ---- compute: the blocks of one stage for this wave's row set --------------------------------

// DOT4: lane (gl, j) = (lane / (CB/2), lane % (CB/2)) owns tiles (2j, 2j+1) of group gl;
// acc[r*M + m] = row (4*gl + r), token m. The pair is read one tile at a time (18 dwords).
template <int M, int G8>
KQ4_DEV void kq4_gv_dot4(const uint8_t *sw, const uint8_t *sq, const float (*sx)[8], int nblk,
                         int lane, float *acc) {
  constexpr int CB = kq4_gv_cb<G8>();
  constexpr int QTS = kq4_gv_qts<G8>();
  const int gl = lane / (CB / 2), j = lane % (CB / 2);
  const uint8_t *tp = sw + gl * (CB * 72) + j * 144;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int b = 2 * j + t;
    if (b >= nblk) break;
    uint32_t tile[18];
    if (t == 0) {   // bytes 0..71 of the pair: 16-B aligned
      const uint4 *p = reinterpret_cast<const uint4 *>(tp);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = p[i];
        tile[4 * i] = v.x; tile[4 * i + 1] = v.y; tile[4 * i + 2] = v.z; tile[4 * i + 3] = v.w;
      }
      const uint2 v = *reinterpret_cast<const uint2 *>(tp + 64);
      tile[16] = v.x; tile[17] = v.y;
    } else {        // bytes 72..143: an 8-B piece, then 16-B aligned
      const uint2 v = *reinterpret_cast<const uint2 *>(tp + 72);
      tile[0] = v.x; tile[1] = v.y;
      const uint4 *p = reinterpret_cast<const uint4 *>(tp + 80);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 u = p[i];
        tile[2 + 4 * i] = u.x; tile[3 + 4 * i] = u.y; tile[4 + 4 * i] = u.z; tile[5 + 4 * i] = u.w;
      }
    }
    float wd[4];
    wd[0] = kq4_h2f(tile[0]);
    wd[1] = kq4_h2f(tile[0] >> 16);
    wd[2] = kq4_h2f(tile[1]);
    wd[3] = kq4_h2f(tile[1] >> 16);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 *qp = reinterpret_cast<const uint4 *>(sq + m * QTS + kq4_gv_qpos(b));
      const uint4 q0 = qp[0], q1 = qp[1];
      const uint32_t qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      const float xs = sx[b][m];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t wv = tile[2 + 4 * k + r];
          s = kq4_dot4(kq4_lo16(wv), qa[k], s);
          s = kq4_dot4(kq4_hi16(wv), qa[4 + k], s);
        }
        acc[r * M + m] = fmaf((float)s, wd[r] * xs, acc[r * M + m]);
      }
    }
  }
}

// MFMA (32-row sets): acc[v] = row (lane%32), token 4*(lane/32)+v.
template <int M>
KQ4_DEV void kq4_gv_mfma_stage(const uint8_t *sw, const uint8_t *sq, const float (*sx)[8],
                               int nblk, int lane, float *acc) {
  constexpr int VT = M < 4 ? M : 4;
  constexpr int P = kq4_gv_pitch<1, 8>();
  constexpr int QTS = kq4_gv_qts<8>();
  const int j = lane & 31, h = lane >> 5;
  const int g = j >> 2, r = j & 3;
  const int t = j < M ? j : M - 1;
  const int sh = h ? 0 : 4;
  const uint8_t *wb = sw + g * P + 8 + 4 * r;
  const uint8_t *sb = sw + g * P + 2 * r;
  const uint8_t *qb = sq + t * QTS + 16 * h;
  for (int b = 0; b < nblk; ++b) {
    const uint8_t *tb = wb + b * 72;
    const kq4_v4i B = kq4_gv_bop(*reinterpret_cast<const uint32_t *>(tb),
                                 *reinterpret_cast<const uint32_t *>(tb + 16),
                                 *reinterpret_cast<const uint32_t *>(tb + 32),
                                 *reinterpret_cast<const uint32_t *>(tb + 48), sh);
    const kq4_v4i A = *reinterpret_cast<const kq4_v4i *>(qb + kq4_gv_qpos(b));
    const kq4_v16i C = kq4_gv_mfma(A, B);
    const float wd = kq4_h2f(*reinterpret_cast<const uint16_t *>(sb + b * 72));
    const float4 xs = *reinterpret_cast<const float4 *>(&sx[b][4 * h]);
    const float xv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
    for (int v = 0; v < VT; ++v) acc[v] = fmaf((float)C[v], wd * xv[v], acc[v]);
  }
}

// Sum over aligned runs of N (8 or 16) lanes of a DPP row; every lane ends with the same bits.
template <int N>
KQ4_DEV float kq4_rowN_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // quad xor 1
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // quad xor 2
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)); // half-row mirror
  if (N == 16)
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)); // row mirror
  return v;
}

template <int M, bool FQ, int UNIT, int D, int KIND, int G8>
__global__ __launch_bounds__(512) void kq4_gemv_kernel(const KQ4GemvArgs a) {
  extern __shared__ __align__(16) uint8_t kq4_gv_lds[];
  constexpr int CB = kq4_gv_cb<G8>();
  constexpr int RSZ = 4 * G8;                     // rows per row set
  constexpr int SLAB = kq4_gv_slab<M, KIND, G8>();
  constexpr int NACC = KIND == 0 ? 4 * M : 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int wg = blockIdx.x;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < KQ4_MAXMAT; ++i)
    if (i < a.nmat && wg >= a.mat[i].wg_begin) mi = i;
  const uint8_t *__restrict__ w = a.mat[mi].w;
  const int rows = a.mat[mi].rows;
  const int row0 = (wg - a.mat[mi].wg_begin) * RSZ;
  const int nb = a.nb;
  const int nst = (nb + CB - 1) / CB;
  uint8_t *slab = kq4_gv_lds + wave * SLAB;
  uint8_t *sw = slab;
  uint8_t *sq = slab + G8 * kq4_gv_pitch<KIND, G8>();
  float (*sx)[8] = reinterpret_cast<float (*)[8]>(sq + M * kq4_gv_qts<G8>());

  KQ4GvOff<UNIT, G8> off;
  kq4_gv_offsets<UNIT, G8>(off, row0 >> 2, rows >> 2, nb, lane);

  float acc[NACC];
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] = 0.0f;
  // D stages in flight per wave, each issued as (activations, weights) in stage order
  KQ4GvAct<M, FQ, G8> ra[D];
  KQ4GvStage<UNIT> rw[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int s0 = wave + d * nw;
    if (s0 < nst) {
      kq4_gv_act_load<M, FQ, G8>(ra[d], a, s0, lane);
      kq4_gv_load<UNIT, G8>(rw[d], w, off, nb, s0, lane);
    }
  }
  for (int base = wave; base < nst; base += D * nw) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int st = base + d * nw;
      if (st >= nst) break;
      kq4_gv_act_put<M, FQ, G8>(ra[d], a, lane, sq, sx);
      kq4_gv_store<UNIT, KIND, G8>(rw[d], sw, lane);
      const int sn = st + D * nw;                  // next stage for this slot
      if (sn < nst) {
        kq4_gv_act_load<M, FQ, G8>(ra[d], a, sn, lane);
        kq4_gv_load<UNIT, G8>(rw[d], w, off, nb, sn, lane);
      }
      const int nblk = nb - st * CB < CB ? nb - st * CB : CB;
      if (KIND == 0)
        kq4_gv_dot4<M, G8>(sw, sq, sx, nblk, lane, acc);
      else
        kq4_gv_mfma_stage<M>(sw, sq, sx, nblk, lane, acc);
    }
  }

  // this wave's partial sums as red[m*RSZ + row] in its slab
  float *__restrict__ out = a.mat[mi].out;
  const float *__restrict__ res = a.mat[mi].res;
  float *red = reinterpret_cast<float *>(slab);
  if (KIND == 0) {
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[i] = kq4_rowN_sum<CB / 2>(acc[i]);
  }
  if (nw > 1) __syncthreads();   // every wave is done reading its slab's weights
  if (KIND == 0) {
    if (lane % (CB / 2) == 0) {
      const int gl = lane / (CB / 2);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) red[m * RSZ + 4 * gl + r] = acc[r * M + m];
    }
  } else {
    const int j = lane & 31, h = lane >> 5;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (4 * h + v < M) red[(4 * h + v) * RSZ + j] = acc[v];
  }
  __syncthreads();
  // the waves' K partials of the row set, added in wave order
  for (int i = threadIdx.x; i < RSZ * M; i += blockDim.x) {
    const int m = i / RSZ, jj = i - m * RSZ;
    const int row = row0 + jj;
    if (row >= rows) continue;
    float s = reinterpret_cast<const float *>(kq4_gv_lds)[i];
    for (int v = 1; v < nw; ++v) s += reinterpret_cast<const float *>(kq4_gv_lds + v * SLAB)[i];
    const size_t o = (size_t)m * rows + row;
    out[o] = res ? res[o] + s : s;
  }
}

template <int M, bool FQ, int UNIT, int D, int KIND, int G8>
static hipError_t gv_launch(const KQ4GemvArgs &a, int nw, int grid, hipStream_t s) {
  const size_t lds = (size_t)nw * kq4_gv_slab<M, KIND, G8>();
  static bool attr = false;   // raise the dynamic LDS limit once per variant
  if (!attr) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&kq4_gemv_kernel<M, FQ, UNIT, D, KIND, G8>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hipLaunchKernelGGL((kq4_gemv_kernel<M, FQ, UNIT, D, KIND, G8>), dim3(grid), dim3(64 * nw), lds,
                     s, a);
  return hipGetLastError();
}

// kind 0 = DOT4 on 32-row sets, 1 = MFMA on 32-row sets, 2 = DOT4 on 16-row sets
template <int M, bool FQ>
static hipError_t gv_launch_k(const KQ4GemvArgs &a, int kind, bool u16, int depth, int nw,
                              int grid, hipStream_t s) {
#define KQ4_GV_L(KIND, G8)                                                                   \
  (depth == 2 ? (u16 ? gv_launch<M, FQ, 16, 2, KIND, G8>(a, nw, grid, s)                     \
                     : gv_launch<M, FQ, 8, 2, KIND, G8>(a, nw, grid, s))                     \
              : (u16 ? gv_launch<M, FQ, 16, 1, KIND, G8>(a, nw, grid, s)                     \
                     : gv_launch<M, FQ, 8, 1, KIND, G8>(a, nw, grid, s)))
  if (kind == 0) return KQ4_GV_L(0, 8);
  if (kind == 1) return KQ4_GV_L(1, 8);
  return KQ4_GV_L(0, 4);
#undef KQ4_GV_L
}

// In-kernel quantization exists for M <= KQ4_GEMV_FQ_MAX_M.
template <int M>
static hipError_t gv_launch_m(const KQ4GemvArgs &a, int kind, bool fq, bool u16, int depth,
                              int nw, int grid, hipStream_t s) {
  constexpr int MF = M <= KQ4_GEMV_FQ_MAX_M ? M : 1;
  if (fq) {
    if (M > KQ4_GEMV_FQ_MAX_M) return hipErrorInvalidValue;
    return gv_launch_k<MF, true>(a, kind, u16, depth, nw, grid, s);
  }
  return gv_launch_k<M, false>(a, kind, u16, depth, nw, grid, s);
}

template <int KIND, int G8>
static int slab_bytes(int n) {
  switch (n) {
    case 1: return kq4_gv_slab<1, KIND, G8>();
    case 2: return kq4_gv_slab<2, KIND, G8>();
    case 3: return kq4_gv_slab<3, KIND, G8>();
    case 4: return kq4_gv_slab<4, KIND, G8>();
    case 5: return kq4_gv_slab<5, KIND, G8>();
    case 6: return kq4_gv_slab<6, KIND, G8>();
    case 7: return kq4_gv_slab<7, KIND, G8>();
    default: return kq4_gv_slab<8, KIND, G8>();
  }
}

int kq4_gemv_slab_bytes(int n_batch, int kind) {
  return kind == 0 ? slab_bytes<0, 8>(n_batch)
                   : (kind == 1 ? slab_bytes<1, 8>(n_batch) : slab_bytes<0, 4>(n_batch));
}

int kq4_gemv_rowset(int kind) { return kind == 2 ? 16 : 32; }

int kq4_launch_gemv(const KQ4GemvArgs &a, int n_batch, int kind, int nw, int depth, int total_wg,
                    hipStream_t s) {
  if (n_batch < 1 || n_batch > KQ4_GEMV_MAX_M || total_wg <= 0 || nw < 1 || nw > 8 ||
      kind < 0 || kind > 2 || (depth != 1 && depth != 2) ||
      (size_t)nw * kq4_gemv_slab_bytes(n_batch, kind) > 160 * 1024)
    return (int)hipErrorInvalidValue;
  // 16-byte units need every group and stage start 16-byte aligned: an even block count
  bool u16 = (a.nb % 2) == 0;
  for (int i = 0; i < a.nmat; ++i) {
    u16 = u16 && ((uintptr_t)a.mat[i].w % 16) == 0;
    if ((uintptr_t)a.mat[i].w % 8) return (int)hipErrorInvalidValue;
    // per-lane offsets within a matrix are 32-bit
    if ((size_t)(a.mat[i].rows / 4) * a.nb * 72 >= ((size_t)1 << 32)) return (int)hipErrorInvalidValue;
  }
  const bool fq = a.xf != nullptr;
  hipError_t e;
  switch (n_batch) {
    case 1: e = gv_launch_m<1>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 2: e = gv_launch_m<2>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 3: e = gv_launch_m<3>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 4: e = gv_launch_m<4>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 5: e = gv_launch_m<5>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 6: e = gv_launch_m<6>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    case 7: e = gv_launch_m<7>(a, kind, fq, u16, depth, nw, total_wg, s); break;
    default: e = gv_launch_m<8>(a, kind, fq, u16, depth, nw, total_wg, s); break;
  }
  return (int)e;
}

// ---- verification: exact per-block integer sums through the GEMV's integer dots --------------
// One wave per (32-row set, block, 32-token set). S_lo / S_hi come from the MFMA kind's operand
// builder and v_mfma (zeroing the B lanes of one K half), and are checked against the DOT4 kind's
// kq4_dot4 sums of the same tile (the lane's row, first token of the set); a mismatch is written
// as INT32_MIN so the test fails.
__global__ __launch_bounds__(64) void kq4_block_sums_kernel(int32_t *__restrict__ s_lo,
                                                            int32_t *__restrict__ s_hi,
                                                            const int8_t *__restrict__ xq,
                                                            const uint8_t *__restrict__ w,
                                                            int rows, int cols, int n_batch) {
  const int nb = cols / 32;
  const int lane = threadIdx.x;
  const int j = lane & 31, h = lane >> 5;
  const int row0 = blockIdx.x * 32, b = blockIdx.y, t0 = blockIdx.z * 32;
  const int G = rows >> 2;
  int g = (row0 + j) >> 2;
  g = g < G ? g : G - 1;
  const uint8_t *tile = w + ((size_t)g * nb + b) * 72;
  const uint32_t *nib = reinterpret_cast<const uint32_t *>(tile + 8);
  const int r = j & 3;
  const uint32_t w0 = nib[r], w1 = nib[4 + r], w2 = nib[8 + r], w3 = nib[12 + r];
  const kq4_v4i B = kq4_gv_bop(w0, w1, w2, w3, h ? 0 : 4);
  const kq4_v4i Z = {0, 0, 0, 0};
  int t = t0 + j;
  t = t < n_batch ? t : n_batch - 1;
  const kq4_v4i A = *reinterpret_cast<const kq4_v4i *>(xq + (size_t)t * cols + (size_t)b * 32 + 16 * h);
  const kq4_v16i Clo = kq4_gv_mfma(A, h == 0 ? B : Z);
  const kq4_v16i Chi = kq4_gv_mfma(A, h == 1 ? B : Z);
  // the DOT4 kind's sums for (row j, token t0): lanes 0..31 compute them for their row
  const uint32_t *q = reinterpret_cast<const uint32_t *>(xq + (size_t)t0 * cols + (size_t)b * 32);
  int dlo = 0, dhi = 0;
  const uint32_t wk[4] = {w0, w1, w2, w3};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    dlo = kq4_dot4(kq4_lo16(wk[k]), q[k], dlo);
    dhi = kq4_dot4(kq4_hi16(wk[k]), q[4 + k], dhi);
  }
  const int row = row0 + j;
  if (row >= rows) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int m = t0 + 8 * (v >> 2) + 4 * h + (v & 3);
    if (m >= n_batch) continue;
    const size_t o = ((size_t)m * rows + row) * nb + b;
    int lo = Clo[v] >> 4, hi = Chi[v] >> 4;   // exact: multiples of 16
    if (m == t0 && (lo != (dlo >> 4) || hi != (dhi >> 4))) lo = hi = INT32_MIN;
    s_lo[o] = lo;
    s_hi[o] = hi;
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
