// kq4_gemm.hip - prefill GEMM over q4 weights (stream layout of VQF 4x4 tiles) x int8
// activations with int8 MFMA (gfx950).
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-element quantization block, so its int32
// result is the block sum 16*S for a 32-token x 32-row tile (weights enter the matrix core as
// 16*(n-8) bytes, see kq4_lo16/kq4_hi16). Each lane owns the same (token, row) outputs for the
// whole K loop, so the per-block fp32 epilogue replays the reference chain exactly:
//   ASM    acc = fma(S, fl(wd * f16r(xd)), acc)  (llama_gemm_q4_0_4x4_asm.c:151-161, the
//          reference's n_batch&~3 main segment, vllm_safetensors.c:4604-4609)
//   GEMV32 the same with the f32 xd (q4x4_dot1_group16_gemv :4229-4251)
//   CTILE  lo/hi accumulators fed by two half-K MFMAs, out = fl(lo + hi) (:4180-4216)
// and out = fl(residual + acc) when fused. The epilogue (convert, scale, fma per output per
// block) runs on the VALU.
// With Q8_0 weights (WF = 1, the q8 stream layout) the MFMA result is S itself and the chain is
//   Q8GEMM acc = fl(acc + fl(fl(wd * f16r(xd)) * S))  (gemm_q8_0_8x8_neon :4973-5050, unfused
//          vmlaq_f32) or GEMV32 as above (q8x8_dot_rows :5178-5225).
//
// Tiling: workgroup = 4 waves = 128 tokens x 128 rows, each wave 64 x 64 (2 x 2 MFMA tiles).
// Per stage of KB = 4 blocks the workgroup stages into LDS (rows padded to 48 B so the 16-byte
// fragment reads are bank-conflict free):
//   A  block-major activations [block][token][32] (contiguous 4 KB per block)
//   B  weights (the stream layout's half-rows, 16 B per lane-load) unpacked to 16*(n-8) int8
//      [block][row][32]
//   sW per-row scale wd/16, sX per-token activation scale
// The workgroup -> tile map keeps the tiles of one XCD (workgroup id mod 8) in one contiguous
// range, token tiles fastest, so the weight tiles a workgroup streams are shared in its L2.
#include "kq4_common.h"
#include "kq4_internal.h"
#include "../../include/kq4.h"

#include <stdlib.h>

typedef int kq4_v4i __attribute__((ext_vector_type(4)));
typedef int kq4_v16i __attribute__((ext_vector_type(16)));

#define KQ4_GEMM_KB 4
#define KQ4_LDS_ROW 48

// MFMA 32x32 output element held by (lane, register v): column = lane % 32 (weight row),
// row = 8*(v/4) + 4*(lane/32) + v%4 (token).
KQ4_DEV int kq4_mfma_tok(int v, int half) { return 8 * (v >> 2) + 4 * half + (v & 3); }

// TM / TN = MFMA token / row tiles per wave: a workgroup covers BM = 64*TM tokens x BN = 64*TN
// rows (128 x 128, or smaller when the launch would otherwise have fewer than two tiles per CU).
template <int CHAIN, int TM, int TN, int WF>
__global__ __launch_bounds__(256, 2) void kq4_gemm_kernel(
    float *__restrict__ out, const float *__restrict__ res, const uint8_t *__restrict__ w,
    const KQ4GemmAct act, int rows, int n_tok, int nb, int nst, int mtiles, int ntiles) {
  constexpr int KQ4_GEMM_BM = 64 * TM, KQ4_GEMM_BN = 64 * TN;
  __shared__ __align__(16) int8_t sA[KQ4_GEMM_KB][KQ4_GEMM_BM * KQ4_LDS_ROW];
  __shared__ __align__(16) int8_t sB[KQ4_GEMM_KB][KQ4_GEMM_BN * KQ4_LDS_ROW];
  __shared__ __align__(16) float sW[KQ4_GEMM_KB][KQ4_GEMM_BN];
  __shared__ __align__(16) float sX[KQ4_GEMM_KB][KQ4_GEMM_BM];

  // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs; give XCD x the
  // contiguous tile range [start(x), start(x) + count(x)) (a bijection for any tile count).
  const int ntile = mtiles * ntiles;
  const int wg = blockIdx.x;
  const int xcd = wg & 7, q8 = ntile >> 3, r8 = ntile & 7;
  const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + (wg >> 3);
  const int mt = tile % mtiles;
  const int nt = tile / mtiles;
  const int m0 = mt * KQ4_GEMM_BM;
  const int n0 = nt * KQ4_GEMM_BN;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, half = lane >> 5;

  float acc[TM][TN][16];
  float acc_hi[TM][TN][16];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jn = 0; jn < TN; ++jn)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        acc[i][jn][v] = 0.0f;
        acc_hi[i][jn][v] = 0.0f;
      }

  // Global -> registers for one stage (issued a whole compute phase ahead), then registers ->
  // LDS. Activations: KB blocks x 128 tokens x 32 B, 16 B per thread per block. Weights from the
  // stream layout: blocks b0 .. b0+3 are nibble units (b0%16)/2 and +1 of the 4 row sets; load
  // (set, unit, lane) = 16 B = the lane's half-row of 2 blocks, unpacked to 16*(n-8) bytes when
  // stored. Row scales (8 B per row, as wd/16) and token scales.
  // q8: per stage 4 blocks x BN rows x 2 halves of 16 B, 2*TN loads per thread
  constexpr int NB = WF ? 2 * TN : TN;
  struct Regs {
    uint4 a[KQ4_GEMM_KB];
    uint4 b[NB];
    uint2 sw;
    float x[KQ4_GEMM_KB * KQ4_GEMM_BM / 256];
  };
  auto load = [&](Regs &rg, int b0) {
#pragma unroll
    for (int u = 0; u < KQ4_GEMM_KB; ++u) {
      const int tok = t >> 1, hh = t & 1;
      const int b = b0 + u;
      rg.a[u] = make_uint4(0, 0, 0, 0);
      if (tok < KQ4_GEMM_BM && b < nb && m0 + tok < n_tok)
        rg.a[u] = *reinterpret_cast<const uint4 *>(act.xq + (long)(m0 + tok) * act.q_ts +
                                                   (long)b * act.q_bs + hh * 16);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int idx = t + 256 * u;
      if (WF) {   // (set sl, block iu of the stage, lane ln): 16 int8 codes
        const int ln = idx & 63, iu = (idx >> 6) & 3, sl = idx >> 8;
        const int rl = 32 * sl + (ln & 31), h = ln >> 5;
        rg.b[u] = make_uint4(0, 0, 0, 0);
        if (n0 + 32 * sl < rows)
          rg.b[u] = *reinterpret_cast<const uint4 *>(w + kq8_stream_code(n0 + rl, b0 + iu, h, nst));
      } else {    // (set sl, nibble unit iu = 2 blocks, lane ln)
        const int ln = idx & 63, iu = (idx >> 6) & 1, sl = idx >> 7;
        const int rl = 32 * sl + (ln & 31), h = ln >> 5;
        rg.b[u] = make_uint4(0, 0, 0, 0);          // row sets past the matrix: weight 0
        if (n0 + 32 * sl < rows)
          rg.b[u] = *reinterpret_cast<const uint4 *>(w + kq4_stream_nib(n0 + rl, b0 + 2 * iu, h, nst));
      }
    }
    rg.sw = make_uint2(0, 0);
    if (t < KQ4_GEMM_BN && n0 + (t & ~31) < rows)
      rg.sw = *reinterpret_cast<const uint2 *>(
          w + (WF ? kq8_stream_scale(n0 + t, b0, nst) : kq4_stream_scale(n0 + t, b0, nst)));
#pragma unroll
    for (int u = 0; u < KQ4_GEMM_KB * KQ4_GEMM_BM / 256; ++u) {
      const int c = t + 256 * u;
      const int bl = c / KQ4_GEMM_BM, tok = c % KQ4_GEMM_BM;
      const int b = b0 + bl;
      rg.x[u] = 0.0f;
      if (b < nb && m0 + tok < n_tok) rg.x[u] = act.xd[(long)(m0 + tok) * act.d_ts + (long)b * act.d_bs];
    }
  };
  auto store = [&](const Regs &rg) {
#pragma unroll
    for (int u = 0; u < KQ4_GEMM_KB; ++u)
      if ((t >> 1) < KQ4_GEMM_BM)
        *reinterpret_cast<uint4 *>(&sA[u][(t >> 1) * KQ4_LDS_ROW + (t & 1) * 16]) = rg.a[u];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int idx = t + 256 * u;
      if (WF) {
        const int ln = idx & 63, iu = (idx >> 6) & 3, sl = idx >> 8;
        const int rl = 32 * sl + (ln & 31), h = ln >> 5;
        *reinterpret_cast<uint4 *>(&sB[iu][rl * KQ4_LDS_ROW + 16 * h]) = rg.b[u];
      } else {
        const int ln = idx & 63, iu = (idx >> 6) & 1, sl = idx >> 7;
        const int rl = 32 * sl + (ln & 31), h = ln >> 5;
        uint32_t o[4];
        kq4_unpack_half(rg.b[u].x, rg.b[u].y, o);
        *reinterpret_cast<uint4 *>(&sB[2 * iu][rl * KQ4_LDS_ROW + 16 * h]) =
            make_uint4(o[0], o[1], o[2], o[3]);
        kq4_unpack_half(rg.b[u].z, rg.b[u].w, o);
        *reinterpret_cast<uint4 *>(&sB[2 * iu + 1][rl * KQ4_LDS_ROW + 16 * h]) =
            make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
    if (t < KQ4_GEMM_BN) {
      constexpr float WS = WF ? 1.0f : 0.0625f;   // q4 enters the MFMA as 16*(n-8)
      sW[0][t] = kq4_h2f(rg.sw.x) * WS;
      sW[1][t] = kq4_h2f(rg.sw.x >> 16) * WS;
      sW[2][t] = kq4_h2f(rg.sw.y) * WS;
      sW[3][t] = kq4_h2f(rg.sw.y >> 16) * WS;
    }
#pragma unroll
    for (int u = 0; u < KQ4_GEMM_KB * KQ4_GEMM_BM / 256; ++u) {
      const int c = t + 256 * u;
      // ASM and Q8GEMM chains: the reference multiplies by the f16-rounded activation scale
      sX[c / KQ4_GEMM_BM][c % KQ4_GEMM_BM] =
          (CHAIN == KQ4_CHAIN_ASM || CHAIN == KQ4_CHAIN_Q8GEMM) ? kq4_f16_round(rg.x[u]) : rg.x[u];
    }
  };

  // The C-tile chain keeps two accumulator sets; it has no registers left for the prefetch and
  // loads each stage just before storing it.
  constexpr bool PREFETCH = CHAIN != KQ4_CHAIN_CTILE;
  Regs rg;
  if (PREFETCH) load(rg, 0);
  for (int b0 = 0; b0 < nb; b0 += KQ4_GEMM_KB) {
    __syncthreads();              // the previous stage's compute is done with the LDS tiles
    if (!PREFETCH) load(rg, b0);
    store(rg);
    __syncthreads();
    if (PREFETCH && b0 + KQ4_GEMM_KB < nb) load(rg, b0 + KQ4_GEMM_KB);   // during the compute

    // ---- compute: per block, 2 x 2 MFMA tiles per wave + exact per-block epilogue
#pragma unroll
    for (int bl = 0; bl < KQ4_GEMM_KB; ++bl) {
      if (b0 + bl >= nb) break;
      kq4_v4i af[TM], bf[TN];
      float wdv[TN];
      float xsv[TM][16];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        af[i] = *reinterpret_cast<const kq4_v4i *>(
            &sA[bl][(32 * TM * wm + 32 * i + l32) * KQ4_LDS_ROW + 16 * half]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 x4 = *reinterpret_cast<const float4 *>(
              &sX[bl][32 * TM * wm + 32 * i + 8 * q + 4 * half]);
          xsv[i][4 * q + 0] = x4.x;
          xsv[i][4 * q + 1] = x4.y;
          xsv[i][4 * q + 2] = x4.z;
          xsv[i][4 * q + 3] = x4.w;
        }
      }
#pragma unroll
      for (int jn = 0; jn < TN; ++jn) {
        bf[jn] = *reinterpret_cast<const kq4_v4i *>(
            &sB[bl][(32 * TN * wn + 32 * jn + l32) * KQ4_LDS_ROW + 16 * half]);
        wdv[jn] = sW[bl][32 * TN * wn + 32 * jn + l32];
      }
      const kq4_v16i zero = {0};
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) {
          if (CHAIN == KQ4_CHAIN_CTILE) {
            // lane half 0 carries elements 0..15 (low nibbles), half 1 elements 16..31
            const kq4_v4i z = {0, 0, 0, 0};
            const kq4_v4i blo = half == 0 ? bf[jn] : z;
            const kq4_v4i bhi = half == 1 ? bf[jn] : z;
            const kq4_v16i clo = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], blo, zero, 0, 0, 0);
            const kq4_v16i chi = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bhi, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const float sc = wdv[jn] * xsv[i][v];
              acc[i][jn][v] = fmaf((float)clo[v], sc, acc[i][jn][v]);
              acc_hi[i][jn][v] = fmaf((float)chi[v], sc, acc_hi[i][jn][v]);
            }
          } else {
            const kq4_v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[jn], zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              if (CHAIN == KQ4_CHAIN_Q8GEMM)
                acc[i][jn][v] = acc[i][jn][v] + (wdv[jn] * xsv[i][v]) * (float)c[v];
              else
                acc[i][jn][v] = fmaf((float)c[v], wdv[jn] * xsv[i][v], acc[i][jn][v]);
            }
          }
        }
    }
  }

  // ---- epilogue: out = [res +] acc (CTILE: fl(lo + hi) first)
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jn = 0; jn < TN; ++jn) {
      const int row = n0 + 32 * TN * wn + 32 * jn + l32;
      if (row >= rows) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = m0 + 32 * TM * wm + 32 * i + kq4_mfma_tok(v, half);
        if (tok >= n_tok) continue;
        float r = acc[i][jn][v];
        if (CHAIN == KQ4_CHAIN_CTILE) r = acc[i][jn][v] + acc_hi[i][jn][v];
        const size_t o = (size_t)tok * rows + row;
        out[o] = res ? res[o] + r : r;
      }
    }
}

template <int TM, int TN>
static hipError_t gemm_launch(float *out, const float *res, const uint8_t *w,
                              const KQ4GemmAct &act, int rows, int n_tok, int nb, int nst,
                              int chain, int wf, hipStream_t s) {
  const int mtiles = (n_tok + 64 * TM - 1) / (64 * TM);
  const int ntiles = (rows + 64 * TN - 1) / (64 * TN);
  const dim3 grid((unsigned)(mtiles * ntiles));
  if (wf) {
    if (chain == KQ4_CHAIN_GEMV32)
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_GEMV32, TM, TN, 1>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles);
    else if (chain == KQ4_CHAIN_Q8GEMM)
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_Q8GEMM, TM, TN, 1>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles);
    else
      return hipErrorInvalidValue;
  } else if (chain == KQ4_CHAIN_CTILE) {
    if constexpr (TM == 2 && TN == 2) return hipErrorInvalidValue;   // capped by the planner
    else
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_CTILE, TM, TN, 0>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles);
  } else if (chain == KQ4_CHAIN_GEMV32) {
    hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_GEMV32, TM, TN, 0>), grid, dim3(256), 0, s, out,
                       res, w, act, rows, n_tok, nb, nst, mtiles, ntiles);
  } else if (chain == KQ4_CHAIN_ASM) {
    hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_ASM, TM, TN, 0>), grid, dim3(256), 0, s, out,
                       res, w, act, rows, n_tok, nb, nst, mtiles, ntiles);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The largest of the 128x128, 64x128 and 64x64 (tokens x rows) tiles that gives at least two
// tiles per CU (else 64x64). The C-tile chain (two accumulator sets) takes 64x128 at most: at
// 128x128 it needs more than 256 registers and spills. KQ4_GEMM_TILE = 1/2/3 forces one (for
// measurement; the C-tile chain still caps it).
int kq4_launch_gemm(float *out, const float *res, const uint8_t *w, const KQ4GemmAct &act,
                    int rows, int cols, int n_tok, int chain, int ncu, hipStream_t s, int wf) {
  const int nb = cols / 32;
  const int cb = wf ? KQ8_STREAM_CB : KQ4_STREAM_CB;
  const int nst = (nb + cb - 1) / cb;
  if (n_tok <= 0 || rows <= 0) return 0;
  auto tiles = [&](int bm, int bn) {
    return (long)((n_tok + bm - 1) / bm) * ((rows + bn - 1) / bn);
  };
  static const int force = [] { const char *e = getenv("KQ4_GEMM_TILE"); return e ? atoi(e) : 0; }();
  int pick = force >= 1 && force <= 3 ? force
             : tiles(128, 128) >= 2L * ncu ? 1 : (tiles(64, 128) >= 2L * ncu ? 2 : 3);
  if (chain == KQ4_CHAIN_CTILE && pick == 1) pick = 2;
  hipError_t e;
  if (pick == 1) e = gemm_launch<2, 2>(out, res, w, act, rows, n_tok, nb, nst, chain, wf, s);
  else if (pick == 2) e = gemm_launch<1, 2>(out, res, w, act, rows, n_tok, nb, nst, chain, wf, s);
  else e = gemm_launch<1, 1>(out, res, w, act, rows, n_tok, nb, nst, chain, wf, s);
  return (int)e;
}
