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
#include <type_traits>

typedef int kq4_v4i __attribute__((ext_vector_type(4)));
typedef int kq4_v16i __attribute__((ext_vector_type(16)));
typedef float kq4_v16f __attribute__((ext_vector_type(16)));
typedef float kq4_v32f __attribute__((ext_vector_type(32)));

#define KQ4_GEMM_KB 4
#define KQ4_LDS_ROW 48

// MFMA 32x32 output element held by (lane, register v): column = lane % 32 (weight row),
// row = 8*(v/4) + 4*(lane/32) + v%4 (token).
KQ4_DEV int kq4_mfma_tok(int v, int half) { return 8 * (v >> 2) + 4 * half + (v & 3); }

// Issue priority by progress through K (q8 = eighths done). Two (or three) workgroups share each CU and
// each SIMD's arbiter issues from the oldest wave first, so without this the CU's first
// workgroup runs at nearly its lone speed, its partner gets the gaps (about half its speed), and
// once the first ends the partner finishes alone at ~0.7 of the pair's throughput (Qwen3-8B
// down, M = 2048: half the workgroups end at ~235 us, the rest at ~330 us). Lowering a
// workgroup's priority as it passes 1/2, 3/4 and 7/8 of K hands the issue slots to a partner
// that is behind, so the two end closer together (graph replays, Qwen3-8B: down M = 512, split
// into 512 workgroups, 104 -> 98.5 us; down M = 2048, 512 workgroups, 330 -> 322 us; gate
// M = 2048, three rounds, 291 -> 286 us). Results do not depend on it. The launcher turns it on
// for 128 x 128 launches of whole rounds and for every pipelined 64 x 128 launch.
KQ4_DEV void kq4_prio_by_progress(int q8) {
  if (q8 < 4) __builtin_amdgcn_s_setprio(3);
  else if (q8 < 6) __builtin_amdgcn_s_setprio(2);
  else if (q8 < 7) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// TM / TN = MFMA token / row tiles per wave: a workgroup covers BM = 64*TM tokens x BN = 64*TN
// rows (128 x 128, or smaller when the launch would otherwise have fewer than two tiles per CU).
// Split K (ksplit > 1): the launch covers ksplit K slices of ks blocks (a multiple of the
// stream layout's stage, so a slice's weights start at a chunk boundary), each slice a GEMM of
// its own over blocks [s*ks, min((s+1)*ks, nb)) with the chain started at zero: slice 0 writes
// `out`, slice s > 0 writes part + (s-1)*pstride, and kq4_split_reduce_kernel adds them in slice
// order. A slice is the same kernel on offset pointers: weights + (first block / stage) chunks
// (the set stride stays nst), activations + first block, with nb the slice's block count.
template <int CHAIN, int TM, int TN, int WF>
__global__ __launch_bounds__(256, (TM == 2 && TN == 1) || (TM == 1 && TN == 2 && CHAIN != KQ4_CHAIN_CTILE) ? 3 : 2) void kq4_gemm_kernel(
    float *__restrict__ out, const float *__restrict__ res, const uint8_t *__restrict__ w,
    KQ4GemmAct act, int rows, int n_tok, int nb, int nst, int mtiles, int ntiles,
    uint32_t wbytes, int ksplit, int ks, float *__restrict__ part, long pstride, int prio) {
  constexpr int KQ4_GEMM_BM = 64 * TM, KQ4_GEMM_BN = 64 * TN;
  // ROT: the software-pipelined form (128 x 128, 128 x 64, 64 x 128; see the compute below).
  // It keeps two stages in LDS at a 32-B row pitch, the two 16-B halves of row r swapped when
  // bit 3 of r is set (so the 16-B fragment reads and the stores stay bank-conflict free
  // without padding): 2 x 36 KB at 128 x 128 (two workgroups per CU), 2 x 26 KB otherwise
  // (three). The other forms (64 x 64, and the C-tile chain) stage once at a 48-B pitch.
  constexpr bool ROT = CHAIN != KQ4_CHAIN_CTILE && (TM == 2 || TN == 2);
  constexpr int SPT = KQ4_GEMM_KB * KQ4_GEMM_BN / 256;   // ROT: row scales per thread (2 or 1)
  constexpr int PITCH = ROT ? 32 : KQ4_LDS_ROW;
  struct Stage {
    int8_t a[KQ4_GEMM_KB][KQ4_GEMM_BM * PITCH];
    int8_t b[KQ4_GEMM_KB][KQ4_GEMM_BN * PITCH];
    // 128 x 64 and 64 x 128: the raw f16 row scales (scaled when read), so that three
    // workgroups fit
    std::conditional_t<ROT && (TN == 1 || TM == 1), uint16_t, float> w[KQ4_GEMM_KB][KQ4_GEMM_BN];
    float x[KQ4_GEMM_KB][KQ4_GEMM_BM];
  };
  __shared__ __align__(16) Stage stg[ROT ? 2 : 1];
  auto &sA = stg[0].a;
  auto &sB = stg[0].b;
  auto &sW = stg[0].w;
  auto &sX = stg[0].x;

  // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs; give XCD x the
  // contiguous tile range [start(x), start(x) + count(x)) (a bijection for any tile count).
  // With split K the range runs over (slice, tile), slices slowest.
  const int ntile = mtiles * ntiles * ksplit;
  const int wg = blockIdx.x;
  const int xcd = wg & 7, q8 = ntile >> 3, r8 = ntile & 7;
  const int vtile = xcd * q8 + (xcd < r8 ? xcd : r8) + (wg >> 3);
  const int tile = vtile % (mtiles * ntiles);
  const int mt = tile % mtiles;
  const int nt = tile / mtiles;
  if (ksplit > 1) {
    const int sl = vtile / (mtiles * ntiles);
    const int k0 = sl * ks;   // a multiple of the stage's blocks
    constexpr int CBK = WF ? KQ8_STREAM_CB : KQ4_STREAM_CB;
    constexpr int CHK = WF ? KQ8_STREAM_CHUNK : KQ4_STREAM_CHUNK;
    w += (size_t)(k0 / CBK) * CHK;
    wbytes -= (uint32_t)((k0 / CBK) * CHK);
    act.xq += k0 * act.q_bs;
    act.xd += k0 * act.d_bs;
    nb = min(ks, nb - k0);
    if (sl > 0) {
      out = part + (size_t)(sl - 1) * pstride;
      res = nullptr;
    }
  }
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
    std::conditional_t<ROT && TM == 1, uint2, uint4> a[KQ4_GEMM_KB];   // 64 tokens: 8 B per thread
    uint4 b[NB];
    uint2 sw;
    float x[KQ4_GEMM_KB * KQ4_GEMM_BM / 256];
  };
  // Buffer loads (kq4_rsrc): tokens past n_tok, row sets past the matrix and blocks past nb read
  // zeros without branches. The stream layouts hold zero codes and zero scales for the blocks
  // between nb and the end of their last stage, so a stage that overhangs K contributes
  // fma(0, 0, acc) = acc (acc is never -0: it starts at +0 and RN sums are -0 only when both
  // addends are), and the compute needs no per-block bound.
  const __amdgpu_buffer_rsrc_t ra = kq4_rsrc(
      act.xq, (uint32_t)((n_tok - 1) * act.q_ts + (long)(nb - 1) * act.q_bs + 32));
  const __amdgpu_buffer_rsrc_t rx = kq4_rsrc(
      act.xd, (uint32_t)(((n_tok - 1) * act.d_ts + (long)(nb - 1) * act.d_bs + 1) * 4));
  const __amdgpu_buffer_rsrc_t rw = kq4_rsrc(w, wbytes);
  // q4 weights, and q8 weights in ROT: the offsets of a stage's loads are a per-thread part,
  // computed once here, plus
  // a wave-uniform part per stage (the buffer instructions' scalar offset), so issuing a stage's
  // loads costs no vector arithmetic (the waves' VALU issue slots are the epilogue's). Every
  // address stays inside its buffer whether or not the hardware's range check counts the scalar
  // offset: the per-thread part alone is past the end for what must read zero, and the scalar
  // part never carries an address past the end.
  //  - activations (token-major, checked by the launcher): a token past n_tok starts past its
  //    buffer's end; a block past nb (a last stage that overhangs K) is clamped to block nb-1,
  //    whose finite codes and scale meet that block's zero weights and zero scale;
  //  - weights: a row set past the matrix starts past the weights' end; the scalar part stays
  //    inside a row set's stripe of nst stages.
  uint32_t va = 0, vs = 0, vb[NB], vx[KQ4_GEMM_KB * KQ4_GEMM_BM / 256];
  int xbl[KQ4_GEMM_KB * KQ4_GEMM_BM / 256];   // wave-uniform block of the stage per scale load
  if constexpr (WF == 0 || ROT) {
    constexpr int CHUNK = WF ? KQ8_STREAM_CHUNK : KQ4_STREAM_CHUNK;
    va = ROT && TM == 1 ? (uint32_t)((m0 + (t >> 2)) * act.q_ts + (t & 3) * 8)
                        : (uint32_t)((m0 + (t >> 1)) * act.q_ts + (t & 1) * 16);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      // q4: (set sl, nibble unit iu = 2 blocks, lane ln); q8: (set sl, block iu, lane ln)
      const int idx = t + 256 * u;
      const int ln = idx & 63, iu = WF ? (idx >> 6) & 3 : (idx >> 6) & 1;
      const int sl = WF ? idx >> 8 : idx >> 7;
      const int rl = 32 * sl + (ln & 31), h = ln >> 5;
      vb[u] = (uint32_t)((size_t)((n0 + rl) >> 5) * nst * CHUNK + 1024 * iu +
                         16 * ((rl & 31) + 32 * h));
    }
    // (ROT: thread t takes the SPT scales of row t % BN from block SPT * (t / BN) on)
    const int sr = ROT ? t % KQ4_GEMM_BN : t;
    vs = (uint32_t)((size_t)((n0 + sr) >> 5) * nst * CHUNK + 8192 + 16 * (sr & 31) +
                    (ROT ? 2 * SPT * (t / KQ4_GEMM_BN) : 0));
#pragma unroll
    for (int u = 0; u < KQ4_GEMM_KB * KQ4_GEMM_BM / 256; ++u) {
      const int c = t + 256 * u;
      vx[u] = (uint32_t)((m0 + c % KQ4_GEMM_BM) * act.d_ts * 4);
      xbl[u] = __builtin_amdgcn_readfirstlane(c / KQ4_GEMM_BM);   // BM is a multiple of 64
    }
  }
  // ROT moves a stage from global memory to registers and from registers to LDS in pieces, one
  // piece between two tile epilogues of the compute (piece p after epilogue p): issued all at
  // once after a barrier, the eight waves of a CU queue 72 loads at the address unit and each
  // wave stalls there for about a tenth of the stage. Weights first (the longest way), then row
  // scales, activations, token scales. No piece branches on the thread (a branch there costs
  // the pipelined compute ~30 registers).
  constexpr int NX = KQ4_GEMM_KB * KQ4_GEMM_BM / 256;
  constexpr int NPIECE = NB + 1 + KQ4_GEMM_KB + NX;
  auto load_piece = [&](Regs &rg, int b0, int p) {
    if (p < NB) {
      rg.b[p] = kq4_bload16s(rw, vb[p], WF ? (uint32_t)((b0 >> 3) * KQ8_STREAM_CHUNK + 1024 * (b0 & 7))
                                           : (uint32_t)((b0 >> 4) * KQ4_STREAM_CHUNK +
                                                        1024 * ((b0 & 15) >> 1)));
    } else if (p == NB) {
      const uint32_t so = WF ? (uint32_t)((b0 >> 3) * KQ8_STREAM_CHUNK + 2 * (b0 & 7))
                             : (uint32_t)((b0 >> 4) * KQ4_STREAM_CHUNK +
                                          512 * ((b0 & 15) >> 3) + 2 * (b0 & 7));
      rg.sw.x = SPT == 2 ? kq4_bload4s(rw, vs, so) : kq4_bload2s(rw, vs, so);
    } else if (p < NB + 1 + KQ4_GEMM_KB) {
      const int u = p - NB - 1;
      if constexpr (ROT && TM == 1)
        rg.a[u] = kq4_bload8s(ra, va, (uint32_t)(min(b0 + u, nb - 1) * act.q_bs));
      else
        rg.a[u] = kq4_bload16s(ra, va, (uint32_t)(min(b0 + u, nb - 1) * act.q_bs));
    } else {
      const int u = p - NB - 1 - KQ4_GEMM_KB;
      rg.x[u] = __uint_as_float(
          kq4_bload4s(rx, vx[u], (uint32_t)(min(b0 + xbl[u], nb - 1) * act.d_bs * 4)));
    }
  };
  // ROT: piece p of a stage from registers into LDS stage buffer S (same piece order).
  auto swz = [](int row, int hh) { return 16 * (hh ^ ((row >> 3) & 1)); };
  auto store_piece = [&](const Regs &rg, Stage &S, int p) {
    if (p < NB && WF) {        // q8: the 16 codes as they are
      const int idx = t + 256 * p;
      const int ln = idx & 63, iu = (idx >> 6) & 3, sl = idx >> 8;
      const int rl = 32 * sl + (ln & 31), h = ln >> 5;
      *reinterpret_cast<uint4 *>(&S.b[iu][rl * PITCH + swz(rl, h)]) = rg.b[p];
    } else if (p < NB) {
      const int idx = t + 256 * p;
      const int ln = idx & 63, iu = (idx >> 6) & 1, sl = idx >> 7;
      const int rl = 32 * sl + (ln & 31), h = ln >> 5;
      uint32_t o[4];
      kq4_unpack_half(rg.b[p].x, rg.b[p].y, o);
      *reinterpret_cast<uint4 *>(&S.b[2 * iu][rl * PITCH + swz(rl, h)]) =
          make_uint4(o[0], o[1], o[2], o[3]);
      kq4_unpack_half(rg.b[p].z, rg.b[p].w, o);
      *reinterpret_cast<uint4 *>(&S.b[2 * iu + 1][rl * PITCH + swz(rl, h)]) =
          make_uint4(o[0], o[1], o[2], o[3]);
    } else if (p == NB) {      // no branch: every thread stores SPT (q4 enters as 16*(n-8))
      const int j = SPT * (t / KQ4_GEMM_BN), r = t % KQ4_GEMM_BN;
      if constexpr (TN == 1) {
        S.w[j][r] = (uint16_t)rg.sw.x;
      } else if constexpr (TM == 1) {   // raw f16 (64 x 128)
        S.w[j][r] = (uint16_t)rg.sw.x;
        S.w[j + 1][r] = (uint16_t)(rg.sw.x >> 16);
      } else {
        constexpr float WS = WF ? 1.0f : 0.0625f;
        S.w[j][r] = kq4_h2f(rg.sw.x) * WS;
        S.w[j + 1][r] = kq4_h2f(rg.sw.x >> 16) * WS;
      }
    } else if (p < NB + 1 + KQ4_GEMM_KB) {
      const int u = p - NB - 1;
      if constexpr (ROT && TM == 1) {   // BM = 64: every thread holds a quarter row (8 B)
        const int r = t >> 2;
        *reinterpret_cast<uint2 *>(&S.a[u][r * PITCH + swz(r, (t >> 1) & 1) + 8 * (t & 1)]) = rg.a[u];
      } else {                   // BM = 128: every thread holds a half row
        const int r = t >> 1;
        *reinterpret_cast<uint4 *>(&S.a[u][r * PITCH + swz(r, t & 1)]) = rg.a[u];
      }
    } else {
      const int u = p - NB - 1 - KQ4_GEMM_KB, c = t + 256 * u;
      // ASM and Q8GEMM chains: the reference multiplies by the f16-rounded activation scale
      S.x[c / KQ4_GEMM_BM][c % KQ4_GEMM_BM] =
          (CHAIN == KQ4_CHAIN_ASM || CHAIN == KQ4_CHAIN_Q8GEMM) ? kq4_f16_round(rg.x[u]) : rg.x[u];
    }
  };
  auto load = [&](Regs &rg, int b0) {
    if constexpr (!ROT) {   // (the pipelined forms stage in pieces)
      if constexpr (WF == 0) {
        if (t < 2 * KQ4_GEMM_BM) {   // a whole wave's choice
#pragma unroll
          for (int u = 0; u < KQ4_GEMM_KB; ++u)
            rg.a[u] = kq4_bload16s(ra, va, (uint32_t)(min(b0 + u, nb - 1) * act.q_bs));
        }
        const uint32_t sw = (uint32_t)((b0 >> 4) * KQ4_STREAM_CHUNK + 1024 * ((b0 & 15) >> 1));
#pragma unroll
        for (int u = 0; u < NB; ++u) rg.b[u] = kq4_bload16s(rw, vb[u], sw);
        if (t < KQ4_GEMM_BN)   // a whole wave's choice
          rg.sw = kq4_bload8s(rw, vs, (uint32_t)((b0 >> 4) * KQ4_STREAM_CHUNK +
                                                 512 * ((b0 & 15) >> 3) + 2 * (b0 & 7)));
#pragma unroll
        for (int u = 0; u < KQ4_GEMM_KB * KQ4_GEMM_BM / 256; ++u)
          rg.x[u] = __uint_as_float(
              kq4_bload4s(rx, vx[u], (uint32_t)(min(b0 + xbl[u], nb - 1) * act.d_bs * 4)));
        return;
      }
#pragma unroll
      for (int u = 0; u < KQ4_GEMM_KB; ++u) {
        const int tok = t >> 1, hh = t & 1;
        const bool ok = tok < KQ4_GEMM_BM && b0 + u < nb && m0 + tok < n_tok;
        rg.a[u] = kq4_bload16(
            ra, ok ? (uint32_t)((m0 + tok) * act.q_ts + (long)(b0 + u) * act.q_bs + hh * 16) : KQ4_OOB);
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int idx = t + 256 * u;
        uint32_t off;
        if (WF) {   // (set sl, block iu of the stage, lane ln): 16 int8 codes
          const int ln = idx & 63, iu = (idx >> 6) & 3, sl = idx >> 8;
          const int rl = 32 * sl + (ln & 31), h = ln >> 5;
          off = n0 + 32 * sl < rows ? (uint32_t)kq8_stream_code(n0 + rl, b0 + iu, h, nst) : KQ4_OOB;
        } else {    // (set sl, nibble unit iu = 2 blocks, lane ln)
          const int ln = idx & 63, iu = (idx >> 6) & 1, sl = idx >> 7;
          const int rl = 32 * sl + (ln & 31), h = ln >> 5;
          off = n0 + 32 * sl < rows ? (uint32_t)kq4_stream_nib(n0 + rl, b0 + 2 * iu, h, nst) : KQ4_OOB;
        }
        rg.b[u] = kq4_bload16(rw, off);   // row sets past the matrix: weight 0
      }
      const bool sok = t < KQ4_GEMM_BN && n0 + (t & ~31) < rows;
      const uint32_t so = (uint32_t)(WF ? kq8_stream_scale(n0 + t, b0, nst) : kq4_stream_scale(n0 + t, b0, nst));
      rg.sw = kq4_bload8(rw, sok ? so : KQ4_OOB);
#pragma unroll
      for (int u = 0; u < KQ4_GEMM_KB * KQ4_GEMM_BM / 256; ++u) {
        const int c = t + 256 * u;
        const int bl = c / KQ4_GEMM_BM, tok = c % KQ4_GEMM_BM;
        const bool ok = b0 + bl < nb && m0 + tok < n_tok;
        rg.x[u] = __uint_as_float(kq4_bload4(
            rx, ok ? (uint32_t)(((m0 + tok) * act.d_ts + (long)(b0 + bl) * act.d_bs) * 4) : KQ4_OOB));
      }
    }
  };
  auto store = [&](const Regs &rg) {
    if constexpr (!ROT) {   // (the pipelined forms stage in pieces)
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
    }
  };

  // The C-tile chain keeps two accumulator sets; it has no registers left for the prefetch and
  // loads each stage just before storing it.
  constexpr bool PREFETCH = CHAIN != KQ4_CHAIN_CTILE;
  const int lastb = (nb - 1) / KQ4_GEMM_KB * KQ4_GEMM_KB;   // the last stage's first block
  Regs rg{};
  if constexpr (ROT) {
    // Stage s is computed from LDS buffer s%2 while stage s+1 moves from registers into buffer
    // (s+1)%2 and stage s+2 from global memory into the registers, piece by piece between the
    // tile epilogues; one barrier per stage. The last stages reload the last one (unused), so
    // every issue is unconditional.
#pragma unroll
    for (int p = 0; p < NPIECE; ++p) load_piece(rg, 0, p);
#pragma unroll
    for (int p = 0; p < NPIECE; ++p) store_piece(rg, stg[0], p);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < NPIECE; ++p) load_piece(rg, min(KQ4_GEMM_KB, lastb), p);
    // (unrolled by two stages, so that each buffer's LDS addresses are constants)
    auto stage = [&](Stage &C, Stage &N, int b0) __attribute__((always_inline)) {
      const int bn = min(b0 + 2 * KQ4_GEMM_KB, lastb);
      // Software-pipelined over the stage's blocks, tiles in the order q = NT*bl + k: the
      // integer MFMA of tile q+1 is issued before tile q's epilogue (two sum slots alternate),
      // and a row tile's scale products for the next block are issued right after that row
      // tile's second (last) epilogue of the current block. Each MFMA result is first read one
      // or two tile epilogues (32 VALU instructions each) after its issue, so the matrix core's
      // latency hides behind the wave's own VALU work (2.5 % at M = 2048 against the in-order
      // form); scheduling barriers keep that order. With one token tile (64 x 128) one scale
      // set serves both row tiles of a block and is reissued after the block's last epilogue
      // (a second set, to issue it earlier, would cost the third wave per SIMD).
      constexpr int NT = TM * TN;             // MFMA tiles per wave and block: k = i + TM * jn
      constexpr int NQ = KQ4_GEMM_KB * NT;
      kq4_v4i af[TM], bf[TN];
      float xv, wv[TN];
      kq4_v16i sacc[2];
      kq4_v32f sc[TM == 2 ? TN : 1];
      const kq4_v16i zero = {0};
      const kq4_v32f z32 = {0};
      auto frag_ab = [&](int bl) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const kq4_v4i *>(
              &C.a[bl][(32 * TM * wm + 32 * i + l32) * PITCH + swz(l32, half)]);
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
          bf[jn] = *reinterpret_cast<const kq4_v4i *>(
              &C.b[bl][(32 * TN * wn + 32 * jn + l32) * PITCH + swz(l32, half)]);
      };
      auto frag_s = [&](int bl) {
        if constexpr (TM == 1) {   // the outer product's two blocks are the wave's row tiles
          xv = C.x[bl][32 * wm + l32];
          wv[0] = kq4_h2f(C.w[bl][32 * TN * wn + lane]) * (WF ? 1.0f : 0.0625f);
          return;
        }
        xv = C.x[bl][64 * wm + lane];
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) {
          if constexpr (TN == 1)   // q4 enters the MFMA as 16*(n-8): wd/16 (exact)
            wv[jn] = kq4_h2f(C.w[bl][32 * TN * wn + 32 * jn + l32]) * (WF ? 1.0f : 0.0625f);
          else
            wv[jn] = C.w[bl][32 * TN * wn + 32 * jn + l32];
        }
      };
      // Scale products fl(wd * xs) from the matrix core: v_mfma_f32_32x32x1_2b_f32 is a rank-1
      // update of two 32 x 32 blocks, each output one product rounded once (with a zero
      // addend), in the MFMA output layout; its blocks are the two token tiles of row tile jn
      // (one token tile: the wave's two row tiles, one product set for both).
      auto issue_sc = [&](int jn) {
        if constexpr (TM == 1) sc[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(xv, wv[0], z32, 0, 0, 0);
        else sc[jn] = __builtin_amdgcn_mfma_f32_32x32x1f32(xv, wv[jn], z32, 0, 0, 0);
      };
      auto issue_s = [&](int q) {
        const int k = q % NT;
        sacc[q & 1] =
            __builtin_amdgcn_mfma_i32_32x32x32_i8(af[k % TM], bf[k / TM], zero, 0, 0, 0);
      };
      auto epi = [&](int q) {
        const int k = q % NT, i = k % TM, jn = k / TM;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float s = TM == 2 ? sc[TM == 2 ? jn : 0][16 * i + v] : sc[0][16 * jn + v];
          if (CHAIN == KQ4_CHAIN_Q8GEMM)   // unfused: fl(acc + fl(scale * S))
            acc[i][jn][v] = acc[i][jn][v] + s * (float)sacc[q & 1][v];
          else
            acc[i][jn][v] = fmaf((float)sacc[q & 1][v], s, acc[i][jn][v]);
        }
      };
      frag_s(0);
      frag_ab(0);
#pragma unroll
      for (int jn = 0; jn < (TM == 2 ? TN : 1); ++jn) issue_sc(jn);
      issue_s(0);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int bl = q / NT, k = q % NT;
        __builtin_amdgcn_sched_barrier(0);
        if (k == 0 && bl + 1 < KQ4_GEMM_KB) frag_s(bl + 1);
        if (q + 1 < NQ) {
          issue_s(q + 1);
          // the fragments of tile q+1's block are done with once its block's last tile is issued
          if ((q + 1) % NT == NT - 1 && (q + 1) / NT + 1 < KQ4_GEMM_KB) frag_ab((q + 1) / NT + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        epi(q);
        __builtin_amdgcn_sched_barrier(0);
        if (bl + 1 < KQ4_GEMM_KB && (k & 1)) issue_sc(k >> 1);
        if constexpr (NPIECE <= NQ) {   // one piece after each of the first NPIECE epilogues
          if (q < NPIECE) {
            store_piece(rg, N, q);
            load_piece(rg, bn, q);
          }
        } else {                         // (q8, one row tile: 9 pieces over 8 epilogues)
#pragma unroll
          for (int pc = q * NPIECE / NQ; pc < (q + 1) * NPIECE / NQ; ++pc) {
            store_piece(rg, N, pc);
            load_piece(rg, bn, pc);
          }
        }
      }
      __syncthreads();
    };
    for (int b0 = 0; b0 < nb; b0 += 2 * KQ4_GEMM_KB) {
      if (prio) kq4_prio_by_progress(8 * b0 / nb);
      stage(stg[0], stg[1], b0);
      if (b0 + KQ4_GEMM_KB < nb) stage(stg[1], stg[0], b0 + KQ4_GEMM_KB);
    }
  } else {
    if (PREFETCH) load(rg, 0);
    for (int b0 = 0; b0 < nb; b0 += KQ4_GEMM_KB) {
      __syncthreads();              // the previous stage's compute is done with the LDS tiles
      if (!PREFETCH) load(rg, b0);
      store(rg);
      __syncthreads();
      if (PREFETCH && b0 + KQ4_GEMM_KB < nb) load(rg, b0 + KQ4_GEMM_KB);   // during the compute

      // ---- compute: per block, TM x TN MFMA tiles per wave + exact per-block epilogue
#pragma unroll
      for (int bl = 0; bl < KQ4_GEMM_KB; ++bl) {
        kq4_v4i af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const kq4_v4i *>(
              &sA[bl][(32 * TM * wm + 32 * i + l32) * KQ4_LDS_ROW + 16 * half]);
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
          bf[jn] = *reinterpret_cast<const kq4_v4i *>(
              &sB[bl][(32 * TN * wn + 32 * jn + l32) * KQ4_LDS_ROW + 16 * half]);
        // Scale products fl(wd * xs) from the matrix core: v_mfma_f32_32x32x1_2b_f32 is a rank-1
        // update of two 32 x 32 blocks, each output one product rounded once (with a zero
        // addend), in the MFMA output layout. With two token tiles its blocks are the tiles of
        // one row tile (one product set per jn); with one token tile they are the two row tiles.
        const kq4_v32f z32 = {0};
        kq4_v32f sc[TM == 2 ? TN : 1];
        if constexpr (TM == 2) {
          const float xv = sX[bl][64 * wm + lane];
#pragma unroll
          for (int jn = 0; jn < TN; ++jn)
            sc[jn] = __builtin_amdgcn_mfma_f32_32x32x1f32(
                xv, sW[bl][32 * TN * wn + 32 * jn + l32], z32, 0, 0, 0);
        } else {
          const float xv = sX[bl][32 * wm + l32];
          const float wv = sW[bl][32 * TN * wn + (TN == 2 ? lane : l32)];
          sc[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(xv, wv, z32, 0, 0, 0);
        }
        const kq4_v16i zero = {0};
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jn = 0; jn < TN; ++jn) {
            auto cs = [&](int v) {
              if constexpr (TM == 2) return sc[jn % (TM == 2 ? TN : 1)][16 * i + v];
              else return sc[0][16 * jn + v];
            };
            if (CHAIN == KQ4_CHAIN_CTILE) {
              // lane half 0 carries elements 0..15 (low nibbles), half 1 elements 16..31
              const kq4_v4i z = {0, 0, 0, 0};
              const kq4_v4i blo = half == 0 ? bf[jn] : z;
              const kq4_v4i bhi = half == 1 ? bf[jn] : z;
              const kq4_v16i clo = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], blo, zero, 0, 0, 0);
              const kq4_v16i chi = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bhi, zero, 0, 0, 0);
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                acc[i][jn][v] = fmaf((float)clo[v], cs(v), acc[i][jn][v]);
                acc_hi[i][jn][v] = fmaf((float)chi[v], cs(v), acc_hi[i][jn][v]);
              }
            } else {
              const kq4_v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[jn], zero, 0, 0, 0);
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                if (CHAIN == KQ4_CHAIN_Q8GEMM)
                  acc[i][jn][v] = acc[i][jn][v] + cs(v) * (float)c[v];
                else
                  acc[i][jn][v] = fmaf((float)c[v], cs(v), acc[i][jn][v]);
              }
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

// ---- fp8 formulation (ASM and GEMV32 chains over q4 weights) -----------------------------
// The block sums come from v_mfma_f32_32x32x64_f8f6f4 on exactly representable integers (see
// kq4_common.h): A = the activations' operand pairs [16*qh | ql] (64 e4m3 bytes per token and
// block, written by the quantizer), B = [w | w] (the weights' 32 e4m3 bytes, read by both lane
// halves), so the MFMA's fp32 result is S itself, exact; the scale products fl(wd * xs) of a
// 32 x 32 tile come from v_mfma_f32_32x32x1_2b_f32 as outer products (one product per output,
// rounded once: exactly the VALU's fl(wd * xs)); each output then takes one fma per block:
// acc = fma(S, fl(wd * xs), acc), the same chain as the int8 kernel above, bit for bit. One
// 32 x 32 tile per block costs 64 + 32 matrix-core cycles and 16 VALU fmas, against 32 and 48
// (convert, product, fma) for the int8 form, so the VALU no longer bounds the kernel.
// Stages of 2 blocks, double-buffered in LDS (one barrier per stage): activations 64 B per
// (token, block) at an 80-B pitch, weights unpacked to e4m3 when stored (kq4_e4m3_nib4) at a
// 48-B pitch, f32 row and token scales.
#define KQ4_F8_KB 2
#define KQ4_F8_AP 80
#define KQ4_F8_BP 48

typedef int kq4_v8i __attribute__((ext_vector_type(8)));
KQ4_DEV kq4_v8i kq4_lds8(const uint8_t *p) {
  const uint4 u0 = *reinterpret_cast<const uint4 *>(p);
  const uint4 u1 = *reinterpret_cast<const uint4 *>(p + 16);
  return kq4_v8i{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w,
                 (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
}

template <int CHAIN, int TM, int TN>
__global__ __launch_bounds__(256, 2) void kq4_gemm_f8_kernel(
    float *__restrict__ out, const float *__restrict__ res, const uint8_t *__restrict__ w,
    const uint8_t *__restrict__ xp, const float *__restrict__ xd, int rows, int n_tok, int nb,
    int nst, int mtiles, int ntiles, long wbytes) {
  constexpr int BM = 64 * TM, BN = 64 * TN;
  constexpr int NA = BM / 32;   // 16-B activation pieces per thread and stage
  __shared__ __align__(16) uint8_t sA[2][KQ4_F8_KB][BM * KQ4_F8_AP];
  __shared__ __align__(16) uint8_t sB[2][KQ4_F8_KB][BN * KQ4_F8_BP];
  __shared__ __align__(16) float sX[2][KQ4_F8_KB][BM];
  __shared__ __align__(16) float sW[2][KQ4_F8_KB][BN];

  // XCD-aware tile order, as the int8 kernel
  const int ntile = mtiles * ntiles;
  const int wg = blockIdx.x;
  const int xcd = wg & 7, q8 = ntile >> 3, r8 = ntile & 7;
  const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + (wg >> 3);
  const int m0 = (tile % mtiles) * BM;
  const int n0 = (tile / mtiles) * BN;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, half = lane >> 5;

  float acc[TM][TN][16];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  struct Regs {
    uint4 a[NA];
    uint4 b;
    uint32_t sw;
    float x0, x1;
  };
  // global -> registers for the stage at block b0 (even): activation pieces (token idx >> 3,
  // block (idx >> 2) & 1, 16-B piece idx & 3); one stream-layout unit per thread of the first
  // 2 * BN (row set t >> 6, lane t & 63: the half-row of blocks b0 and b0 + 1); row scales (the
  // two f16 of blocks b0, b0 + 1, adjacent) for t < BN, token scales for t in [128, 128 + BM)
  // Buffer loads (kq4_rsrc): tokens past n_tok, rows past the matrix and the block past an odd
  // nb read zeros without branches.
  const __amdgpu_buffer_rsrc_t ra = kq4_rsrc(xp, (uint32_t)((size_t)n_tok * nb * 64));
  const __amdgpu_buffer_rsrc_t rw = kq4_rsrc(w, (uint32_t)wbytes);
  const __amdgpu_buffer_rsrc_t rx = kq4_rsrc(xd, (uint32_t)((size_t)n_tok * nb * 4));
  auto load = [&](Regs &rg, int b0) {
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int idx = t + 256 * u;
      const int tok = idx >> 3, bl = (idx >> 2) & 1, pc = idx & 3;
      const uint32_t off =
          b0 + bl < nb ? ((uint32_t)(m0 + tok) * nb + b0 + bl) * 64u + 16u * pc : KQ4_OOB;
      rg.a[u] = kq4_bload16(ra, off);
    }
    rg.b = kq4_bload16(rw, t < 2 * BN ? (uint32_t)kq4_stream_nib(n0 + 32 * (t >> 6) + (lane & 31),
                                                                  b0, lane >> 5, nst)
                                       : KQ4_OOB);
    rg.sw = kq4_bload4(rw, t < BN ? (uint32_t)kq4_stream_scale(n0 + t, b0, nst) : KQ4_OOB);
    const int tok = t - 128;
    const uint32_t xo = ((uint32_t)(m0 + tok) * nb + b0) * 4u;
    const bool xt = t >= 128 && t < 128 + BM;
    rg.x0 = __uint_as_float(kq4_bload4(rx, xt ? xo : KQ4_OOB));
    rg.x1 = __uint_as_float(kq4_bload4(rx, xt && b0 + 1 < nb ? xo + 4 : KQ4_OOB));
  };
  auto store = [&](const Regs &rg, int buf) {
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int idx = t + 256 * u;
      const int tok = idx >> 3, bl = (idx >> 2) & 1, pc = idx & 3;
      *reinterpret_cast<uint4 *>(&sA[buf][bl][tok * KQ4_F8_AP + 16 * pc]) = rg.a[u];
    }
    if (t < 2 * BN) {
      const int row = 32 * (t >> 6) + (lane & 31), h = lane >> 5;
      // dword d of a block's half-row: low nibbles = elements 8d .. 8d+3, high = 8d+4 .. 8d+7
      const uint32_t d[4] = {rg.b.x, rg.b.y, rg.b.z, rg.b.w};
#pragma unroll
      for (int bl = 0; bl < 2; ++bl) {
        uint4 o;
        o.x = kq4_e4m3_nib4(d[2 * bl] & 0x0F0F0F0Fu);
        o.y = kq4_e4m3_nib4((d[2 * bl] >> 4) & 0x0F0F0F0Fu);
        o.z = kq4_e4m3_nib4(d[2 * bl + 1] & 0x0F0F0F0Fu);
        o.w = kq4_e4m3_nib4((d[2 * bl + 1] >> 4) & 0x0F0F0F0Fu);
        *reinterpret_cast<uint4 *>(&sB[buf][bl][row * KQ4_F8_BP + 16 * h]) = o;
      }
    }
    if (t < BN) {
      sW[buf][0][t] = kq4_h2f(rg.sw);
      sW[buf][1][t] = kq4_h2f(rg.sw >> 16);
    } else if (t >= 128 && t < 128 + BM) {
      // ASM chain: the reference multiplies by the f16-rounded activation scale
      sX[buf][0][t - 128] = CHAIN == KQ4_CHAIN_ASM ? kq4_f16_round(rg.x0) : rg.x0;
      sX[buf][1][t - 128] = CHAIN == KQ4_CHAIN_ASM ? kq4_f16_round(rg.x1) : rg.x1;
    }
  };
  auto compute = [&](int buf, int b0) {
#pragma unroll
    for (int bl = 0; bl < KQ4_F8_KB; ++bl) {
      if (b0 + bl >= nb) break;
      kq4_v8i a[TM], bq[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = kq4_lds8(&sA[buf][bl][(32 * TM * wm + 32 * i + l32) * KQ4_F8_AP + 32 * half]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bq[j] = kq4_lds8(&sB[buf][bl][(32 * TN * wn + 32 * j + l32) * KQ4_F8_BP]);
      const kq4_v32f z32 = {0};
      const kq4_v16f z16 = {0};
      if constexpr (TM == 2) {
        // the outer product's two blocks are the wave's two token tiles (lanes 0-31, 32-63)
        const float xv = sX[buf][bl][64 * wm + lane];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const float wv = sW[buf][bl][32 * TN * wn + 32 * j + l32];
          const kq4_v32f c = __builtin_amdgcn_mfma_f32_32x32x1f32(xv, wv, z32, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const kq4_v16f sb =
                __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], bq[j], z16, 0, 0, 0, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(sb[v], c[16 * i + v], acc[i][j][v]);
          }
        }
      } else {
        // one token tile: the outer product's two blocks are the wave's row tiles
        const float xv = sX[buf][bl][32 * wm + l32];
        const float wv = sW[buf][bl][32 * TN * wn + (TN == 2 ? lane : l32)];
        const kq4_v32f c = __builtin_amdgcn_mfma_f32_32x32x1f32(xv, wv, z32, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const kq4_v16f sb =
              __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[0], bq[j], z16, 0, 0, 0, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[0][j][v] = fmaf(sb[v], c[16 * j + v], acc[0][j][v]);
        }
      }
    }
  };

  Regs rg;
  load(rg, 0);
  store(rg, 0);
  __syncthreads();
  int buf = 0;
  for (int b0 = 0; b0 < nb; b0 += KQ4_F8_KB) {
    const bool more = b0 + KQ4_F8_KB < nb;
    if (more) load(rg, b0 + KQ4_F8_KB);   // in flight during the compute
    compute(buf, b0);
    if (more) store(rg, buf ^ 1);         // the other buffer: nobody reads it this stage
    __syncthreads();
    buf ^= 1;
  }

  // out = [res +] acc
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int row = n0 + 32 * TN * wn + 32 * j + l32;
      if (row >= rows) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = m0 + 32 * TM * wm + 32 * i + kq4_mfma_tok(v, half);
        if (tok >= n_tok) continue;
        const size_t o = (size_t)tok * rows + row;
        out[o] = res ? res[o] + acc[i][j][v] : acc[i][j][v];
      }
    }
}

template <int TM, int TN>
static hipError_t gemm_f8_launch(float *out, const float *res, const uint8_t *w, const uint8_t *xp,
                                 const float *xd, int rows, int n_tok, int nb, int nst, int chain,
                                 hipStream_t s) {
  const int mtiles = (n_tok + 64 * TM - 1) / (64 * TM);
  const int ntiles = (rows + 64 * TN - 1) / (64 * TN);
  const dim3 grid((unsigned)(mtiles * ntiles));
  const long wbytes = (long)kq4_stream_bytes(rows, nb * 32);
  if (chain == KQ4_CHAIN_ASM)
    hipLaunchKernelGGL((kq4_gemm_f8_kernel<KQ4_CHAIN_ASM, TM, TN>), grid, dim3(256), 0, s, out, res,
                       w, xp, xd, rows, n_tok, nb, nst, mtiles, ntiles, wbytes);
  else if (chain == KQ4_CHAIN_GEMV32)
    hipLaunchKernelGGL((kq4_gemm_f8_kernel<KQ4_CHAIN_GEMV32, TM, TN>), grid, dim3(256), 0, s, out,
                       res, w, xp, xd, rows, n_tok, nb, nst, mtiles, ntiles, wbytes);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

int kq4_launch_gemm_f8(float *out, const float *res, const uint8_t *w, const uint8_t *xp,
                       const float *xd, int rows, int cols, int n_tok, int chain, int ncu,
                       hipStream_t s, int tile) {
  const int nb = cols / 32;
  const int nst = (nb + KQ4_STREAM_CB - 1) / KQ4_STREAM_CB;
  if (n_tok <= 0 || rows <= 0) return 0;
  if (chain != KQ4_CHAIN_ASM && chain != KQ4_CHAIN_GEMV32) return (int)hipErrorInvalidValue;
  // 32-bit buffer offsets: operand pairs and weights below 4 GB
  if (((size_t)n_tok + 128) * nb * 64 >= KQ4_OOB || kq4_stream_bytes(rows, cols) >= KQ4_OOB)
    return (int)hipErrorInvalidValue;
  auto tiles = [&](int bm, int bn) {
    return (long)((n_tok + bm - 1) / bm) * ((rows + bn - 1) / bn);
  };
  // tile: 1 / 2 / 3 / 4 = 128x128 / 64x128 / 64x64 / 128x64 (tokens x rows), as the int8 form
  const int pick = tile >= 1 && tile <= 4 ? tile
                   : tiles(128, 128) >= 2L * ncu ? 1 : (tiles(64, 128) >= 2L * ncu ? 2 : 3);
  hipError_t e;
  if (pick == 1) e = gemm_f8_launch<2, 2>(out, res, w, xp, xd, rows, n_tok, nb, nst, chain, s);
  else if (pick == 2) e = gemm_f8_launch<1, 2>(out, res, w, xp, xd, rows, n_tok, nb, nst, chain, s);
  else if (pick == 4) e = gemm_f8_launch<2, 1>(out, res, w, xp, xd, rows, n_tok, nb, nst, chain, s);
  else e = gemm_f8_launch<1, 1>(out, res, w, xp, xd, rows, n_tok, nb, nst, chain, s);
  return (int)e;
}

// out[i] = [res[i] +] (..((out[i] + part[0][i]) + part[1][i]) .. + part[np-1][i]): the K
// slices' outputs added in slice order, 4 floats per thread (n4 = elements / 4).
__global__ __launch_bounds__(256) void kq4_split_reduce_kernel(float *__restrict__ out,
                                                               const float *__restrict__ res,
                                                               const float *__restrict__ part,
                                                               int np, long pstride, long n4) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  float4 v = reinterpret_cast<const float4 *>(out)[i];
  for (int p = 0; p < np; ++p) {
    const float4 q = reinterpret_cast<const float4 *>(part + (size_t)p * pstride)[i];
    v.x = v.x + q.x;
    v.y = v.y + q.y;
    v.z = v.z + q.z;
    v.w = v.w + q.w;
  }
  if (res) {
    const float4 r = reinterpret_cast<const float4 *>(res)[i];
    v.x = r.x + v.x;
    v.y = r.y + v.y;
    v.z = r.z + v.z;
    v.w = r.w + v.w;
  }
  reinterpret_cast<float4 *>(out)[i] = v;
}

template <int TM, int TN>
static hipError_t gemm_launch(float *out, const float *res, const uint8_t *w,
                              const KQ4GemmAct &act, int rows, int n_tok, int nb, int nst,
                              int chain, int wf, uint32_t wbytes, hipStream_t s, int ksplit = 1,
                              int ks = 0, float *part = nullptr, long pstride = 0, int prio = 0) {
  const int mtiles = (n_tok + 64 * TM - 1) / (64 * TM);
  const int ntiles = (rows + 64 * TN - 1) / (64 * TN);
  const dim3 grid((unsigned)(mtiles * ntiles * ksplit));
  if (wf) {
    if (chain == KQ4_CHAIN_GEMV32)
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_GEMV32, TM, TN, 1>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles, wbytes, ksplit, ks,
                         part, pstride, prio);
    else if (chain == KQ4_CHAIN_Q8GEMM)
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_Q8GEMM, TM, TN, 1>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles, wbytes, ksplit, ks,
                         part, pstride, prio);
    else
      return hipErrorInvalidValue;
  } else if (chain == KQ4_CHAIN_CTILE) {
    if constexpr (TM == 2) return hipErrorInvalidValue;   // capped by the planner
    else
      hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_CTILE, TM, TN, 0>), grid, dim3(256), 0, s,
                         out, res, w, act, rows, n_tok, nb, nst, mtiles, ntiles, wbytes, ksplit, ks,
                         part, pstride, prio);
  } else if (chain == KQ4_CHAIN_GEMV32) {
    hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_GEMV32, TM, TN, 0>), grid, dim3(256), 0, s, out,
                       res, w, act, rows, n_tok, nb, nst, mtiles, ntiles, wbytes, ksplit, ks, part,
                       pstride, prio);
  } else if (chain == KQ4_CHAIN_ASM) {
    hipLaunchKernelGGL((kq4_gemm_kernel<KQ4_CHAIN_ASM, TM, TN, 0>), grid, dim3(256), 0, s, out,
                       res, w, act, rows, n_tok, nb, nst, mtiles, ntiles, wbytes, ksplit, ks, part,
                       pstride, prio);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Blocks per K slice for ksplit slices: ceil(nb / ksplit) rounded up to whole stream-layout
// stages; 0 when ksplit slices of that length do not all hold blocks.
static int split_len(int nb, int cb, int ksplit) {
  if (ksplit < 2) return nb;
  const int ks = ((nb + ksplit - 1) / ksplit + cb - 1) / cb * cb;
  return (long)(ksplit - 1) * ks < nb ? ks : 0;
}

// The planner. A launch runs in rounds of workgroups, two per CU for the 128 x 128 form and three
// for the 64-token forms (their LDS rings and registers), so it chooses the form that fills its
// rounds best, splitting K where the tiles alone leave CUs idle:
//   * 128 x 128 tiles from two per CU;
//   * K split over 128 x 128 tiles (KA: fewer tiles than CUs, K >= 256 blocks): the most slices
//     of >= 64 blocks with slices x tiles <= two per CU (Qwen3-8B down at M = 512: 128 tiles,
//     4 slices of 96 blocks, 512 workgroups, one whole round);
//   * K split over 64-token tiles (KB: K >= 128 blocks, 64 x 64 tiles for one token tile, else
//     64 x 128): the most slices (<= 8) of >= 32 blocks with slices x tiles <= three per CU;
//     taken over KA where it fills more of its round (Qwen3-8B down at M = 768: KA 384 of 512,
//     KB 768 of 768 workgroups, 145 -> 123 us; at M = 512 and 1024 both fill one round and KA
//     stays) and in place of the unsplit forms below (gate, K = 4096, M = 64 / 128 / 256: 64 x 64
//     tiles unsplit 34.6 / 43.3 / 54.3 us, KB 24.7 / 35.4 / 51.2 us; down at M = 32-128 39-44 ->
//     25-34 us); for 64-127 blocks (K = 2048-4064) over 64 x 64 tiles only, up to 4 slices of
//     >= 16 blocks while the tiles are at most one per two CUs (Qwen3-VL-2B QKV 4096 x 2048 at
//     M = 24: 19.1 -> 12.2 us, O 2048 x 2048 at M = 128: 19.3 -> 13.0 us; the gate, 6144 rows,
//     at M = 128: 192 tiles, split no faster);
//   * unsplit, K >= 128 blocks and more 128 x 128 tiles than CUs: 64 x 128 (three workgroups
//     per CU, progress priority) when 0.82 of its rounds is fewer than 128 x 128's rounds of
//     two per CU, else 128 x 128 (Qwen3-8B, graph replays, 128 x 128 / 64 x 128 µs: gate M = 768
//     138.5 / 117.9, M = 1536 218.7 / 203.0, M = 2048 264 / 274; QKV M = 1536 139.6 / 119.4;
//     down M = 1152 / 1536 (64 x 128 one round) 257.9 / 264.5 against 192.9 / 218.0, where the
//     128 x 64 form this replaced took 246.6 / 263.8; down M = 1792 271.3 / 305.4);
//   * else 64 x 128 from one tile per CU for K >= 128 blocks (Qwen3-8B gate at M = 320: 74.3 us
//     as 64 x 64, 59.1 us as 64 x 128), from two per CU for shorter K (Qwen3-VL-2B gate,
//     K = 2048, at M = 384: 30.5 us as 64 x 64, 33.2 us as 64 x 128), else 64 x 64.
// The C-tile chain (two accumulator sets) takes 64 x 128 at most (at 128 x 128 it spills) and
// is never split by the planner. The options force a tile and / or a slice count (the planner
// then picks the other part for it). Every planner split keeps its partial sums within
// KQ4_SPLIT_PART_MAX (24 MiB, what the workspace reserves beyond 8 tokens).
KQ4GemmPlan kq4_gemm_plan(int n_tok, int rows, int cols, int wf, int chain, int ncu,
                          int force_tile, int force_split) {
  KQ4GemmPlan p{3, 1};
  if (n_tok <= 0 || rows <= 0 || cols <= 0) return p;
  const int nb = cols / 32;
  const int cb = wf ? KQ8_STREAM_CB : KQ4_STREAM_CB;
  const long cu = ncu < 1 ? 1 : (ncu < 256 ? ncu : 256);
  auto tiles = [&](int t) {
    const int bm = t == 1 || t == 4 ? 128 : 64, bn = t == 3 || t == 4 ? 64 : 128;
    return (long)((n_tok + bm - 1) / bm) * ((rows + bn - 1) / bn);
  };
  // the most slices of >= minb blocks with slices x tiles <= cap whose partial sums fit the
  // workspace's KQ4_SPLIT_PART_MAX
  auto most = [&](long t, long cap, int minb) {
    for (int k = KQ4_GEMM_SPLIT_MAX; k >= 2; --k)
      if (k * t <= cap && split_len(nb, cb, k) >= minb &&
          (long)(k - 1) * n_tok * rows * 4 <= (long)KQ4_SPLIT_PART_MAX)
        return k;
    return 1;
  };
  const bool ctile = chain == KQ4_CHAIN_CTILE;
  const bool shortk = nb >= 64 && nb < 128;
  const int tb = n_tok <= 64 || shortk ? 3 : 2;                 // KB's tile
  const int ka = !ctile && tiles(1) <= cu && nb >= 256 ? most(tiles(1), 2 * cu, 64) : 1;
  const int kb = ctile                                ? 1
                 : nb >= 128                          ? most(tiles(tb), 3 * cu, 32)
                 : shortk && 2 * tiles(3) <= cu ? most(tiles(3), 2 * cu, 16)
                                                      : 1;
  // forced slices: 0 / 1 none; counts the blocks do not allow are taken as none
  int fk = force_split;
  if (fk >= 0 && (fk <= 1 || fk > KQ4_GEMM_SPLIT_MAX || !split_len(nb, cb, fk))) fk = 1;
  if (force_tile >= 1 && force_tile <= 4) {
    p.tile = force_tile;
    p.ksplit = fk >= 1 ? fk : force_tile == 1 ? ka : force_tile == tb ? kb : 1;
  } else if (fk > 1) {
    p = KQ4GemmPlan{1, fk};
  } else if (fk < 0 && ka > 1 && ka * tiles(1) * 3 >= kb * tiles(tb) * 2) {
    p = KQ4GemmPlan{1, ka};   // KA fills as much of its round as KB
  } else if (fk < 0 && kb > 1 && tiles(1) < 2 * cu) {
    p = KQ4GemmPlan{tb, kb};
  } else if (nb >= 128 && tiles(1) > cu) {
    // rounds of each form; a 64 x 128 workgroup takes ~0.82 of a 128 x 128 one's time
    const long r1 = (tiles(1) + 2 * cu - 1) / (2 * cu), r2 = (tiles(2) + 3 * cu - 1) / (3 * cu);
    p.tile = 82 * r2 < 100 * r1 ? 2 : 1;
  } else {
    p.tile = tiles(1) >= 2 * cu                            ? 1
             : tiles(2) >= (nb >= 128 ? cu : 2 * cu) ? 2
                                                           : 3;
  }
  if (ctile && (p.tile == 1 || p.tile == 4)) p.tile = 2;
  return p;
}

int kq4_launch_gemm(float *out, const float *res, const uint8_t *w, const KQ4GemmAct &act,
                    int rows, int cols, int n_tok, int chain, int ncu, hipStream_t s, int wf,
                    int tile, int ksplit, float *part, int prio_opt) {
  const int nb = cols / 32;
  const int cb = wf ? KQ8_STREAM_CB : KQ4_STREAM_CB;
  const int nst = (nb + cb - 1) / cb;
  if (n_tok <= 0 || rows <= 0) return 0;
  auto tiles = [&](int bm, int bn) {
    return (long)((n_tok + bm - 1) / bm) * ((rows + bn - 1) / bn);
  };
  const int ks = split_len(nb, cb, ksplit);
  if (ksplit < 1 || ksplit > KQ4_GEMM_SPLIT_MAX || !ks || (ksplit > 1 && !part))
    return (int)hipErrorInvalidValue;
  int pick = tile >= 1 && tile <= 4 ? tile
                                    : kq4_gemm_plan(n_tok, rows, cols, wf, chain, ncu, -1, ksplit).tile;
  if (chain == KQ4_CHAIN_CTILE && (pick == 1 || pick == 4)) pick = 2;
  // 32-bit buffer offsets: weights and activation operands below 4 GB
  const size_t wb = wf ? kq8_stream_bytes(rows, cols) : kq4_stream_bytes(rows, cols);
  // (the last token tile's padding tokens, up to 127 past n_tok, address past the buffers' ends)
  const long ab = (n_tok + 127) * act.q_ts + (long)(nb - 1) * act.q_bs + 32;
  const long db = ((n_tok + 127) * act.d_ts + (long)(nb - 1) * act.d_bs + 1) * 4;
  if (wb >= KQ4_OOB || ab >= (long)KQ4_OOB || db >= (long)KQ4_OOB) return (int)hipErrorInvalidValue;
  // token-major activations: token t+1 starts past token t's last block (the q4 kernel's
  // zero reads for padding tokens rest on it)
  if (act.q_ts < (nb - 1) * act.q_bs + 32 || act.d_ts < (nb - 1) * act.d_bs + 1)
    return (int)hipErrorInvalidValue;
  const uint32_t wbytes = (uint32_t)wb;
  const long ps = (long)n_tok * rows;   // floats per slice output
  // The progress priority (kq4_prio_by_progress; planner option gemm_prio) for 128 x 128
  // launches of whole rounds (a multiple of two workgroups per CU), where every CU's last pair
  // should end together. With a part round left over it costs time: balanced pairs end together
  // and the rest then runs one workgroup per CU (Qwen3-8B gate, M = 1024: 768 workgroups,
  // 162 -> 167 us with it).
  // The pipelined 64 x 128 form (three workgroups per CU) gains from it on every launch, whole
  // rounds or not (Qwen3-8B, graph replays: gate M = 512, one round of 768 workgroups, 80.7 ->
  // 75.8 us; gate M = 448, 672 workgroups, 77.7 -> 72.0 us; QKV M = 768, 576, 77.5 -> 71.5 us;
  // the K-split launches at M = 128-768 3-6 %), so it is on there unless the option is 0.
  const long wgs = tiles(128, 128) * ksplit;
  const bool whole = ncu > 0 && wgs % (2L * ncu) == 0;
  const int prio = pick == 1 && (prio_opt == 1 || (prio_opt < 0 && whole));
  const int prio2 = pick == 2 && chain != KQ4_CHAIN_CTILE && prio_opt != 0;
  hipError_t e;
  if (pick == 1)
    e = gemm_launch<2, 2>(out, ksplit > 1 ? nullptr : res, w, act, rows, n_tok, nb, nst, chain,
                          wf, wbytes, s, ksplit, ks, part, ps, prio);
  else if (pick == 2)
    e = gemm_launch<1, 2>(out, ksplit > 1 ? nullptr : res, w, act, rows, n_tok, nb, nst, chain,
                          wf, wbytes, s, ksplit, ks, part, ps, prio2);
  else if (pick == 4)
    e = gemm_launch<2, 1>(out, ksplit > 1 ? nullptr : res, w, act, rows, n_tok, nb, nst, chain,
                          wf, wbytes, s, ksplit, ks, part, ps);
  else
    e = gemm_launch<1, 1>(out, ksplit > 1 ? nullptr : res, w, act, rows, n_tok, nb, nst, chain,
                          wf, wbytes, s, ksplit, ks, part, ps);
  if (e != hipSuccess || ksplit < 2) return (int)e;
  const long n4 = ps / 4;   // rows % 4 == 0
  hipLaunchKernelGGL(kq4_split_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                     out, res, part, ksplit - 1, ps, n4);
  return (int)hipGetLastError();
}
