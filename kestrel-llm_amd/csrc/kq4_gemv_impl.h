// kq4_gemv_impl.h - decode GEMV (1..8 tokens) over q4 weights in the kq4 stream layout x int8
// activations, gfx950: the kernel template, instantiated per token count by kq4_gemv_m<M>.hip
// (compiled in parallel) and dispatched by kq4_launch_gemv (kq4_gemv.hip).
//
// Computes out[m][n] = [res +] sum_b S[m,n,b] * fl(wd[n,b] * xs[m,b]), the op of
// q4x4_gemm_batched / dyn_matvec_q4_q8 (kestrel-llm src/model/vllm_safetensors.c:4593-4631,
// 6147-6174): S is the exact integer dot of row n's 32 nibble weights (n-8) with the token's
// int8 block, xs the token's block scale (f16-rounded for ASM-chain tokens, as the reference's
// asm path multiplies by the f16 scale it repacks, :4104-4105). Every per-block term is the
// reference's; the blocks of one output are summed serially within each wave's share of K and
// the shares are then added in wave order, so outputs agree with the reference's single serial
// chain to a few ulp of the row magnitude.
//
// The weights are in the stream layout (kq4_common.h): per (32-row set, 16-block stage) one
// 9216-B chunk in which lane l of a wave finds, at 16-B units l, l+64, .. (1 KB apart), the
// nibbles of its row (l%32) and K-half (l/32) for the stage's 16 blocks, and at 8192+16*l the
// f16 scales. So a stage is 9 + 1 full-width coalesced loads per lane (the second scale load
// reads the other half's 8 scales of the same row) and every lane then holds its own operands:
// no weight bytes pass through LDS.
//
// Work decomposition (the weight stream is the whole cost):
//   * a workgroup takes a group of output rows over one K slice: R whole 32-row sets (R = 1..3,
//     so that each workgroup's activation staging serves R sets), or half / a quarter of one set
//     (16 / 8 rows, for launches with few row sets), and the whole K or a slice of it (the
//     slices' sums are combined by the last slice to finish, see kq4_gemv_kernel); W <= 16 waves
//     take the slice's stages w, w + W, .., each issued as (activations, weights).
//   * each wave stages its own activations (int8 codes + per-block scales) in a small LDS slab,
//     quantizing them from fp32 itself (FQ) or copying a pre-quantized buffer, so the stage loop
//     has no workgroup barrier.
//   * the integer dot, two kinds:
//       DOT4: lane (row, half) dots its 16 weights of each block with v_dot4_i32_i8 against the
//             token's 16 codes (an LDS broadcast read) and keeps one fp32 chain per token and
//             half (the C-tile kernel's lo/hi split, :4180-4216); each wave adds its halves
//             before the waves' sums are added. Cost grows with M.
//       MFMA: per block one v_mfma_i32_32x32x32_i8 with A = the tokens' codes (32 rows, M <= 8
//             used) and B = the lanes' weight operands as they are; the result 16*S is at lane
//             (row = lane%32, token = 4*(lane/32) + v). Cost independent of M.
//   * at the end the partials of an output are added in a fixed order, each wave's lanes by lane
//     swaps, then the waves' sums through LDS, then (K slices) the slices in slice order:
//     deterministic.
#pragma once

#include "kq4_common.h"
#include "kq4_internal.h"

#define KQ4_GV_CB KQ4_STREAM_CB       // blocks per stage
#define KQ4_GV_CHUNK KQ4_STREAM_CHUNK // bytes per (32-row set, stage)
#define KQ4_GV_QTS 672                // LDS bytes per token row of a stage's int8 codes
#define KQ4_GV_XS (KQ4_GV_CB * 8 * 4) // LDS bytes of a stage's scales [16 blocks][8 tokens]

// Weight formats: 0 = q4 (kq4 stream layout); 1 = q8 (q8 stream layout) with the fused VDOT
// chain acc = fma(S, fl(wd*xs), acc); 2 = q8 with the unfused GEMM chain
// acc = fl(acc + fl(fl(wd*xs) * S)) (xs f16-rounded through asm_tokens).
template <int WF>
struct KQ4Wf {
  static constexpr int CB = WF ? KQ8_STREAM_CB : KQ4_STREAM_CB;          // blocks per stage
  static constexpr int CHUNK = WF ? KQ8_STREAM_CHUNK : KQ4_STREAM_CHUNK;
  static constexpr int BPU = WF ? 1 : 2;                                  // blocks per 16-B unit
  static constexpr float XS = WF ? 1.0f : 0.0625f;  // q4 enters the MFMA as 16*(n-8): undo it
};

typedef int kq4_v4i __attribute__((ext_vector_type(4)));
typedef int kq4_v16i __attribute__((ext_vector_type(16)));

// LDS bytes of one wave's slab: [activation codes][scales]; it also holds the wave's partial
// sums at the end (at most 8 tokens x 32 floats).
template <int M>
constexpr int kq4_gv_mx() {   // scale row width of the slab: 8 tokens, 16 in the wide kernel
  return M > 8 ? 16 : 8;
}
template <int M>
constexpr int kq4_gv_slab() {
  return M * KQ4_GV_QTS + KQ4_GV_CB * kq4_gv_mx<M>() * 4;
}

// Byte offset of block blk's 32 codes in a token row: block pairs at an 80-B pitch (16-B pad),
// which spreads the two halves' 16-B reads over the banks.
KQ4_DEV int kq4_gv_qpos(int blk) { return (blk >> 1) * 80 + (blk & 1) * 32; }

KQ4_DEV kq4_v16i kq4_gv_mfma(kq4_v4i a, kq4_v4i b) {
  const kq4_v16i z = {0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

// ---- weights of one stage -------------------------------------------------------------------
// A workgroup takes NR = 32 >> HS rows of a set (rows NR*hs .. +NR-1): HS = 0 the full set, 1 a
// half, 2 a quarter. Lane (r, p, h) = (lane % NR, (lane / NR) % NP, lane / 32) with NP = 1 << HS
// parities holds row NR*hs + r's half h of the units i = NP*u + p (u = 0 .. NU-1, NU = 8 >> HS
// unit loads; a q4 unit is 2 blocks, a q8 unit 1), so one load instruction covers NP units at
// 16*NR-byte runs. In every mode the row's scales (2 loads for q4, 1 for q8; the lanes of one
// row share them).

template <int HS>
struct KQ4GvStage {
  static constexpr int NU = 8 >> HS;      // 16-B nibble loads per lane
  uint32_t n[4 * NU];                     // lane block jb (0 .. 2*NU-1): n[2jb], n[2jb+1]
  uint32_t sc[8];                         // scale pairs (kq4_gv_load, kq4_gv_wd)
};

// Scales first: the loads complete in issue order, so the first block then waits only for the
// scales and its own unit, and each later block for one more unit.
// q8 (WF > 0): the same unit loads, one block per unit, and the row's 8 scales in one load.
// ORD: keep that issue order (left to itself the compiler may issue unit 0 near the end, and the
// first block then waits for nearly all of them): 1 = a scheduling barrier after each load, which
// also keeps every later instruction below the loads; 2 = a compiler memory barrier after each,
// which orders only the memory operations (the quantization's VALU work can still move above).
// Stage unit (2 blocks of q4, 1 of q8) held in load slot u by a lane of parity p: u*NP + p, but
// for q4 half sets units 2p, 2p+1, 4+2p, 5+2p (blocks 4p .. 4p+3 of each 8-block scale line).
template <int HS, int WF>
KQ4_DEV int kq4_gv_unit(int u, int p) {
  if (WF == 0 && HS == 1) return 2 * p + (u & 1) + 4 * (u >> 1);
  return (u << HS) + p;
}

template <int HS, int WF, int ORD = 0>
KQ4_DEV void kq4_gv_load(KQ4GvStage<HS> &st, const uint8_t *__restrict__ chunk, int rr, int h,
                         int p) {
  // the weights are read once per launch: non-temporal loads
  const uint4 *sc = reinterpret_cast<const uint4 *>(chunk + 8192) + rr;
  if constexpr (WF == 0 && HS == 2) {
    // quarter sets: the lane's blocks use one scale pair of each 8-block line (pair p), so it
    // loads those 4 bytes, not the lines (which 16 lanes share)
    const uint32_t *sw = reinterpret_cast<const uint32_t *>(sc) + p;
    st.sc[0] = __builtin_nontemporal_load(sw);
    st.sc[1] = __builtin_nontemporal_load(sw + 128);
  } else if constexpr (WF == 0 && HS == 1) {
    // half sets: parity p takes blocks 4p .. 4p+3 of each 8-block line (kq4_gv_unit), whose
    // scales are the 8 bytes at 8p of the line
    const uint2 *sw = reinterpret_cast<const uint2 *>(sc) + p;
    const kq4_v2u a = __builtin_nontemporal_load(reinterpret_cast<const kq4_v2u *>(sw));
    const kq4_v2u b = __builtin_nontemporal_load(reinterpret_cast<const kq4_v2u *>(sw + 64));
    st.sc[0] = a.x; st.sc[1] = a.y; st.sc[2] = b.x; st.sc[3] = b.y;
  } else {
    const uint4 a = kq4_ld_nt(sc);
    st.sc[0] = a.x; st.sc[1] = a.y; st.sc[2] = a.z; st.sc[3] = a.w;
    if (WF == 0) {
      const uint4 b = kq4_ld_nt(sc + 32);
      st.sc[4] = b.x; st.sc[5] = b.y; st.sc[6] = b.z; st.sc[7] = b.w;
    }
  }
  if constexpr (ORD == 1) __builtin_amdgcn_sched_barrier(0);
  if constexpr (ORD == 2) asm volatile("" ::: "memory");
  const uint4 *src = reinterpret_cast<const uint4 *>(chunk) + rr + 32 * h;
#pragma unroll
  for (int u = 0; u < KQ4GvStage<HS>::NU; ++u) {
    const int i = kq4_gv_unit<HS, WF>(u, p);
    const uint4 v = kq4_ld_nt(src + 64 * i);
    st.n[4 * u] = v.x; st.n[4 * u + 1] = v.y; st.n[4 * u + 2] = v.z; st.n[4 * u + 3] = v.w;
    if constexpr (ORD == 1) __builtin_amdgcn_sched_barrier(0);
    if constexpr (ORD == 2) asm volatile("" ::: "memory");
  }
}

// Load-order mode of kq4_gv_load for the first row set of a stage: a scheduling barrier for one
// token from fp32 activations, a memory barrier for two and three (Qwen3-8B gate/up and QKV at
// M = 2: 12.2-12.5 -> 11.7-12.0 and 5.8-5.9 -> 5.3-5.5 us). Not from four tokens on: there it
// measured mixed (8B down at M = 4 0.5 us slower, the 2B QKV 0.3 us faster), and for 4-6 tokens
// in single-set kernels it costs a wave per SIMD (74-96 -> 100-101 VGPRs).
template <int M, int FQ>
constexpr int kq4_gv_ord() {
  if (FQ != 1) return 0;
  return M == 1 ? 1 : (M <= 3 ? 2 : 0);
}

// Stage block of lane block jb (p = the lane's unit parity).
template <int HS, int WF>
KQ4_DEV int kq4_gv_blk(int jb, int p) {
  if (WF) return (jb << HS) + p;
  return 2 * kq4_gv_unit<HS, WF>(jb >> 1, p) + (jb & 1);
}

// a if p == 0, b if p == 1 (p in {0, 1}), by masks: a select between two elements of one register
// array would be folded into a lane-dependent index, which puts the array in scratch memory.
KQ4_DEV uint32_t kq4_gv_pick(uint32_t a, uint32_t b, int p) {
  const uint32_t m = 0u - (uint32_t)p;
  return (a & ~m) | (b & m);
}

// v[p] of the NP = 1 << HS registers v[0 .. NP-1] (p < NP), by masks.
template <int HS>
KQ4_DEV uint32_t kq4_gv_pickn(const uint32_t *v, int p) {
  if (HS == 0) return v[0];
  if (HS == 1) return kq4_gv_pick(v[0], v[1], p);
  return kq4_gv_pick(kq4_gv_pick(v[0], v[1], p & 1), kq4_gv_pick(v[2], v[3], p & 1), p >> 1);
}

// Row scale (f32) of lane block jb; the register index is compile-time in all modes.
// q8: block b = NP*jb + p, its scale at sc[b/2] >> 16*(b%2) (the row's line as loaded); q4:
// block kq4_gv_blk(jb, p), full sets at sc[jb/2] >> 16*(jb%2) of the row's two lines, half and
// quarter sets at sc[jb/2] >> 16*(jb%2) of the lane's own pairs.
template <int HS, int WF>
KQ4_DEV float kq4_gv_wd(const KQ4GvStage<HS> &st, int jb, int p) {
  if (WF) {
    if (HS == 0) return kq4_h2f(st.sc[jb >> 1] >> (16 * (jb & 1)));
    if (HS == 1) return kq4_h2f(st.sc[jb] >> (16 * p));
    return kq4_h2f(kq4_gv_pick(st.sc[2 * jb], st.sc[2 * jb + 1], p >> 1) >> (16 * (p & 1)));
  }
  // half and quarter sets hold only the lane's scales (kq4_gv_load), in load-slot order
  const uint32_t w = HS >= 1 ? st.sc[jb >> 1] : kq4_gv_pickn<HS>(&st.sc[(jb >> 1) << HS], p);
  return kq4_h2f(w >> (16 * (jb & 1)));
}

// The MFMA B operand of lane block jb: q4 unpacks its 8 nibble bytes to 16*(n-8); q8 is the
// 16-B unit as loaded.
template <int WF>
KQ4_DEV void kq4_gv_bop(const uint32_t *n, int jb, uint32_t *o) {
  if (WF) {
    o[0] = n[4 * jb]; o[1] = n[4 * jb + 1]; o[2] = n[4 * jb + 2]; o[3] = n[4 * jb + 3];
  } else {
    kq4_unpack_half(n[2 * jb], n[2 * jb + 1], o);
  }
}

// ---- activations of a stage -------------------------------------------------------------------
// Loaded into registers together with (just before) the stage's weights, then written to the
// wave's slab as int8 codes (token row m at m*KQ4_GV_QTS, block at kq4_gv_qpos) and the
// effective per-block scale sx[blk][m] = xs/16 for q4 (xs = f16-rounded xd for ASM-chain tokens;
// the /16 undoes the 16*(n-8) weight scaling exactly), xs for q8. A stage is 16 blocks of q4 or 8
// of q8. Issuing them before the weights keeps the in-order load counter from making the
// quantization wait for the weights.
//
// FQ = 0: pre-quantized; 1: fp32 activations; 2: fp32 gate and up, activation = silu_mul(g, u)
// (kq4_silu_mul, the dense FFN's down input, vllm_safetensors.c:10932-10958).
// FQ 1, 2 (passes of kq4_gv_mq tokens): lane quad (4q .. 4q+3) owns block q for one token, 8
// fp32 each; the quantization restates quantize_row_q8_0_act (vllm_safetensors.c:7893-7920):
// d = amax/127 is a true division, x/d the Markstein-corrected quotient q = x*y,
// q += fma(-q, d, x)*y with y = RN(1/d), which is the correctly rounded x/d for these normal
// operands, so the codes are the reference's bit for bit.
// Pre-quantized: lane i copies 16-B units i, i+64, .. of the stage's codes and scales i, i+64.
template <int M, int FQ, int WF>
struct KQ4GvAct {
  static constexpr int CB = KQ4Wf<WF>::CB;
  static constexpr int NQ = FQ ? 1 : (2 * CB * M + 63) / 64;   // uint4 per lane
  static constexpr int NX = FQ ? 1 : (CB * M + 63) / 64;       // scales per lane
  float4 f[FQ ? 2 * M : 1];
  float4 u[FQ == 2 ? 2 * M : 1];
  uint4 q[NQ];
  float x[NX];
};

// M = tokens of this pass; the in-kernel quantization (FQ) takes the tokens in passes of up to
// kq4_gv_mq<> tokens from token t0 on (registers), the pre-quantized copy all of them at t0 = 0.
template <int M, int FQ, int WF, bool WIDE = false>
KQ4_DEV void kq4_gv_act_load(KQ4GvAct<M, FQ, WF> &r, const KQ4GemvArgs &a, int st, int lane,
                             int t0) {
  constexpr int CB = KQ4Wf<WF>::CB;
  const int nb = a.nb, cols = a.cols;
  const int kb = st * CB;
  const int mlim = WIDE ? a.ntok - t0 : M;   // the wide kernel's padding tokens read nothing
  if (FQ) {
    const int b = kb + (lane >> 2), qq = lane & 3;
    const bool live = (lane >> 2) < CB && b < nb;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (live && m < mlim) {
        const float4 *src = reinterpret_cast<const float4 *>(a.xf + (size_t)(t0 + m) * cols +
                                                             (size_t)b * 32 + 8 * qq);
        r.f[2 * m] = src[0];
        r.f[2 * m + 1] = src[1];
        if (FQ == 2) {
          const float4 *su = reinterpret_cast<const float4 *>(a.xu + (size_t)(t0 + m) * cols +
                                                              (size_t)b * 32 + 8 * qq);
          r.u[2 * m] = su[0];
          r.u[2 * m + 1] = su[1];
        }
      } else {
        r.f[2 * m] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        r.f[2 * m + 1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (FQ == 2) {
          r.u[2 * m] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          r.u[2 * m + 1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, WF>::NQ; ++c) {
      const int i = lane + 64 * c;
      const int m = i / (2 * CB), u = i % (2 * CB), b = kb + (u >> 1), hh = u & 1;
      r.q[c] = make_uint4(0, 0, 0, 0);
      if (m < M && m < mlim && b < nb)
        r.q[c] = *reinterpret_cast<const uint4 *>(a.xq + (size_t)m * cols + (size_t)b * 32 + 16 * hh);
    }
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, WF>::NX; ++c) {
      const int i = lane + 64 * c;
      const int m = i / CB, b = kb + i % CB;
      r.x[c] = (m < M && m < mlim && b < nb) ? a.xd[(size_t)m * nb + b] : 0.0f;
    }
  }
}

template <int M, int FQ, int WF, int MX = 8>
KQ4_DEV void kq4_gv_act_put(const KQ4GvAct<M, FQ, WF> &r, const KQ4GemvArgs &a, int lane,
                            uint8_t *sq, float (*sx)[MX], int t0) {
  constexpr int CB = KQ4Wf<WF>::CB;
  constexpr float XS = KQ4Wf<WF>::XS;
  if constexpr (FQ != 0) {
    const int blk = lane >> 2, qq = lane & 3;
    static_assert(M <= 4, "one token of a pass per lane of the quad");
    float v[M][8];
    float amax[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float f[8] = {r.f[2 * m].x, r.f[2 * m].y, r.f[2 * m].z, r.f[2 * m].w,
                          r.f[2 * m + 1].x, r.f[2 * m + 1].y, r.f[2 * m + 1].z, r.f[2 * m + 1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) v[m][i] = f[i];
      if (FQ == 2) {
        const float u[8] = {r.u[2 * m].x, r.u[2 * m].y, r.u[2 * m].z, r.u[2 * m].w,
                            r.u[2 * m + 1].x, r.u[2 * m + 1].y, r.u[2 * m + 1].z, r.u[2 * m + 1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[m][i] = kq4_silu_mul(v[m][i], u[i]);
      }
      amax[m] = 1e-10f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax[m] = fmaxf(amax[m], fabsf(v[m][i]));
      amax[m] = kq4_quad_max_pos(amax[m]);
    }
    // The two true divisions of a (block, token) are done once per quad: lane qq of the quad
    // divides for token qq of the pass, and every lane of the quad takes token m's d and 1/d
    // from lane m (a DPP broadcast), instead of each lane dividing for every token.
    float am = amax[0];
#pragma unroll
    for (int m = 1; m < M; ++m) am = qq == m ? amax[m] : am;
    const float dq = am / 127.0f;
    const float yq = 1.0f / dq;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float d = M == 1 ? dq : kq4_quad_bcast(dq, m);
      const float y = M == 1 ? yq : kq4_quad_bcast(yq, m);
      int c[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = v[m][i] * y;
        const float e = fmaf(-q, d, v[m][i]);
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
      if (blk < CB)   // q8 stages have 8 blocks: lanes 32-63 hold nothing
        *reinterpret_cast<uint2 *>(sq + (t0 + m) * KQ4_GV_QTS + kq4_gv_qpos(blk) + 8 * qq) =
            make_uint2(pk[0], pk[1]);
    }
    if (blk < CB && qq < M)
      sx[blk][t0 + qq] = ((t0 + qq < a.asm_tokens) ? kq4_f16_round(dq) : dq) * XS;
  } else {
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, WF>::NQ; ++c) {
      const int i = lane + 64 * c;
      const int m = i / (2 * CB), u = i % (2 * CB);
      if (m < M)
        *reinterpret_cast<uint4 *>(sq + m * KQ4_GV_QTS + kq4_gv_qpos(u >> 1) + 16 * (u & 1)) = r.q[c];
    }
#pragma unroll
    for (int c = 0; c < KQ4GvAct<M, FQ, WF>::NX; ++c) {
      const int i = lane + 64 * c;
      const int m = i / CB, blk = i % CB;
      if (m < M) sx[blk][m] = ((m < a.asm_tokens) ? kq4_f16_round(r.x[c]) : r.x[c]) * XS;
    }
  }
}

// ---- compute ---------------------------------------------------------------------------------

// Materialises x here: the unrolled block loops below would otherwise have every block's product
// sunk to the end of the stage, keeping all blocks' operands live at once (far more registers
// than a wave has).
KQ4_DEV void kq4_gv_pin(float &x) { asm volatile("" : "+v"(x)); }

// DOT4: acc[m] = token m's chain over this lane's blocks of its row and half.
// One token in half- or quarter-set mode (the decode shapes with few row sets): all the lane's
// blocks' codes and scales are read from LDS first (40 or 20 registers), so the blocks do not wait
// for LDS one by one once the weights are in.
template <int M, int HS>
KQ4_DEV void kq4_gv_dot4(const KQ4GvStage<HS> &st, const uint8_t *sq, const float (*sx)[8], int h,
                         int p, float *acc) {
  constexpr int NJB = 2 * KQ4GvStage<HS>::NU;
  constexpr bool PRE = M == 1 && HS >= 1;
  uint4 qv[PRE ? NJB : 1];
  float xv[PRE ? NJB : 1];
  if (PRE) {
#pragma unroll
    for (int jb = 0; jb < NJB; ++jb) {
      const int b = kq4_gv_blk<HS, 0>(jb, p);
      qv[jb] = *reinterpret_cast<const uint4 *>(sq + kq4_gv_qpos(b) + 16 * h);
      xv[jb] = sx[b][0];
    }
  }
#pragma unroll
  for (int jb = 0; jb < NJB; ++jb) {
    const int b = kq4_gv_blk<HS, 0>(jb, p);
    uint32_t o[4];
    kq4_unpack_half(st.n[2 * jb], st.n[2 * jb + 1], o);
    const float wd = kq4_gv_wd<HS, 0>(st, jb, p);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 q = PRE ? qv[jb]
                          : *reinterpret_cast<const uint4 *>(sq + m * KQ4_GV_QTS + kq4_gv_qpos(b) +
                                                             16 * h);
      int s = kq4_dot4(o[0], q.x, 0);
      s = kq4_dot4(o[1], q.y, s);
      s = kq4_dot4(o[2], q.z, s);
      s = kq4_dot4(o[3], q.w, s);
      acc[m] = fmaf((float)s, wd * (PRE ? xv[jb] : sx[b][m]), acc[m]);
      kq4_gv_pin(acc[m]);
    }
  }
}

// MFMA: one v_mfma_i32_32x32x32_i8 per lane block. B column = lane%32 = row + NR*p (the NP
// parities hold different blocks), k half = lane/32. A row = lane%32 holds the codes of token
// min(lane % NR, M-1) for the lane's own block, so output (token row T, column c) is valid where
// T's block matches c's: T = token + NR*p, which the 32x32 output layout puts in result register
// (NR/2)*p + v for token 4h+v. acc[v] = token 4h+v of the lane's row (and parity).
template <int M, int HS, int WF, int MX = 8>
KQ4_DEV void kq4_gv_mfma_stage(const KQ4GvStage<HS> &st, const uint8_t *sq, const float (*sx)[MX],
                               int lane, int p, float *acc) {
  constexpr int VT = M < 4 ? M : 4;
  constexpr int NG = M > 8 ? 2 : 1;   // token groups 0-7, 8-15 (result registers 4j + v)
  const int h = lane >> 5;
  constexpr int NR = 32 >> HS;
  const int tr = lane & (NR - 1);
  const int t = tr < M ? tr : M - 1;
  const uint8_t *qb = sq + t * KQ4_GV_QTS + 16 * h;
#pragma unroll
  for (int jb = 0; jb < KQ4GvStage<HS>::NU * KQ4Wf<WF>::BPU; ++jb) {
    const int b = kq4_gv_blk<HS, WF>(jb, p);
    uint32_t o[4];
    kq4_gv_bop<WF>(st.n, jb, o);
    const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    const kq4_v4i A = *reinterpret_cast<const kq4_v4i *>(qb + kq4_gv_qpos(b));
    const kq4_v16i C = kq4_gv_mfma(A, B);
    const float wd = kq4_gv_wd<HS, WF>(st, jb, p);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const float4 xs = *reinterpret_cast<const float4 *>(&sx[b][8 * j + 4 * h]);
      const float xv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
      for (int v = 0; v < VT; ++v) {
        uint32_t cv[1 << HS];
#pragma unroll
        for (int pp = 0; pp < (1 << HS); ++pp) cv[pp] = (uint32_t)C[(NR / 2) * pp + 4 * j + v];
        const int c = (int)kq4_gv_pickn<HS>(cv, p);
        float &ac = acc[4 * j + v];
        if (WF == 2) ac = ac + (wd * xv[v]) * (float)c;   // the q8 GEMM chain, unfused
        else ac = fmaf((float)c, wd * xv[v], ac);
        kq4_gv_pin(ac);
      }
    }
  }
}

// The matrix of workgroup wg (a launch covers up to KQ4_MAXMAT matrices, each a contiguous range
// of workgroups). Every entry's fields are read first and then chosen by compares: indexing the
// argument array by the chosen entry would be a second scalar load that waits for the first, and
// the weight loads wait for both (the empty asm keeps the compiler from turning the selects back
// into an indexed load).
// The pointers are kept in the global address space (kernel arguments are global memory; a
// generic pointer out of the asm would make every weight load a flat load, which also counts
// against the LDS wait counter).
typedef const __attribute__((address_space(1))) uint8_t *kq4_gw_t;
typedef __attribute__((address_space(1))) float *kq4_go_t;
typedef const __attribute__((address_space(1))) float *kq4_gr_t;

struct KQ4GvMatSel {
  kq4_gw_t w;
  kq4_go_t out;
  kq4_gr_t res;
  int rows, wg_begin;
};

KQ4_DEV KQ4GvMatSel kq4_gv_select(const KQ4GemvArgs &a, int wg) {
  static_assert(KQ4_MAXMAT == 4, "kq4_gv_select reads 4 entries");
  kq4_gw_t w1 = (kq4_gw_t)a.mat[1].w, w2 = (kq4_gw_t)a.mat[2].w, w3 = (kq4_gw_t)a.mat[3].w;
  kq4_go_t o1 = (kq4_go_t)a.mat[1].out, o2 = (kq4_go_t)a.mat[2].out, o3 = (kq4_go_t)a.mat[3].out;
  kq4_gr_t r1 = (kq4_gr_t)a.mat[1].res, r2 = (kq4_gr_t)a.mat[2].res, r3 = (kq4_gr_t)a.mat[3].res;
  int n1 = a.mat[1].rows, n2 = a.mat[2].rows, n3 = a.mat[3].rows;
  int b1 = a.mat[1].wg_begin, b2 = a.mat[2].wg_begin, b3 = a.mat[3].wg_begin;
  asm volatile("" : "+s"(w1), "+s"(w2), "+s"(w3), "+s"(o1), "+s"(o2), "+s"(o3), "+s"(r1),
               "+s"(r2), "+s"(r3), "+s"(n1), "+s"(n2), "+s"(n3), "+s"(b1), "+s"(b2), "+s"(b3));
  KQ4GvMatSel s{(kq4_gw_t)a.mat[0].w, (kq4_go_t)a.mat[0].out, (kq4_gr_t)a.mat[0].res,
                a.mat[0].rows, 0};
  const int nm = a.nmat;
  if (nm > 1 && wg >= b1) s = KQ4GvMatSel{w1, o1, r1, n1, b1};
  if (nm > 2 && wg >= b2) s = KQ4GvMatSel{w2, o2, r2, n2, b2};
  if (nm > 3 && wg >= b3) s = KQ4GvMatSel{w3, o3, r3, n3, b3};
  return s;
}


// Tokens per pass of the in-kernel quantization: a lane holds 8 fp32 elements per token (16 with
// the SiLU's up) in registers while it quantizes, so larger batches are taken in passes of MQ
// tokens and a last pass of the M % MQ left.
template <int M, int FQ>
constexpr int kq4_gv_mq() {
  return FQ == 0 ? M : (FQ == 2 ? (M < 2 ? M : 2) : (M < 4 ? M : 4));
}

// Workgroup -> work. Workgroups are numbered over the launch's matrices, each matrix a
// contiguous range from its wg_begin; within a matrix, workgroup gl = sg * NP + hs covers the R
// row sets sg * R .. sg * R + R - 1 (HS = 0), or part hs of row set sg (half / quarter sets,
// R = 1), over the whole K. Each wave takes the stages wave, wave + nw, ..; for each stage it
// stages (quantizes) the activations once into its LDS slab and then streams the stage's chunk
// of every one of the group's R row sets, the next set's loads issued before the current set's
// dots. At the end each output's partials are added in a fixed order (lane swaps, then the
// waves through LDS), so results are deterministic.
// Up to 16 waves per workgroup for single-set groups (128 VGPRs), 8 for R > 1 (whose prefetched
// second set needs more registers).
template <int M, int FQ, int KIND, int HS, int WF, int R>
__global__ __launch_bounds__(R > 1 ? 512 : 1024) void kq4_gemv_kernel(const KQ4GemvArgs a) {
  extern __shared__ __align__(16) uint8_t kq4_gv_lds[];
  constexpr int SLAB = kq4_gv_slab<M>();
  constexpr int MX = kq4_gv_mx<M>();               // scale row width of the slab
  constexpr bool WIDE = M > 8;                     // 16-token kernel: a.ntok tokens, the rest padding
  constexpr int NACC = KIND == 0 ? M : (WIDE ? 8 : 4);
  constexpr int NR = 32 >> HS;                     // output rows per row set of the workgroup
  constexpr int NP = 1 << HS;                      // lane parities
  constexpr int MQ = kq4_gv_mq<M, FQ>();           // tokens per quantization pass
  constexpr int MT = M % MQ;                       // tokens of the last, shorter pass
  constexpr int NOUT = R * M * NR;                 // outputs of the workgroup
  static_assert(R == 1 || HS == 0, "several row sets per workgroup take whole sets");
  static_assert(!WIDE || (KIND == 1 && HS <= 1 && M == 16),
                "16 tokens: MFMA kind, whole or half sets (A rows 16p + token)");
  static_assert(NOUT * 4 <= SLAB, "a wave's partials fit its slab");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = a.nw;
  const int gg = (int)blockIdx.x;                  // group over the launch
  const KQ4GvMatSel ms = kq4_gv_select(a, gg);
  const int gl = gg - ms.wg_begin;
  const int set0 = (gl >> HS) * R;                 // first row set of the group
  const int hs = gl & (NP - 1);                    // the group's part of the set (HS > 0)
  const int rows = ms.rows;
  const int sets = (rows + 31) >> 5;
  const int nb = a.nb;
  constexpr int CB = KQ4Wf<WF>::CB, CHUNK = KQ4Wf<WF>::CHUNK;
  const int nst = (nb + CB - 1) / CB;
  const uint8_t *__restrict__ wb = (const uint8_t *)ms.w;
  uint8_t *slab = kq4_gv_lds + wave * SLAB;
  uint8_t *sq = slab;
  float (*sx)[MX] = reinterpret_cast<float (*)[MX]>(sq + M * KQ4_GV_QTS);
  const int h = lane >> 5;
  const int p = (lane >> (5 - HS)) & (NP - 1);
  const int r = lane & (NR - 1);                   // row within the set part
  const int rr = hs * NR + r;                      // row within the set

  float acc[R][NACC];
#pragma unroll
  for (int q = 0; q < R; ++q)
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[q][i] = 0.0f;
  for (int st = wave; st < nst; st += nw) {
    // issued as (activations, weights), so quantizing the activations waits only for them
    KQ4GvAct<MQ, FQ, WF> ra;
    KQ4GvStage<HS> rw[R > 1 ? 2 : 1];
    kq4_gv_act_load<MQ, FQ, WF, WIDE>(ra, a, st, lane, 0);
    kq4_gv_load<HS, WF, kq4_gv_ord<M, FQ>()>(rw[0], wb + ((size_t)set0 * nst + st) * CHUNK, rr,
                                             h, p);
    // One token, fp32 activations: every load is issued before the quantization waits for the
    // activations (the compiler otherwise sinks the weight loads below it, and the two memory
    // latencies add up). Not from two tokens on: there, issuing the weights before the
    // quantization costs a wave per SIMD (110-120 VGPRs instead of 82-83 at four tokens) and
    // measured slower for every Qwen3-8B decode shape (8B gate/up at 2 tokens 12.15 -> 13.0 us),
    // faster only for the 2B QKV and O launches (one workgroup per CU: 4.7 -> 4.1 us at 4 tokens).
    if constexpr (M == 1 && FQ == 1) __builtin_amdgcn_sched_barrier(0);
    kq4_gv_act_put<MQ, FQ, WF, MX>(ra, a, lane, sq, sx, 0);
#pragma unroll
    for (int t0 = MQ; t0 + MQ <= M; t0 += MQ) {
      if (WIDE && t0 >= a.ntok) break;   // passes of padding tokens only: their outputs are not
                                         // stored, so their stale slab rows are never read back
      kq4_gv_act_load<MQ, FQ, WF, WIDE>(ra, a, st, lane, t0);
      kq4_gv_act_put<MQ, FQ, WF, MX>(ra, a, lane, sq, sx, t0);
    }
    if constexpr (MT > 0) {
      KQ4GvAct<MT, FQ, WF> rt;
      kq4_gv_act_load<MT, FQ, WF>(rt, a, st, lane, M - MT);
      kq4_gv_act_put<MT, FQ, WF>(rt, a, lane, sq, sx, M - MT);
    }
#pragma unroll
    for (int q = 0; q < R; ++q) {
      // the next set's loads are unconditional (a group's sets past the matrix reload its last
      // set, computed on but not stored): behind a branch, the wait counts at the join had to
      // hold for both paths, and the current set's blocks waited for some of the next set's loads
      if (q + 1 < R) {
        const int sn = set0 + q + 1 < sets ? set0 + q + 1 : sets - 1;
        kq4_gv_load<HS, WF>(rw[(q + 1) & 1], wb + ((size_t)sn * nst + st) * CHUNK, rr, h, p);
      }
      if (q == 0 || set0 + q < sets) {
        if constexpr (WIDE) kq4_gv_mfma_stage<M, HS, WF, MX>(rw[q & 1], sq, sx, lane, p, acc[q]);
        else if (KIND == 0) kq4_gv_dot4<M, HS>(rw[q & 1], sq, sx, h, p, acc[q]);
        else kq4_gv_mfma_stage<M, HS, WF>(rw[q & 1], sq, sx, lane, p, acc[q]);
      }
    }
  }

  // Each output's lane partials are first added inside the wave by a fixed tree of lane swaps
  // (DOT4: the two K halves' chains, then the parities; MFMA: the parities; lane bits 3 and 4 of
  // quarter sets, bit 4 of half sets), and the wave's sum goes to its slab at
  // red[(q * M + m) * NR + r]; then the waves' sums are added in wave order.
  float *__restrict__ out = (float *)ms.out;
  const float *__restrict__ res = (const float *)ms.res;
  float *red = reinterpret_cast<float *>(slab);   // only this wave used its slab so far
#pragma unroll
  for (int q = 0; q < R; ++q) {
    if (KIND == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = kq4_xor_add<32>(acc[q][m]);
        if (HS == 2) v = kq4_xor_add<8>(v);
        if (HS >= 1) v = kq4_xor_add<16>(v);
        if (lane < NR) red[(q * M + m) * NR + r] = v;
      }
    } else {
#pragma unroll
      for (int v = 0; v < NACC; ++v) {   // register v: token 8 * (v / 4) + 4h + v % 4
        float t = acc[q][v];
        if (HS == 2) t = kq4_xor_add<8>(t);
        if (HS >= 1) t = kq4_xor_add<16>(t);
        const int tk = 8 * (v >> 2) + 4 * h + (v & 3);
        if (p == 0 && tk < M) red[(q * M + tk) * NR + r] = t;
      }
    }
  }
  auto out_row = [&](int i) { return (set0 + i / (M * NR)) * 32 + hs * NR + (i & (NR - 1)); };
  auto wave_sum = [&](int i) {
    float s = 0.0f;
    for (int w = 0; w < nw; ++w) s += reinterpret_cast<const float *>(kq4_gv_lds + w * SLAB)[i];
    return s;
  };
  // the first pass's residual is loaded before the barrier, so its latency hides behind the
  // wait (measured: 2B down and O with residual 0.04-0.08 us faster per launch at one token)
  const int mstore = WIDE ? a.ntok : M;            // tokens whose outputs are stored
  float res0 = 0.0f;
  {
    const int i = threadIdx.x, row = out_row(i);
    if (res && i < NOUT && row < rows && (i / NR) % M < mstore)
      res0 = res[(size_t)((i / NR) % M) * rows + row];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NOUT; i += 64 * nw) {
    const int row = out_row(i);
    if (row >= rows || (i / NR) % M >= mstore) continue;
    const float s = wave_sum(i);
    const size_t o = (size_t)((i / NR) % M) * rows + row;
    out[o] = res ? (i == (int)threadIdx.x ? res0 : res[o]) + s : s;
  }
}

template <int M, int FQ, int KIND, int HS, int WF, int R>
static hipError_t kq4_gv_launch1(const KQ4GemvArgs &a, int grid, hipStream_t s) {
  const size_t lds = (size_t)a.nw * kq4_gv_slab<M>();
  const void *fn = reinterpret_cast<const void *>(&kq4_gemv_kernel<M, FQ, KIND, HS, WF, R>);
  if (lds > 64 * 1024) {   // above the default dynamic LDS limit: raise it
    static std::atomic<unsigned long long> attr{0};
    hipError_t e = kq4_lds_limit_once(fn, 160 * 1024 - 64, attr);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((kq4_gemv_kernel<M, FQ, KIND, HS, WF, R>), dim3(grid), dim3(64 * a.nw), lds,
                     s, a);
  return hipGetLastError();
}

template <int M, int FQ, int KIND, int WF>
static hipError_t kq4_gv_launch_hr(const KQ4GemvArgs &a, int hs, int rps, int grid,
                                   hipStream_t s) {
  if (hs == 2) return kq4_gv_launch1<M, FQ, KIND, 2, WF, 1>(a, grid, s);
  if (hs == 1) return kq4_gv_launch1<M, FQ, KIND, 1, WF, 1>(a, grid, s);
  if (rps == 3) return kq4_gv_launch1<M, FQ, KIND, 0, WF, 3>(a, grid, s);
  if (rps == 2) return kq4_gv_launch1<M, FQ, KIND, 0, WF, 2>(a, grid, s);
  return kq4_gv_launch1<M, FQ, KIND, 0, WF, 1>(a, grid, s);
}

template <int M, int FQ>
static hipError_t kq4_gv_launch_k(const KQ4GemvArgs &a, int kind, int hs, int rps, int grid,
                                  hipStream_t s) {
  if (a.wf == 1)   // q8: the MFMA kind only (its block sums span both K halves)
    return kq4_gv_launch_hr<M, FQ, 1, 1>(a, hs, rps, grid, s);
  if (a.wf == 2) return kq4_gv_launch_hr<M, FQ, 1, 2>(a, hs, rps, grid, s);
  if (kind == 0) {
    if constexpr (M <= KQ4_GEMV_DOT4_MAX_M) return kq4_gv_launch_hr<M, FQ, 0, 0>(a, hs, rps, grid, s);
    else return hipErrorInvalidValue;
  }
  return kq4_gv_launch_hr<M, FQ, 1, 0>(a, hs, rps, grid, s);
}

// One GEMV launch for M tokens: fq 0 = pre-quantized activations, 1 = fp32 (quantized in the
// kernel), 2 = fp32 gate and up (the SiLU product quantized in the kernel, q4 only).
template <int M>
hipError_t kq4_gv_launch_m(const KQ4GemvArgs &a, int kind, int fq, int hs, int rps, int grid,
                           hipStream_t s) {
  if (fq == 2) {
    if (a.wf) return hipErrorInvalidValue;
    if (kind == 0) {
      if constexpr (M <= KQ4_GEMV_DOT4_MAX_M) return kq4_gv_launch_hr<M, 2, 0, 0>(a, hs, rps, grid, s);
      else return hipErrorInvalidValue;
    }
    return kq4_gv_launch_hr<M, 2, 1, 0>(a, hs, rps, grid, s);
  }
  if (fq == 1) return kq4_gv_launch_k<M, 1>(a, kind, hs, rps, grid, s);
  return kq4_gv_launch_k<M, 0>(a, kind, hs, rps, grid, s);
}
