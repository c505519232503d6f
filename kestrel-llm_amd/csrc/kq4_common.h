// kq4_common.h - shared device helpers for the gfx950 q4 x int8 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define KQ4_DEV __device__ __forceinline__

// Exact f16 -> f32 of a tile row scale (hardware cvt keeps f16 subnormals; the reference
// decodes the same value in f16_to_f32_bits vllm_safetensors.c:3614-3631).
KQ4_DEV float kq4_h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xFFFFu)));
}

// f32 -> f16 (RNE, subnormals kept) -> f32: the activation scale the reference's asm GEMM
// path multiplies by (repack_q8_0_4x4 vllm_safetensors.c:4104-4105).
KQ4_DEV float kq4_f16_round(float x) { return __half2float(__float2half_rn(x)); }

// Nibble bytes of one tile dword (4 bytes of one row) as 16*(n-8) int8 lanes:
// the stored nibble is n^8, the 4-bit two's complement of n-8, so shifting it into the
// high half of each byte gives 16*(n-8) exactly (vllm_safetensors.c:4133-4151).
KQ4_DEV uint32_t kq4_lo16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
KQ4_DEV uint32_t kq4_hi16(uint32_t w) { return w & 0xF0F0F0F0u; }

// ---- SiLU(g) * u of the dense FFN ---------------------------------------------------------
// The reference's dense path runs its SiLU-multiply on AArch64 as vllm_silu_mul_worker
// (vllm_safetensors.c:10932-10958): 4-wide, every element of n & ~3, with exp_neon4 (:4041-4068),
// the FRECPE reciprocal estimate and two FRECPS Newton steps. Each step below is the same IEEE
// binary32 operation as the NEON instruction it stands for (vfmaq/vfmsq = one fused rounding,
// vrndnq = round to nearest even, vcvtq_s32 = truncation), so the result is that path's, bit for
// bit, for finite inputs.

// exp_neon4: clamp to [-87, 87], n = rne(x * log2e), r = x - n*ln2 (fused), degree-6 Taylor
// polynomial in Horner form (fused steps), 2^n added to the exponent field.
KQ4_DEV float kq4_exp_neon(float x) {
  x = fminf(fmaxf(x, -87.0f), 87.0f);
  const float n = rintf(x * 1.4426950408889634f);
  const float r = fmaf(-n, 0.6931471805599453f, x);
  float p = 0.001388888888888889f;
  p = fmaf(p, r, 0.008333333333333333f);
  p = fmaf(p, r, 0.041666666666666664f);
  p = fmaf(p, r, 0.16666666666666666f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return __int_as_float(__float_as_int(p) + ((int)n << 23));
}

// FRECPE (ARMv8 FPRecipEstimate, single precision, no FEAT_RPRES) for positive normal x below
// 2^126, the range of 1 + exp_neon4(-g): the 8 fraction bits f below the leading one select
// a = 2*(256 + f) + 1, the estimate mantissa is r = (floor(2^19 / a) + 1) / 2 in [256, 511] and
// the exponent 253 - e. floor(2^19 / a) is taken from a float reciprocal: a is odd, so the exact
// quotient is at least 1/a >= 1/1023 away from an integer, far more than the reciprocal's
// error (< 2^-22 relative, < 3e-4 absolute here).
KQ4_DEV float kq4_frecpe(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t e = (b >> 23) & 0xFFu;
  const int a = 2 * (256 + (int)((b >> 15) & 0xFFu)) + 1;
  const int q = (int)(524288.0f * __builtin_amdgcn_rcpf((float)a));
  const uint32_t r = (uint32_t)((q + 1) >> 1);
  return __uint_as_float((b & 0x80000000u) | ((253u - e) << 23) | ((r & 0xFFu) << 15));
}

// fl(fl(g * rec) * u) with rec = 1 / (1 + e^-g) from FRECPE and two FRECPS steps
// (FRECPS = 2 - d*r with one rounding).
KQ4_DEV float kq4_silu_mul(float g, float u) {
  const float den = kq4_exp_neon(-g) + 1.0f;
  float rec = kq4_frecpe(den);
  rec = rec * fmaf(-den, rec, 2.0f);
  rec = rec * fmaf(-den, rec, 2.0f);
  return (g * rec) * u;
}

// v + v(lane ^ MASK) for MASK = 8, 16, 32 in VALU instructions, no LDS: a DPP row rotate by 8
// (xor 8 within a 16-lane row), v_permlane16_swap (rows 0<->1, 2<->3) and v_permlane32_swap
// (lanes 0-31 <-> 32-63). Both lanes of a pair get the same (commutative) sum.
template <int MASK>
KQ4_DEV float kq4_xor_add(float v) {
  static_assert(MASK == 8 || MASK == 16 || MASK == 32, "kq4_xor_add: mask 8, 16 or 32");
  const uint32_t u = __float_as_uint(v);
  if constexpr (MASK == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (MASK == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, (int)u, 0x128, 0xf, 0xf, false));
  }
}

// max of v over the lane quad (lanes 4q .. 4q+3) by two DPP quad permutes (xor 1, xor 2): VALU
// only, no LDS round trip. For non-NaN values every lane of the quad gets the same maximum.
KQ4_DEV float kq4_quad_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf,
                                                          false)));   // quad_perm [1,0,3,2]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf,
                                                          false)));   // quad_perm [2,3,0,1]
  return v;
}

// The same maximum for a non-negative, never-NaN v (a block's amax built by fmaxf from 1e-10 or
// +0): such floats order as their bit patterns, so an integer maximum with the DPP operand folds
// into one instruction per step (the float form adds a move and a canonicalizing max per step).
KQ4_DEV float kq4_quad_max_pos(float v) {
  uint32_t u = __float_as_uint(v);
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0xB1, 0xf, 0xf, false));
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, 0x4E, 0xf, 0xf, false));
  return __uint_as_float(u);
}

// Lane m's value (m = 0..3, a constant after unrolling) broadcast to every lane of its quad.
KQ4_DEV float kq4_quad_bcast(float v, int m) {
  const int u = __float_as_int(v);
  switch (m) {
    case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x00, 0xf, 0xf, false));
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x55, 0xf, 0xf, false));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0xAA, 0xf, 0xf, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0xFF, 0xf, 0xf, false));
  }
}

// 16-byte load with the non-temporal hint (global_load_dwordx4 ... nt), for data read once per
// launch (weight streams): measured on MI355X, plain streaming reads of 7-56 MB run 9-14 %
// faster with it than without.
typedef unsigned int kq4_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int kq4_v2u __attribute__((ext_vector_type(2)));
KQ4_DEV uint4 kq4_ld_nt(const void *p) {
  const kq4_v4u v = __builtin_nontemporal_load(reinterpret_cast<const kq4_v4u *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// max of v over each 32-lane half of the wave (lanes 0-31, 32-63): the quad max, DPP row rotates
// by 4 and 8 (the 16-lane row), then v_permlane16_swap (rows 0<->1, 2<->3). VALU only.
KQ4_DEV float kq4_max32(float v) {
  v = kq4_quad_max(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf,
                                                          false)));   // row_ror:4
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf,
                                                          false)));   // row_ror:8
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// 4 x int8 dot product accumulated into c (v_dot4_i32_i8).
KQ4_DEV int kq4_dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---- fp8 (OCP e4m3) operands of the prefill GEMM -------------------------------------------
// The GEMM's matrix-core operands hold small integers exactly in e4m3 (sign, 4 exponent bits with
// bias 7, 3 mantissa bits): weights w = n - 8 in [-8, 7]; activations q in [-127, 127] split as
// q = 16*qh + ql with qh = q >> 4 in [-8, 7] and ql = q & 15 in [0, 15], entering as 16*qh and
// ql. Every product and every partial sum of a block is an integer below 2^24, so the fp32
// result of the fp8 MFMA is the exact block sum S.
// e4m3 bytes of v = -8 .. 7 (index v + 8): the low 8 and the high 8 of the table.
#define KQ4_E4M3_NEG 0xb8c0c4c8caccced0ull   // v = -8 .. -1
#define KQ4_E4M3_POS 0x4e4c4a4844403800ull   // v =  0 ..  7

// e4m3 byte of the integer v in [-8, 7].
KQ4_DEV uint32_t kq4_e4m3_i4(int v) {
  const uint64_t t = v < 0 ? KQ4_E4M3_NEG : KQ4_E4M3_POS;
  return (uint32_t)(t >> (8 * (v & 7))) & 0xFFu;
}

// e4m3 bytes of 16*qh and ql for an int8 code q (16*qh is qh's e4m3 with the exponent 4 higher;
// ql >= 8 lies in the binade [8, 16) whose step is 1: byte 0x48 + ql).
KQ4_DEV uint32_t kq4_e4m3_hi(int q) {
  const int qh = q >> 4;
  return qh ? kq4_e4m3_i4(qh) + 0x20u : 0u;
}
KQ4_DEV uint32_t kq4_e4m3_lo(int q) {
  const int ql = q & 15;
  return ql < 8 ? kq4_e4m3_i4(ql) : 0x48u + (uint32_t)ql;
}

// The e4m3 bytes of the four 4-bit two's complement codes in the low nibbles of t's bytes (t's
// high nibbles zero): a byte permute picks each from the table of its sign, a third one the
// right table per byte.
KQ4_DEV uint32_t kq4_e4m3_nib4(uint32_t t) {
  const uint32_t pos = __builtin_amdgcn_perm((uint32_t)(KQ4_E4M3_POS >> 32), (uint32_t)KQ4_E4M3_POS, t);
  const uint32_t neg = __builtin_amdgcn_perm((uint32_t)(KQ4_E4M3_NEG >> 32), (uint32_t)KQ4_E4M3_NEG,
                                             t & 0x07070707u);
  const uint32_t sel = ((t >> 1) & 0x04040404u) | 0x03020100u;   // byte k: k (pos) or 4 + k (neg)
  return __builtin_amdgcn_perm(neg, pos, sel);
}

// ---- raw buffer loads -------------------------------------------------------------------------
// Loads through a buffer resource of `bytes` bytes: the hardware's range check returns zeros for
// offsets at or past the end, so loads of tiles that overhang a matrix need no branches (an
// offset of KQ4_OOB reads zeros too).
#define KQ4_OOB 0xFFFFFFF0u
KQ4_DEV __amdgpu_buffer_rsrc_t kq4_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                           0x00020000);   // gfx9 raw buffer, 32-bit data
}
KQ4_DEV uint4 kq4_bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
KQ4_DEV uint2 kq4_bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}
KQ4_DEV uint32_t kq4_bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// The same with the offset split into a per-lane part (voff) and a wave-uniform one (soff, the
// instruction's scalar offset): loads whose uniform part changes per loop step cost no vector
// arithmetic.
KQ4_DEV uint4 kq4_bload16s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, (int)soff, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
KQ4_DEV uint2 kq4_bload8s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, (int)soff, 0);
  return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}
KQ4_DEV uint32_t kq4_bload4s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, (int)soff, 0);
}
KQ4_DEV uint32_t kq4_bload2s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, (int)soff, 0);
}

// ---- stream layout of the device weights -------------------------------------------------
// A q4 matrix lives in HBM as 9216-B chunks, one per (32-row set, 16-block stage), in
// [set][stage] order. In a chunk, "lane" l = row + 32*h (row = row within the set, h = half of
// the 32-element block: elements 16h .. 16h+15) holds
//   * at 1024*i + 16*l, i = 0..7: 8 nibble bytes for block 2i, then 8 for block 2i+1 (of the
//     stage); dword d, byte k carries the stored 4-bit codes of elements 16h+8d+k (low nibble)
//     and 16h+8d+4+k (high nibble). The stored code is the VQF one (the legacy nibble n XOR 8,
//     the 4-bit two's complement of n-8), so kq4_lo16 / kq4_hi16 of dword d are the 16*(n-8)
//     int8 values of elements 16h+8d .. +3 and 16h+8d+4 .. +7: a lane's 8 bytes are one half
//     of one row of one block, in element order - the B operand of v_mfma_i32_32x32x32_i8.
//   * at 8192 + 16*l: the f16 row scales of blocks 8h .. 8h+7 (of the stage) of its row.
// Rows past the matrix and blocks past its K are zero bytes (zero scale, zero codes).
#define KQ4_STREAM_CB 16
#define KQ4_STREAM_CHUNK 9216

// Byte offset of the 8 nibble bytes of (row, block b, half h) in a matrix of nst stages.
KQ4_DEV size_t kq4_stream_nib(int row, int b, int h, int nst) {
  return ((size_t)(row >> 5) * nst + (b >> 4)) * KQ4_STREAM_CHUNK + 1024 * ((b & 15) >> 1) +
         16 * ((row & 31) + 32 * h) + 8 * (b & 1);
}

// Byte offset of the f16 scale of (row, block b).
KQ4_DEV size_t kq4_stream_scale(int row, int b, int nst) {
  return ((size_t)(row >> 5) * nst + (b >> 4)) * KQ4_STREAM_CHUNK + 8192 +
         16 * ((row & 31) + 32 * ((b & 15) >> 3)) + 2 * (b & 7);
}

// ---- q8 stream layout (device copy of Q8_0 tiles) -----------------------------------------
// One 8704-B chunk per (32-row set, 8-block stage), in [set][stage] order; lane l = row + 32*h
//   * at 1024*i + 16*l, i = 0..7: the 16 int8 codes of elements 16h .. 16h+15 of block i of the
//     stage, row `row` - in element order, the B operand of v_mfma_i32_32x32x32_i8 as loaded;
//   * at 8192 + 16*row: the row's 8 f16 scales (blocks 0..7 of the stage).
// Rows past the matrix and blocks past its K are zero bytes.
#define KQ8_STREAM_CB 8
#define KQ8_STREAM_CHUNK 8704

KQ4_DEV size_t kq8_stream_code(int row, int b, int h, int nst) {
  return ((size_t)(row >> 5) * nst + (b >> 3)) * KQ8_STREAM_CHUNK + 1024 * (b & 7) +
         16 * ((row & 31) + 32 * h);
}

KQ4_DEV size_t kq8_stream_scale(int row, int b, int nst) {
  return ((size_t)(row >> 5) * nst + (b >> 3)) * KQ8_STREAM_CHUNK + 8192 + 16 * (row & 31) +
         2 * (b & 7);
}

// The 16*(n-8) int8 operand (4 dwords, element order) of 8 nibble bytes.
KQ4_DEV void kq4_unpack_half(uint32_t d0, uint32_t d1, uint32_t *o) {
  o[0] = kq4_lo16(d0);
  o[1] = kq4_hi16(d0);
  o[2] = kq4_lo16(d1);
  o[3] = kq4_hi16(d1);
}

// Exact integer block sum S of (row, block b) against 32 int8 activations q (8 dwords).
KQ4_DEV int kq4_stream_row_dot(const uint8_t *__restrict__ w, int row, int b, int nst,
                               const uint32_t *q) {
  int s = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint2 v = *reinterpret_cast<const uint2 *>(w + kq4_stream_nib(row, b, h, nst));
    uint32_t o[4];
    kq4_unpack_half(v.x, v.y, o);
#pragma unroll
    for (int k = 0; k < 4; ++k) s = kq4_dot4(o[k], q[4 * h + k], s);
  }
  return s >> 4;   // exact: 16*S
}
