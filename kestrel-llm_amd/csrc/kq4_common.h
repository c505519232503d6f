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

// 4 x int8 dot product accumulated into c (v_dot4_i32_i8).
KQ4_DEV int kq4_dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Butterfly all-reduce over the 16 lanes of a DPP row; every lane ends with the same bits.
KQ4_DEV float kq4_row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // quad xor 1
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // quad xor 2
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)); // half-row mirror
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)); // row mirror
  return v;
}

struct KQ4Tile2 {   // two consecutive 72-byte tiles (144 B = 9 x 16 B)
  uint32_t d[36];
};
