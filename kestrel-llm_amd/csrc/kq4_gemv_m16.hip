// kq4_gemv_m16.hip - the 16-token decode GEMV (kq4_gemv_impl.h) for q4 batches of 9-16 tokens in
// one launch: a.ntok tokens, the rest of the 16 padding (never loaded or stored). MFMA kind only
// (token t of a half set's parity p in A row 16p + t), half sets or 1-3 whole sets per
// workgroup, activations pre-quantized or quantized in the kernel.
#include "kq4_gemv_impl.h"

template <int FQ>
static hipError_t kq4_gv_launch_wide_fq(const KQ4GemvArgs &a, int hs, int rps, int grid,
                                        hipStream_t s) {
  if (hs) return kq4_gv_launch1<16, FQ, 1, 1, 0, 1>(a, grid, s);
  if (rps == 3) return kq4_gv_launch1<16, FQ, 1, 0, 0, 3>(a, grid, s);
  if (rps == 2) return kq4_gv_launch1<16, FQ, 1, 0, 0, 2>(a, grid, s);
  return kq4_gv_launch1<16, FQ, 1, 0, 0, 1>(a, grid, s);
}

hipError_t kq4_gv_launch_wide(const KQ4GemvArgs &a, int fq, int hs, int rps, int grid,
                              hipStream_t s) {
  if (a.wf || fq < 0 || fq > 1 || hs < 0 || hs > 1 || rps < 1 || rps > 3 || (hs && rps != 1) ||
      a.ntok <= KQ4_GEMV_MAX_M || a.ntok > KQ4_GEMV_WIDE_M)
    return hipErrorInvalidValue;
  return fq ? kq4_gv_launch_wide_fq<1>(a, hs, rps, grid, s)
            : kq4_gv_launch_wide_fq<0>(a, hs, rps, grid, s);
}
