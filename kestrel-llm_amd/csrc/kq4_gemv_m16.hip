// kq4_gemv_m16.hip - the 16-token decode GEMV (kq4_gemv_impl.h) for q4 batches of 9-16 tokens in
// one launch: a.ntok tokens, the rest of the 16 padding (never loaded or stored). MFMA kind only
// (token t of a half set's parity p in A row 16p + t), whole or half single sets, activations
// pre-quantized or quantized in the kernel.
#include "kq4_gemv_impl.h"

hipError_t kq4_gv_launch_wide(const KQ4GemvArgs &a, int fq, int hs, int grid, hipStream_t s) {
  if (a.wf || fq < 0 || fq > 1 || hs < 0 || hs > 1 || a.ntok <= KQ4_GEMV_MAX_M ||
      a.ntok > KQ4_GEMV_WIDE_M)
    return hipErrorInvalidValue;
  if (fq)
    return hs ? kq4_gv_launch1<16, 1, 1, 1, 0, 1>(a, grid, s)
              : kq4_gv_launch1<16, 1, 1, 0, 0, 1>(a, grid, s);
  return hs ? kq4_gv_launch1<16, 0, 1, 1, 0, 1>(a, grid, s)
            : kq4_gv_launch1<16, 0, 1, 0, 0, 1>(a, grid, s);
}
