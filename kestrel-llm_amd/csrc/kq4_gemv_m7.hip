// kq4_gemv_m7.hip - the decode GEMV kernels for 7 token(s) (kq4_gemv_impl.h), a translation unit
// of its own so the instantiations compile in parallel.
#include "kq4_gemv_impl.h"

template hipError_t kq4_gv_launch_m<7>(const KQ4GemvArgs &, int, int, int, int, int, hipStream_t);
