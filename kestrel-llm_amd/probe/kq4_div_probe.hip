// kq4_div_probe.hip - exhaustive check of the quantizers' quotient on gfx950 (a verification
// tool, not library code).
//
// The activation quantizers (kq4_quantize_kernel and the GEMV's in-kernel quantization) compute
// each x/d as the Markstein-corrected quotient
//     y = RN(1/d);  q = RN(x*y);  q = RN(q + RN(x - q*d)*y)   (the last two as fmas)
// where the reference (quantize_row_q8_0_act, kestrel-llm src/model/vllm_safetensors.c:7893-7920)
// divides. Away from overflow and underflow, whether a rounded quotient is the correctly rounded
// one depends only on the two significands (scaling x or d by a power of two scales every step
// exactly), so this tool compares the sequence with the correctly rounded IEEE division (hipcc's
// default f32 divide) for every pair of float32 significands, x and d in [1, 2): 2^46 pairs in
// 64 launches of 2^40, one progress line each. It also counts the two-correction form (a second
// residual and fma) for comparison. Exit status 0 and "mismatches ... 0" on every line is the
// pass. Runs for about a minute on one MI355X.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#define CK(x)                                                               \
  do {                                                                      \
    hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                 \
      printf("HIP error %s: %s\n", #x, hipGetErrorString(e_));              \
      exit(2);                                                              \
    }                                                                       \
  } while (0)

// thread = one d significand; loops over nx x significands from x0
__global__ __launch_bounds__(256) void div_check(uint32_t x0, uint32_t nx,
                                                 unsigned long long *bad1,
                                                 unsigned long long *bad2, uint32_t *first) {
  const uint32_t di = blockIdx.x * 256u + threadIdx.x;   // < 2^23
  const float d = __uint_as_float(0x3f800000u | di);
  const float y = 1.0f / d;
  uint32_t n1 = 0, n2 = 0;
  for (uint32_t i = 0; i < nx; ++i) {
    const float x = __uint_as_float(0x3f800000u | (x0 + i));
    const float qi = x / d;
    float q = x * y;
    q = fmaf(fmaf(-q, d, x), y, q);
    const float q2 = fmaf(fmaf(-q, d, x), y, q);
    if (__float_as_uint(q) != __float_as_uint(qi)) {
      ++n1;
      if (atomicCAS(first, 0u, 1u) == 0u) {
        first[1] = __float_as_uint(x);
        first[2] = __float_as_uint(d);
      }
    }
    n2 += __float_as_uint(q2) != __float_as_uint(qi);
  }
  if (n1) atomicAdd(bad1, (unsigned long long)n1);
  if (n2) atomicAdd(bad2, (unsigned long long)n2);
}

int main() {
  unsigned long long *b1, *b2;
  uint32_t *first;
  CK(hipMalloc(&b1, 8));
  CK(hipMalloc(&b2, 8));
  CK(hipMalloc(&first, 16));
  CK(hipMemset(b1, 0, 8));
  CK(hipMemset(b2, 0, 8));
  CK(hipMemset(first, 0, 16));
  const uint32_t nd = 1u << 23, chunk = 1u << 17;
  unsigned long long h1 = 0, h2 = 0;
  for (uint32_t x0 = 0; x0 < (1u << 23); x0 += chunk) {
    hipLaunchKernelGGL(div_check, dim3(nd / 256), dim3(256), 0, 0, x0, chunk, b1, b2, first);
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(&h1, b1, 8, hipMemcpyDeviceToHost));
    CK(hipMemcpy(&h2, b2, 8, hipMemcpyDeviceToHost));
    printf("x significands [%u, %u): mismatches one-correction %llu, two-correction %llu\n", x0,
           x0 + chunk, h1, h2);
    fflush(stdout);
  }
  uint32_t f[3];
  CK(hipMemcpy(f, first, 12, hipMemcpyDeviceToHost));
  if (f[0]) printf("first one-correction mismatch: x=%08x d=%08x\n", f[1], f[2]);
  printf("checked %llu pairs\n", (unsigned long long)nd << 23);
  return h1 ? 1 : 0;
}
