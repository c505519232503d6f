// kq4_issue_probe.hip - how the matrix cores and the VALU share one SIMD's issue on gfx950,
// measured with the prefill GEMM's own instruction mix (a measurement tool, not library code).
//
// Every wave runs `iters` iterations of one instruction mix on registers only (no memory
// traffic in the loop); the grid puts w waves on every SIMD (w = 1, 2). Per mix the tool prints
// cycles per wave and iteration, calibrated against the VALU-only mix (64 dependent-free fp32
// fmas = 256 issue cycles: a wave64 VALU instruction issues over 4 cycles), so the GPU's clock
// drops out. Mixes:
//   mfma      4 v_mfma_i32_32x32x32_i8 (accumulating)                      MFMA 128 cycles
//   valu      64 v_fma_f32                                                 VALU 256
//   indep     both of the above, independent of each other                 sum 384
//   int8      the int8 GEMM's block of one wave (64 x 64 outputs), in its pipelined order: 4
//             int8 MFMAs (zero accumulator), each issued one tile epilogue ahead of its use, 2
//             v_mfma_f32_32x32x1_2b_f32 scale outer products, and per output a convert and an
//             fma                                                           128 + 128 + 512 = 768
//   fp8       the fp8-operand form's block: 4 v_mfma_scale_f32_32x32x64_f8f6f4 (fp8) + 2 outer
//             products + one fma per output                                256 + 128 + 256 = 640
//   f16       an f16-operand form's block: 8 v_mfma_f32_32x32x16_f16 (two per tile, the second
//             accumulating; issued two and one tiles ahead) + 2 outer products + one fma per
//             output                                                       256 + 128 + 256 = 640
// The last column is the sum of the MFMA cycles (32 per int8 32x32x32 and f16 32x32x16, 64 per
// fp8 32x32x64 and per f32 32x32x1_2b) and the VALU issue cycles: the time if the two units did
// not overlap at all.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

enum { MFMA, VALU, INDEP, INT8, FP8, F16, NMIX };
static const char *kName[NMIX] = {"mfma", "valu", "indep", "int8", "fp8", "f16"};
static const double kSum[NMIX] = {128, 256, 384, 768, 640, 640};

template <int MIX>
__global__ __launch_bounds__(256, 2) void probe(float *out, unsigned long long *clk, int iters,
                                                 float c1, float c2) {
  const int t = threadIdx.x;
  // shader-clock and 100 MHz real-time counters around the loop (the first wave of each
  // workgroup), so the cycles per iteration and the clock need no calibration
  unsigned long long c0 = 0, r0 = 0;
  if (t == 0) {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  v4i a = {t, 3 * t, 5 * t, 7 * t};
  const v4i b = {t ^ 1, t ^ 2, t ^ 3, t ^ 4};
  v8i a8;
#pragma unroll
  for (int i = 0; i < 8; ++i) a8[i] = 0x38383838 ^ (t << (i & 3));
  const v16i z = {0};
  const v16f zf = {0};
  const v32f z32 = {0};
  v16i s[4];
  v16f sf[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s[j] = z;
    sf[j] = zf;
  }
  float f[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) f[i] = (float)(t + i);
  v32f sc0 = __builtin_amdgcn_mfma_f32_32x32x1f32(c1, c2, z32, 0, 0, 0);
  v32f sc1 = __builtin_amdgcn_mfma_f32_32x32x1f32(c2, c1, z32, 0, 0, 0);
  for (int it = 0; it < iters; ++it) {
    if (MIX == MFMA || MIX == INDEP) {
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a + j, b, s[j], 0, 0, 0);
    }
    if (MIX == VALU || MIX == INDEP) {
#pragma unroll
      for (int i = 0; i < 64; ++i) f[i] = fmaf(f[i], c1, c2);
    }
    if (MIX == INT8 || MIX == FP8 || MIX == F16) {
      // The GEMM's order: the sums of tile j+1 are issued before tile j's epilogue (sum slots
      // alternate; f16: tile j+2's first half too), and a row tile's scale products for the
      // next block right after its last epilogue.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int jn = (j + 1) & 3;   // the next tile (tile 0 of the next iteration at j = 3)
        if (MIX == INT8) s[jn & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a + jn, b, z, 0, 0, 0);
        if (MIX == FP8)
          sf[jn & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8 + jn, a8, zf, 0, 0, 0, 0, 0, 0);
        if (MIX == F16) {
          const int j2 = (j + 2) & 3;
          sf[jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              __builtin_bit_cast(h8, b), __builtin_bit_cast(h8, a + jn), sf[jn], 0, 0, 0);
          sf[j2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a + j2),
                                                          __builtin_bit_cast(h8, b), zf, 0, 0, 0);
        }
        const v16f cur = MIX == INT8 ? zf : (MIX == FP8 ? sf[j & 1] : sf[j]);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = (j < 2 ? sc0 : sc1)[16 * (j & 1) + v];
          f[16 * j + v] = MIX == INT8 ? fmaf((float)s[j & 1][v], p, f[16 * j + v])
                                      : fmaf(cur[v], p, f[16 * j + v]);
        }
        if (j == 1) sc0 = __builtin_amdgcn_mfma_f32_32x32x1f32(c1 + (float)it, c2, z32, 0, 0, 0);
        if (j == 3) sc1 = __builtin_amdgcn_mfma_f32_32x32x1f32(c2 + (float)it, c1, z32, 0, 0, 0);
      }
      a.x += 1;
      a8[0] += 1;
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) r += f[i];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) r += (float)s[j][v] + sf[j][v];
#pragma unroll
  for (int v = 0; v < 32; ++v) r += sc0[v] + sc1[v];
  out[blockIdx.x * 256 + t] = r;
  if (t == 0) {
    const unsigned long long c1t = __builtin_amdgcn_s_memtime();
    const unsigned long long r1t = __builtin_amdgcn_s_memrealtime();
    clk[2 * blockIdx.x] = c1t - c0;
    clk[2 * blockIdx.x + 1] = r1t - r0;
  }
}

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_));    \
      exit(1);                                                                     \
    }                                                                              \
  } while (0)

struct Res {
  float ms;          // per launch, host events
  double cyc_iter;   // shader cycles per iteration of one wave (median over workgroups)
  double ghz;        // shader clock (median)
};

template <int MIX>
static Res run(float *out, unsigned long long *clk, int blocks, int iters, int reps) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL(probe<MIX>, dim3(blocks), dim3(256), 0, 0, out, clk, iters, 1.0001f, 0.5f);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e0));
  for (int r = 0; r < reps; ++r)
    hipLaunchKernelGGL(probe<MIX>, dim3(blocks), dim3(256), 0, 0, out, clk, iters, 1.0001f, 0.5f);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  // the last launch's per-workgroup counters
  unsigned long long *h = (unsigned long long *)malloc((size_t)blocks * 2 * sizeof(*h));
  CHECK(hipMemcpy(h, clk, (size_t)blocks * 2 * sizeof(*h), hipMemcpyDeviceToHost));
  double *cy = (double *)malloc(blocks * sizeof(double)), *gz = (double *)malloc(blocks * sizeof(double));
  for (int b = 0; b < blocks; ++b) {
    cy[b] = (double)h[2 * b] / iters;
    gz[b] = (double)h[2 * b] / ((double)h[2 * b + 1] * 10.0);   // real-time counter: 100 MHz
  }
  auto median = [&](double *v) {
    for (int i = 1; i < blocks; ++i)
      for (int j = i; j > 0 && v[j - 1] > v[j]; --j) {
        const double x = v[j];
        v[j] = v[j - 1];
        v[j - 1] = x;
      }
    return v[blocks / 2];
  };
  Res r{ms / reps, median(cy), median(gz)};
  free(h);
  free(cy);
  free(gz);
  return r;
}

int main() {
  int dev = 0, ncu = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  const int iters = 4000, reps = 5;
  printf("CUs %d. Per mix: SIMD cycles per wave and iteration (the shader clock's count over the\n"
         "loop / iterations / waves per SIMD), the same from host events and the VALU mix's\n"
         "calibration (256), the clock, and the sum of MFMA and VALU cycles\n",
         ncu);
  for (int w = 1; w <= 2; ++w) {
    const int blocks = ncu * w;   // 4 waves per workgroup, one per SIMD
    float *out = nullptr;
    unsigned long long *clk = nullptr;
    CHECK(hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)));
    CHECK(hipMalloc(&clk, (size_t)blocks * 2 * sizeof(unsigned long long)));
    Res r[NMIX];
    r[MFMA] = run<MFMA>(out, clk, blocks, iters, reps);
    r[VALU] = run<VALU>(out, clk, blocks, iters, reps);
    r[INDEP] = run<INDEP>(out, clk, blocks, iters, reps);
    r[INT8] = run<INT8>(out, clk, blocks, iters, reps);
    r[FP8] = run<FP8>(out, clk, blocks, iters, reps);
    r[F16] = run<F16>(out, clk, blocks, iters, reps);
    printf("waves/SIMD %d\n", w);
    for (int m = 0; m < NMIX; ++m)
      printf("  %-6s %7.1f cycles (counter)  %7.1f (events, calibrated)  %.2f GHz   sum %5.0f   "
             "counter / sum %.3f\n",
             kName[m], r[m].cyc_iter / w, 256.0 * r[m].ms / r[VALU].ms, r[m].ghz, kSum[m],
             r[m].cyc_iter / w / kSum[m]);
    CHECK(hipFree(out));
    CHECK(hipFree(clk));
  }
  return 0;
}
