// kq4_moe.hip - MoE FFN (q4 experts, int8 activation track) for gfx950.
//
// Restates the grouped expert path of kestrel-llm (st_moe_ffn_sparse_q4
// src/model/vllm_safetensors.c:12921-13398 and its batched twin st_moe_ffn_sparse_q4_batch_arm
// :14894-15064, int8 track VLLM_ACTQ=1):
//   route   top-k by insertion (ties -> smaller id), p = fl(exp(l - max) * fl(1/sum))
//   group   expert -> (token, rank) table in (token, rank) order          (:15004-15018)
//   gu      per (t,j), expert e: g/u rows [e*ef, e*ef+ef), V4 chain
//           acc = fl(acc + fl(fl(sc*xd) * S)) over blocks ascending        (:11861-11924)
//           av = fl(fl(g / fl(1 + exp(-g))) * u), re-quantized per 32 rows  (:12671-12675)
//   down    unweighted P[(t,j)][n] over the column band of expert e, V4 chain (:14799-14840)
//   combine y = fl(y + fl(p * P)) for j ascending from 0                    (:14875-14886)
// Every fp32 chain is the reference's: the per-block terms fl(fl(sc*xd)*S) are computed in
// parallel (they are independent and exact to compute), staged in LDS, and each output then adds
// its terms in block order in one lane. exp() is evaluated in double and rounded to float
// (correctly rounded; the reference's libm expf agrees except in rare last-ulp cases).
// G/U ([ne*ef rows][d cols]) and D ([d rows][ne*ef cols]) are in the stream layout; tiles are
// addressed per (row, block) through kq4_stream_nib / kq4_stream_scale.
#include "kq4_common.h"
#include "kq4_internal.h"

#define KQ4_MOE_MAXTK 32

KQ4_DEV float kq4_expf(float x) { return (float)exp((double)x); }

// ---- routing + expert grouping (one workgroup) -------------------------------------------
__global__ __launch_bounds__(256) void kq4_moe_route_kernel(int *__restrict__ sel,
                                                            float *__restrict__ pr,
                                                            const float *__restrict__ logits,
                                                            int T, int ne, int tk) {
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const float *lg = logits + (size_t)t * ne;
    int sl[KQ4_MOE_MAXTK];
    float sv[KQ4_MOE_MAXTK];
    for (int k = 0; k < tk; ++k) { sl[k] = -1; sv[k] = -INFINITY; }
    for (int e = 0; e < ne; ++e) {
      const float v = lg[e];
      for (int k = 0; k < tk; ++k) {
        if (v > sv[k] || (v == sv[k] && (sl[k] < 0 || e < sl[k]))) {
          for (int q = tk - 1; q > k; --q) { sl[q] = sl[q - 1]; sv[q] = sv[q - 1]; }
          sl[k] = e;
          sv[k] = v;
          break;
        }
      }
    }
    float mx = -INFINITY;
    for (int k = 0; k < tk; ++k) mx = sv[k] > mx ? sv[k] : mx;
    float p[KQ4_MOE_MAXTK];
    float sum = 0.0f;
    for (int k = 0; k < tk; ++k) { p[k] = kq4_expf(sv[k] - mx); sum += p[k]; }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int k = 0; k < tk; ++k) {
      sel[(size_t)t * tk + k] = sl[k];
      pr[(size_t)t * tk + k] = p[k] * inv;
    }
  }
}

__global__ __launch_bounds__(256) void kq4_moe_group_kernel(int *__restrict__ ex_off,
                                                            int *__restrict__ ex_pair,
                                                            const int *__restrict__ sel,
                                                            int n_pairs, int ne) {
  extern __shared__ int s_cnt[];   // ne + 1
  for (int e = threadIdx.x; e < ne; e += blockDim.x) {
    int c = 0;
    for (int i = 0; i < n_pairs; ++i) c += (sel[i] == e);
    s_cnt[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int e = 0; e < ne; ++e) {
      const int c = s_cnt[e];
      s_cnt[e] = acc;
      ex_off[e] = acc;
      acc += c;
    }
    ex_off[ne] = acc;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < ne; e += blockDim.x) {
    int pos = s_cnt[e];
    for (int i = 0; i < n_pairs; ++i)
      if (sel[i] == e) ex_pair[pos++] = i;
  }
}

// ---- one weight row-block of the stream layout ---------------------------------------------
// The 32 weights of (row, block b) as 16*(n-8) int8 (8 dwords, element order) and its scale.
KQ4_DEV float kq4_load_rowblk(uint32_t *o, const uint8_t *__restrict__ w, int row, int b,
                              int nst) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint2 v = *reinterpret_cast<const uint2 *>(w + kq4_stream_nib(row, b, h, nst));
    kq4_unpack_half(v.x, v.y, o + 4 * h);
  }
  return kq4_h2f(*reinterpret_cast<const uint16_t *>(w + kq4_stream_scale(row, b, nst)));
}

KQ4_DEV int kq4_rowblk_dot(const uint32_t *o, const uint32_t *qa) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) acc = kq4_dot4(o[k], qa[k], acc);
  return acc >> 4;   // exact: 16*S
}

KQ4_DEV void kq4_load_q(uint32_t *qa, const int8_t *src) {
  const uint4 *p = reinterpret_cast<const uint4 *>(src);
  const uint4 a = p[0], b = p[1];
  qa[0] = a.x; qa[1] = a.y; qa[2] = a.z; qa[3] = a.w;
  qa[4] = b.x; qa[5] = b.y; qa[6] = b.z; qa[7] = b.w;
}

// ---- gate/up + SiLU + av quantization ----------------------------------------------------
// grid: ne * (ef/32) workgroups; workgroup (e, rb) owns expert e's rows rb*32 .. +32 of G and
// U (8 tile groups each) and every (token, rank) routed to e, in chunks of `pc` pairs.
__global__ __launch_bounds__(256) void kq4_moe_gu_kernel(
    const uint8_t *__restrict__ G, const uint8_t *__restrict__ U, const int8_t *__restrict__ xq,
    const float *__restrict__ xd, const int *__restrict__ ex_off, const int *__restrict__ ex_pair,
    float *__restrict__ av, int8_t *__restrict__ avq, float *__restrict__ avd,
    float *__restrict__ g_out, float *__restrict__ u_out, int ne, int d, int ef, int tk, int pc) {
  extern __shared__ float s_term[];   // [pc][64 rows][nbG]
  const int rbs = ef / 32;
  const int e = blockIdx.x / rbs, rb = blockIdx.x % rbs;
  const int o0 = ex_off[e], m = ex_off[e + 1] - o0;
  if (m <= 0) return;
  const int nbG = d / 32;
  const int nstG = (nbG + KQ4_STREAM_CB - 1) / KQ4_STREAM_CB;
  const int t = threadIdx.x;

  for (int c0 = 0; c0 < m; c0 += pc) {
    const int np = (m - c0) < pc ? (m - c0) : pc;
    // phase A: terms for 64 rows (32 gate, 32 up) x nbG blocks
    for (int c = t; c < 64 * nbG; c += 256) {
      const int q = c / nbG, b = c - q * nbG;
      const uint8_t *mat = q < 32 ? G : U;
      const int row = e * ef + rb * 32 + (q & 31);
      uint32_t wv[8];
      const float sc = kq4_load_rowblk(wv, mat, row, b, nstG);
      for (int p = 0; p < np; ++p) {
        const int tok = ex_pair[o0 + c0 + p] / tk;
        uint32_t qa[8];
        kq4_load_q(qa, xq + (size_t)tok * d + (size_t)b * 32);
        const float x = xd[(size_t)tok * nbG + b];
        s_term[((size_t)p * 64 + q) * nbG + b] = (sc * x) * (float)kq4_rowblk_dot(wv, qa);
      }
    }
    __syncthreads();
    // phase B: block-ordered sums, SiLU, quantize each pair's 32 av values (one half-wave)
    if (t < 32 * np) {
      const int p = t >> 5, r = t & 31;
      const float *tg = s_term + ((size_t)p * 64 + r) * nbG;
      const float *tu = s_term + ((size_t)p * 64 + 32 + r) * nbG;
      float g = 0.0f, u = 0.0f;
      for (int b = 0; b < nbG; ++b) { g = g + tg[b]; u = u + tu[b]; }
      const float a = (g / (1.0f + kq4_expf(-g))) * u;
      const int pair = ex_pair[o0 + c0 + p];
      const size_t o = (size_t)pair * ef + (size_t)rb * 32 + r;
      av[o] = a;
      if (g_out) { g_out[o] = g; u_out[o] = u; }
      float amax = fmaxf(fabsf(a), 1e-10f);
#pragma unroll
      for (int s = 16; s > 0; s >>= 1) amax = fmaxf(amax, __shfl_xor(amax, s, 32));
      const float dq = amax / 127.0f;
      int qv = (int)(a / dq + 0.5f);
      qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
      avq[o] = (int8_t)qv;
      if (r == 0) avd[(size_t)pair * rbs + rb] = dq;
    }
    __syncthreads();
  }
}

// Re-quantize caller-provided av (stage-wise verification of the down projection).
__global__ __launch_bounds__(256) void kq4_moe_avq_kernel(const float *__restrict__ av,
                                                          int8_t *__restrict__ avq,
                                                          float *__restrict__ avd, long nblk) {
  const int lane = threadIdx.x & 31;
  const long blk = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (blk >= nblk) return;
  const float a = av[blk * 32 + lane];
  float amax = fmaxf(fabsf(a), 1e-10f);
#pragma unroll
  for (int s = 16; s > 0; s >>= 1) amax = fmaxf(amax, __shfl_xor(amax, s, 32));
  const float dq = amax / 127.0f;
  int qv = (int)(a / dq + 0.5f);
  qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
  avq[blk * 32 + lane] = (int8_t)qv;
  if (lane == 0) avd[blk] = dq;
}

// ---- down projection: unweighted partials ------------------------------------------------
// grid: ne * (d/32); workgroup (e, rb) owns output rows rb*32 .. +32 (8 tile groups of D) over
// expert e's column band (tiles e*ef/32 .. +ef/32) for every (token, rank) routed to e.
__global__ __launch_bounds__(256) void kq4_moe_down_kernel(
    const uint8_t *__restrict__ D, const int8_t *__restrict__ avq, const float *__restrict__ avd,
    const int *__restrict__ ex_off, const int *__restrict__ ex_pair, float *__restrict__ P,
    int ne, int d, int ef, int pc) {
  extern __shared__ float s_term[];   // [pc][32 rows][cbe]
  const int rbs = d / 32;
  const int e = blockIdx.x / rbs, rb = blockIdx.x % rbs;
  const int o0 = ex_off[e], m = ex_off[e + 1] - o0;
  if (m <= 0) return;
  const int cbe = ef / 32;
  const int nstD = (ne * ef / 32 + KQ4_STREAM_CB - 1) / KQ4_STREAM_CB;
  const size_t cb0 = (size_t)e * ef / 32;
  const int t = threadIdx.x;
  for (int c0 = 0; c0 < m; c0 += pc) {
    const int np = (m - c0) < pc ? (m - c0) : pc;
    for (int c = t; c < 32 * cbe; c += 256) {
      const int q = c / cbe, cb = c - q * cbe;
      uint32_t wv[8];
      const float sc = kq4_load_rowblk(wv, D, rb * 32 + q, (int)cb0 + cb, nstD);
      for (int p = 0; p < np; ++p) {
        const int pair = ex_pair[o0 + c0 + p];
        uint32_t qa[8];
        kq4_load_q(qa, avq + (size_t)pair * ef + (size_t)cb * 32);
        const float x = avd[(size_t)pair * cbe + cb];
        s_term[((size_t)p * 32 + q) * cbe + cb] = (sc * x) * (float)kq4_rowblk_dot(wv, qa);
      }
    }
    __syncthreads();
    if (t < 32 * np) {
      const int p = t >> 5, r = t & 31;
      const float *tp = s_term + ((size_t)p * 32 + r) * cbe;
      float acc = 0.0f;
      for (int cb = 0; cb < cbe; ++cb) acc = acc + tp[cb];
      const int pair = ex_pair[o0 + c0 + p];
      P[(size_t)pair * d + (size_t)rb * 32 + r] = acc;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void kq4_moe_combine_kernel(float *__restrict__ Y,
                                                              const float *__restrict__ P,
                                                              const int *__restrict__ sel,
                                                              const float *__restrict__ pr,
                                                              int T, int tk, int d, int ne) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)T * d) return;
  const int t = (int)(i / d), n = (int)(i - (long)t * d);
  float y = 0.0f;
  for (int j = 0; j < tk; ++j) {
    const int s = t * tk + j;
    const int e = sel[s];
    if (e < 0 || e >= ne) continue;
    y = y + pr[s] * P[(size_t)s * d + n];
  }
  Y[i] = y;
}

int kq4_launch_moe_route(int *sel, float *pr, const float *logits, int T, int ne, int tk,
                         hipStream_t s) {
  if (tk > KQ4_MOE_MAXTK) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kq4_moe_route_kernel, dim3(1), dim3(256), 0, s, sel, pr, logits, T, ne, tk);
  return (int)hipGetLastError();
}

static int moe_pc(int per_pair_floats) {
  const int budget = 48 * 1024 / 4;   // floats of LDS for staged terms
  int pc = budget / per_pair_floats;
  if (pc > 8) pc = 8;
  if (pc < 1) pc = 1;
  return pc;
}

int kq4_launch_moe_dbg(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                       const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d,
                       int ef, const KQ4MoeWs &ws, float *g_out, float *u_out,
                       const float *av_in, hipStream_t s) {
  const int n_pairs = T * tk;
  hipLaunchKernelGGL(kq4_moe_group_kernel, dim3(1), dim3(256), (ne + 1) * sizeof(int), s,
                     ws.ex_off, ws.ex_pair, sel, n_pairs, ne);
  int rc = kq4_launch_quantize(X, ws.xq, ws.xd, nullptr, T, d, 0, s);
  if (rc) return rc;
  const int nbG = d / 32, cbe = ef / 32;
  const int pcg = moe_pc(64 * nbG) > 4 ? 4 : moe_pc(64 * nbG);   // phase B: 32*pc <= 256 lanes
  hipLaunchKernelGGL(kq4_moe_gu_kernel, dim3(ne * (ef / 32)), dim3(256),
                     (size_t)pcg * 64 * nbG * sizeof(float), s, G, U, ws.xq, ws.xd, ws.ex_off,
                     ws.ex_pair, ws.av, ws.avq, ws.avd, g_out, u_out, ne, d, ef, tk, pcg);
  if (av_in) {
    const long nblk = (long)n_pairs * cbe;
    hipLaunchKernelGGL(kq4_moe_avq_kernel, dim3((unsigned)((nblk + 7) / 8)), dim3(256), 0, s,
                       av_in, ws.avq, ws.avd, nblk);
  }
  const int pcd = moe_pc(32 * cbe) > 8 ? 8 : moe_pc(32 * cbe);
  hipLaunchKernelGGL(kq4_moe_down_kernel, dim3(ne * (d / 32)), dim3(256),
                     (size_t)pcd * 32 * cbe * sizeof(float), s, D, ws.avq, ws.avd, ws.ex_off,
                     ws.ex_pair, ws.P, ne, d, ef, pcd);
  const long n = (long)T * d;
  hipLaunchKernelGGL(kq4_moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     Y, ws.P, sel, pr, T, tk, d, ne);
  return (int)hipGetLastError();
}

int kq4_launch_moe(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                   const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                   const KQ4MoeWs &ws, hipStream_t s) {
  return kq4_launch_moe_dbg(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, ws, nullptr, nullptr,
                            nullptr, s);
}
