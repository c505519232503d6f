// kq4_moe.hip - MoE FFN (q4 experts, int8 activation track) for gfx950.
//
// Restates the grouped expert path of kestrel-llm (st_moe_ffn_sparse_q4
// src/model/vllm_safetensors.c:12921-13398 and its batched twin st_moe_ffn_sparse_q4_batch_arm
// :14894-15064, int8 track VLLM_ACTQ=1):
//   route   top-k by insertion (ties -> smaller id), p = fl(exp(l - max) * fl(1/sum))
//   group   expert -> (token, rank) table                                  (:15004-15018)
//   gu      per (t,j), expert e: g/u rows [e*ef, e*ef+ef), V4 chain
//           acc = fl(acc + fl(fl(sc*xd) * S)) over blocks ascending        (:11861-11924)
//           av = fl(fl(g / fl(1 + exp(-g))) * u), re-quantized per 32 rows  (:12671-12675)
//   down    unweighted P[(t,j)][n] over the column band of expert e, V4 chain (:14799-14840)
//   combine y = fl(y + fl(p * P)) for j ascending from 0                    (:14875-14886)
// Every fp32 chain is the reference's, bit for bit. exp() is evaluated in double and rounded to
// float (correctly rounded; the reference's libm expf agrees except in rare last-ulp cases).
//
// Four launches: prep (grouping + activation quantizer), gate/up, down, combine. The weights are
// in the stream layout (kq4_common.h): G/U as [ne*ef rows][d cols], D as [d rows][ne*ef cols].
// The gate/up and down kernels stream them the way the decode GEMV does: one workgroup per
// (active expert, 32-row set), its waves splitting K, each wave holding its chunk's weights in
// registers as loaded (full-width coalesced loads), the integer dots on
// v_mfma_i32_32x32x32_i8 with A = the expert's (token, rank) pairs' codes (4 or 8 per pass)
// and B = the lanes' weight registers. The reference's serial chain over the blocks is kept
// exactly: each wave computes its blocks' terms fl(fl(sc*xd)*S) in registers, then the waves
// add them to the running sum one after another in block order, handing the sum on through LDS
// (one barrier per wave). SiLU, the product and the av re-quantization are fused into the gate/up
// kernel's end (a 32-row set is exactly one quantization block of av).
#include "kq4_common.h"
#include "kq4_internal.h"

#include <stdlib.h>
#include <type_traits>

#define KQ4_MOE_MAXTK 32
#define KQ4_MOE_MAXNE 2048  // routing: a lane's experts fit one 32-bit mask
#define KQ4_MOE_PCG 4       // gate/up pairs per pass: MFMA token rows 4*(lane/32)+v, v < 2
#define KQ4_MOE_PCD 8       // down pairs per pass: token rows 4*(lane/32)+v, v < 4
#define KQ4_MOE_QTS 672     // LDS bytes per pair row of a 16-block stage's codes
#define KQ4_MOE_QTS8 320    // the same for an 8-block half stage
#define KQ4_MOE_DOWNW_DEFAULT 4   // row sets (waves) per workgroup of kq4_moe_downw_kernel

typedef int kq4_v4i __attribute__((ext_vector_type(4)));
typedef int kq4_v16i __attribute__((ext_vector_type(16)));

// LDS slab of one stage's activations for pc pairs: codes [pair][qpos(block)] then scales
// [block][pair].
constexpr int kq4_moe_slab(int blocks, int pc) {
  return pc * (blocks == 16 ? KQ4_MOE_QTS : KQ4_MOE_QTS8) + blocks * pc * 4;
}

KQ4_DEV float kq4_expf(float x) { return (float)exp((double)x); }

// Block pairs at an 80-B pitch: the two K halves' 16-B reads spread over the banks.
KQ4_DEV int kq4_moe_qpos(int blk) { return (blk >> 1) * 80 + (blk & 1) * 32; }

KQ4_DEV kq4_v16i kq4_moe_mfma(kq4_v4i a, kq4_v4i b) {
  const kq4_v16i z = {0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

// Materialises x here (keeps the unrolled block loop from sinking every term to its end).
KQ4_DEV void kq4_moe_pin(float &x) { asm volatile("" : "+v"(x)); }

// Marks the packed weights as changed here, so the per-pass unpacking is not hoisted out of the
// pass loop (the unpacked operands take twice the registers).
template <int N>
KQ4_DEV void kq4_moe_touch(uint32_t (&a)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(a[i]));
}

// ---- routing (one wave per token) -----------------------------------------------------------
// The k largest logits, ties to the smaller id, in order: the reference's insertion top-k
// (:12968-12984) gives the same list (a NaN logit is never inserted; -inf is, into an empty
// slot). Then p = fl(exp(l - max)) summed in rank order, scaled by fl(1/sum).
//
// Lane l holds the logits of experts l, l+64, .. in registers (read once). A candidate is the
// 64-bit key (order-preserving bits of the logit, ~id), so the wave maximum of the keys is the
// largest logit with ties to the smaller id; -0 is keyed as +0 (the reference compares values),
// NaN is never a candidate, and 0 means none. The maximum takes DPP quad permutes and row
// rotates and the two permlane swaps: VALU only. Each round only the winner's lane rescans.
template <int CTRL>
KQ4_DEV uint64_t kq4_dpp64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}

KQ4_DEV uint64_t kq4_max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

KQ4_DEV uint64_t kq4_wave_max_u64(uint64_t k) {
  k = kq4_max_u64(k, kq4_dpp64<0xB1>(k));    // quad_perm [1,0,3,2]
  k = kq4_max_u64(k, kq4_dpp64<0x4E>(k));    // quad_perm [2,3,0,1]
  k = kq4_max_u64(k, kq4_dpp64<0x124>(k));   // row_ror:4 (the quads of a 16-lane row)
  k = kq4_max_u64(k, kq4_dpp64<0x128>(k));   // row_ror:8
  {
    const uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    const auto a = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    k = kq4_max_u64(((uint64_t)b[0] << 32) | a[0], ((uint64_t)b[1] << 32) | a[1]);
  }
  {
    const uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    const auto a = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    k = kq4_max_u64(((uint64_t)b[0] << 32) | a[0], ((uint64_t)b[1] << 32) | a[1]);
  }
  return k;
}

KQ4_DEV uint64_t kq4_route_key(float v, int e) {
  const uint32_t u = __float_as_uint(v + 0.0f);   // -0 -> +0
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (0xFFFFFFFFu - (uint32_t)e);
}

KQ4_DEV float kq4_route_val(uint64_t key) {
  const uint32_t o = (uint32_t)(key >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

__global__ __launch_bounds__(256) void kq4_moe_route_kernel(int *__restrict__ sel,
                                                            float *__restrict__ pr,
                                                            const float *__restrict__ logits,
                                                            int T, int ne, int tk) {
  constexpr int NV = KQ4_MOE_MAXNE / 64;   // logits per lane at most
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;   // whole waves
  const float *lg = logits + (size_t)t * ne;
  const int nv = (ne + 63) >> 6;   // uniform
  float vals[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (i >= nv) break;
    const int e = lane + 64 * i;
    vals[i] = e < ne ? lg[e] : __builtin_nanf("");
  }
  uint32_t taken = 0;   // bit i: this lane's expert lane + 64*i is already selected
  auto local_best = [&]() {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (i >= nv) break;
      const float v = vals[i];
      if (!((taken >> i) & 1u) && v == v) best = kq4_max_u64(best, kq4_route_key(v, lane + 64 * i));
    }
    return best;
  };
  uint64_t mine = local_best();
  int sk[KQ4_MOE_MAXTK];
  float vk[KQ4_MOE_MAXTK];
#pragma unroll
  for (int k = 0; k < KQ4_MOE_MAXTK; ++k) {
    if (k >= tk) break;
    const uint64_t key = kq4_wave_max_u64(mine);
    const int be = key ? (int)(0xFFFFFFFFu - (uint32_t)key) : -1;
    sk[k] = be;
    vk[k] = be >= 0 ? kq4_route_val(key) : -INFINITY;   // the logit, until the pass below
    if (be >= 0 && (be & 63) == lane) {
      taken |= 1u << (be >> 6);
      mine = local_best();
    }
  }
  // softmax over the k picks: lane k forms p_k = fl(exp(l_k - max)) (the picks are the same in
  // every lane), the p_k are summed in rank order (lane reads), lane k writes fl(p_k * fl(1/sum))
  float mx = -INFINITY, lk = -INFINITY;
  int sid = -1;
#pragma unroll
  for (int k = 0; k < KQ4_MOE_MAXTK; ++k) {
    if (k >= tk) break;
    mx = vk[k] > mx ? vk[k] : mx;
    if (lane == k) { lk = vk[k]; sid = sk[k]; }
  }
  const float pk = lane < tk ? kq4_expf(lk - mx) : 0.0f;
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < KQ4_MOE_MAXTK; ++k) {
    if (k >= tk) break;
    sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pk), k));
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  if (lane < tk) {
    sel[(size_t)t * tk + lane] = sid;
    pr[(size_t)t * tk + lane] = pk * inv;
  }
}

// ---- router logits ----------------------------------------------------------------------------
// logits[t][e] = the reference's serial fp32 chain s = fl(s + fl(rw[e][i] * x[t][i])), i ascending
// (st_moe_ffn_sparse_q4 :12961-12966; the batched router :14937-14962 keeps the same chain per
// (token, expert)). A chain cannot be split without changing its roundings, so one lane runs one
// (token, expert) chain and does nothing else: a workgroup takes one token and 16 experts; lanes
// 0-15 of wave 0 add, waves 1-4 form the products. Per 512-column tile each producer thread
// loads 8 float4s of one row (256 B apart) and the matching x (issued a tile ahead, so the loads
// are in flight during a whole tile's 512 dependent adds, ~1.6 us), multiplies and stores the products
// to LDS (double-buffered; row pitch 516 floats, so the adders' 16-B reads hit distinct banks);
// each adder then adds its row's products in order.
#define KQ4_RT_E 16        // experts (chains) per workgroup
#define KQ4_RT_C 512       // columns per tile
#define KQ4_RT_P 516       // LDS row pitch (floats)

__global__ __launch_bounds__(320) void kq4_moe_logits_kernel(float *__restrict__ logits,
                                                             const float *__restrict__ router,
                                                             const float *__restrict__ X, int ne,
                                                             int d) {
  extern __shared__ __align__(16) float kq4_rt_lds[];   // [2][KQ4_RT_E][KQ4_RT_P] + 32 pad
  const int t = blockIdx.y;
  const int e0 = blockIdx.x * KQ4_RT_E;
  const int wave = threadIdx.x >> 6;
  const float *__restrict__ xt = X + (size_t)t * d;
  const int ntile = (d + KQ4_RT_C - 1) / KQ4_RT_C;
  // producer thread p: row p/16 of the tile, the float4s q, q+16, .. (q = p%16) of its 512
  // columns, so the 16 threads of a row store 256 contiguous bytes per instruction (a thread
  // owning 32 consecutive columns put all 16 on the same LDS banks, and those stores delayed the
  // adders' reads)
  const int p = threadIdx.x - 64;
  const int pr = p >> 4, pc = 4 * (p & 15);
  const bool prow = wave > 0 && e0 + pr < ne;
  const float *__restrict__ rw = router + (size_t)(e0 + pr) * d;
  // One register array for both roles (no wave has both; as separate arrays the kernel took 138
  // VGPRs, and two 5-wave workgroups did not fit a CU): a producer's next-tile weights rb[0..7]
  // and x rb[8..15], loaded a tile ahead; the adder's two chunks of products.
  float4 rb[16];
  float4 *cur = rb, *xv = rb + 8;
  auto load = [&](int k) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = k * KQ4_RT_C + pc + 64 * j;
      const bool live = prow && c < d;   // d % 32 == 0: a float4 is wholly in or out
      cur[j] = live ? *reinterpret_cast<const float4 *>(rw + c) : make_float4(0, 0, 0, 0);
      xv[j] = live ? *reinterpret_cast<const float4 *>(xt + c) : make_float4(0, 0, 0, 0);
    }
  };
  auto store = [&](int k) {
    if (!prow) return;
    float *dst = kq4_rt_lds + ((k & 1) * KQ4_RT_E + pr) * KQ4_RT_P + pc;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k * KQ4_RT_C + pc + 64 * j < d)
        *reinterpret_cast<float4 *>(dst + 64 * j) = make_float4(
            cur[j].x * xv[j].x, cur[j].y * xv[j].y, cur[j].z * xv[j].z, cur[j].w * xv[j].w);
  };
  if (wave > 0) load(0);
  float s = 0.0f;
  const bool adder = wave == 0 && threadIdx.x < KQ4_RT_E;
  for (int k = 0; k < ntile; ++k) {
    if (wave > 0) {
      store(k);
      if (k + 1 < ntile) load(k + 1);
    }
    __syncthreads();   // tile k's products are in LDS; the adders are done with buffer k-1
    if (adder) {
      // 32-column chunks, each read before the previous one is added (two register sets), so
      // the LDS latency stays off the add chain. The loop body is straight-line (one chunk past
      // n may be read and not added; the LDS has a 32-float pad after the last row), so every
      // add waits for exactly its own read.
      const int n = min(KQ4_RT_C, d - k * KQ4_RT_C);   // a multiple of 32
      const float *src = kq4_rt_lds + ((k & 1) * KQ4_RT_E + threadIdx.x) * KQ4_RT_P;
      float4 *va = rb, *vb = rb + 8;
      auto rd = [&](float4 *v, int i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4 *>(src + i + 4 * j);
        __builtin_amdgcn_sched_barrier(0);   // issued here, not sunk below the adds
      };
      auto add = [&](const float4 *v) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          s += v[j].x;
          s += v[j].y;
          s += v[j].z;
          s += v[j].w;
        }
      };
      rd(va, 0);
      int i = 0;
      for (; i + 64 <= n; i += 64) {
        rd(vb, i + 32);
        add(va);
        rd(va, i + 64);
        add(vb);
      }
      if (i < n) add(va);   // n % 64 == 32: the last chunk, already read
    }
  }
  if (adder && e0 + threadIdx.x < ne) logits[(size_t)t * ne + e0 + threadIdx.x] = s;
}

int kq4_launch_moe_logits(float *logits, const float *router, const float *X, int T, int ne,
                          int d, hipStream_t s) {
  if (T <= 0) return 0;
  if (d % 32) return (int)hipErrorInvalidValue;
  const size_t lds = (2 * KQ4_RT_E * KQ4_RT_P + 32) * sizeof(float);
  static std::atomic<unsigned long long> attr{0};   // 66 KB of LDS
  hipError_t e = kq4_lds_limit_once(reinterpret_cast<const void *>(&kq4_moe_logits_kernel),
                                    (int)lds, attr);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(kq4_moe_logits_kernel,
                     dim3((unsigned)((ne + KQ4_RT_E - 1) / KQ4_RT_E), (unsigned)T), dim3(320),
                     lds, s, logits, router, X, ne, d);
  return (int)hipGetLastError();
}

// ---- prep: grouping + activation quantizer ---------------------------------------------------
// Workgroup 0 builds the expert -> (token, rank) table: counts by LDS atomics, an exclusive scan,
// then each pair takes a slot by an atomic cursor. The order of an expert's pairs is whatever the
// atomics give: every pair is computed on its own (its own MFMA token row, its own fp32 chain), so
// no output depends on it. It also writes one record per slot (the active experts in id order):
// rec[16s] = expert (-1 for slots [active, nslot)), rec[16s+1] = the offset of its pairs in
// ex_pair, rec[16s+2] = their count, rec[16s+4 ..] = its first KQ4_MOE_RECP pair ids, so an
// expert workgroup finds its expert and pairs with one load instead of a chain of three.
// Workgroups 1..: the activation quantizer of kq4_quant.hip (one half-wave per 32-block).
__global__ __launch_bounds__(256) void kq4_moe_prep_kernel(
    int *__restrict__ ex_off, int *__restrict__ ex_pair, int *__restrict__ rec, int nslot,
    const int *__restrict__ sel, int n_pairs, int ne, const float *__restrict__ X,
    int8_t *__restrict__ xq, float *__restrict__ xd, int T, int d) {
  if (blockIdx.x == 0) {
    // LDS: cnt[ne] (then each expert's offset), cursor[ne], slot[ne], the waves' totals part[w] and
    // part[blockDim + w]
    extern __shared__ int kq4_moe_cnt[];
    int *cnt = kq4_moe_cnt, *cur = kq4_moe_cnt + ne, *slt = kq4_moe_cnt + 2 * ne,
        *part = kq4_moe_cnt + 3 * ne;
    const int nt = blockDim.x, tid = threadIdx.x;
    // the first 4 * blockDim pairs' expert ids stay in registers for the scatter below
    int ev[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ev[j] = tid + nt * j < n_pairs ? sel[tid + nt * j] : -1;
    for (int e = tid; e < ne; e += nt) cnt[e] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ev[j] >= 0 && ev[j] < ne) atomicAdd(&cnt[ev[j]], 1);
    for (int i = tid + 4 * nt; i < n_pairs; i += nt) {
      const int e = sel[i];
      if (e >= 0 && e < ne) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scans of the counts and of the active flags: thread tid owns experts
    // [tid*per, tid*per + per); its totals are scanned inside each wave by lane shifts, and the
    // waves' totals (through LDS, one barrier) give each wave its offset and every thread the
    // block totals tc (pairs) and ta (active experts).
    const int per = (ne + nt - 1) / nt, e0 = tid * per;
    int sc = 0, sa = 0;
    for (int e = e0; e < e0 + per && e < ne; ++e) { sc += cnt[e]; sa += cnt[e] > 0; }
    const int lane = tid & 63, wv = tid >> 6, nwv = nt >> 6;
    int ic = sc, ia = sa;   // inclusive scans within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int vc = __shfl_up(ic, o, 64), va = __shfl_up(ia, o, 64);
      if (lane >= o) { ic += vc; ia += va; }
    }
    if (lane == 63) { part[wv] = ic; part[nt + wv] = ia; }
    __syncthreads();
    int oc = 0, oa = 0;   // the earlier waves' totals
    for (int w = 0; w < wv; ++w) { oc += part[w]; oa += part[nt + w]; }
    int tc = 0, ta = 0;
    for (int w = 0; w < nwv; ++w) { tc += part[w]; ta += part[nt + w]; }
    int acc = oc + ic - sc, na = oa + ia - sa;   // exclusive prefixes
    for (int e = e0; e < e0 + per && e < ne; ++e) {
      const int c = cnt[e];
      cur[e] = acc;
      cnt[e] = acc;
      ex_off[e] = acc;
      if (c) {
        rec[KQ4_MOE_REC * na] = e;
        rec[KQ4_MOE_REC * na + 1] = acc;
        rec[KQ4_MOE_REC * na + 2] = c;
        slt[e] = na++;
      }
      acc += c;
    }
    if (tid == nt - 1) ex_off[ne] = tc;
    __syncthreads();
    for (int s = ta + tid; s < nslot; s += nt) rec[KQ4_MOE_REC * s] = -1;
    auto place = [&](int e, int i) {   // pair i of expert e
      const int pos = atomicAdd(&cur[e], 1);
      ex_pair[pos] = i;
      if (pos - cnt[e] < KQ4_MOE_RECP) rec[KQ4_MOE_REC * slt[e] + 4 + pos - cnt[e]] = i;
    };
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ev[j] >= 0 && ev[j] < ne) place(ev[j], tid + nt * j);
    for (int i = tid + 4 * nt; i < n_pairs; i += nt) {
      const int e = sel[i];
      if (e >= 0 && e < ne) place(e, i);
    }
    return;
  }
  const int nb = d / 32;
  const int lane = threadIdx.x & 31;
  const long blk = (long)(blockIdx.x - 1) * (blockDim.x >> 5) + (threadIdx.x >> 5);
  if (blk >= (long)T * nb) return;   // whole 32-lane halves exit together
  const float v = X[blk * 32 + lane];
  const float a = kq4_max32(fmaxf(fabsf(v), 1e-10f));
  const float dq = a / 127.0f;
  int q = (int)(v / dq + 0.5f);
  q = q > 127 ? 127 : (q < -127 ? -127 : q);
  xq[blk * 32 + lane] = (int8_t)q;
  if (lane == 0) xd[blk] = dq;
}

// ---- shared pieces of the expert kernels ----------------------------------------------------

// Slot s's record (written by the prep kernel), the header and the first NI pair ids: uniform
// loads kept in scalar registers.
template <int NI>
struct KQ4MoeSlot {
  int r[4 + NI];
};

template <int NI>
KQ4_DEV KQ4MoeSlot<NI> kq4_moe_slot(const int *__restrict__ rec, int slot) {
  static_assert(NI % 4 == 0 && NI <= KQ4_MOE_RECP, "kq4_moe_slot: 0, 4, 8 or 12 pair ids");
  KQ4MoeSlot<NI> s;
  const int4 *p = reinterpret_cast<const int4 *>(rec + KQ4_MOE_REC * slot);
#pragma unroll
  for (int k = 0; k < 1 + NI / 4; ++k) {
    const int4 v = p[k];
    s.r[4 * k] = __builtin_amdgcn_readfirstlane(v.x);
    s.r[4 * k + 1] = __builtin_amdgcn_readfirstlane(v.y);
    s.r[4 * k + 2] = __builtin_amdgcn_readfirstlane(v.z);
    s.r[4 * k + 3] = __builtin_amdgcn_readfirstlane(v.w);
  }
  return s;
}

template <int NI>
KQ4_DEV int kq4_moe_pair(const KQ4MoeSlot<NI> &s, const int *__restrict__ ex_pair, int j) {
  static_assert(NI <= KQ4_MOE_RECP, "kq4_moe_pair: the record holds KQ4_MOE_RECP pair ids");
  if (j >= NI) return ex_pair[s.r[1] + j];
  uint32_t v = 0;
#pragma unroll
  for (int k = 0; k < NI; ++k) v |= (uint32_t)s.r[4 + k] & (0u - (uint32_t)(j == k));
  return (int)v;
}

// This lane's weights of one (row set, stage) chunk of the stream layout: units u0 .. u0+NU-1
// (2 blocks each) of its (row, half), and the f16 scales of its row's blocks 8*sh .. 8*sh+7
// (NS = 1) or 0 .. 15 (NS = 2). Scales first: loads complete in issue order.
template <int NU, int NS>
struct KQ4MoeW {
  uint32_t n[4 * NU];
  uint32_t sc[4 * NS];
};

template <int NU, int NS>
KQ4_DEV void kq4_moe_wload(KQ4MoeW<NU, NS> &w, const uint8_t *__restrict__ chunk, int lane, int u0,
                           int sh) {
  // each chunk is read once per launch: non-temporal loads
  const uint4 *sc = reinterpret_cast<const uint4 *>(chunk + 8192) + (lane & 31);
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const uint4 v = kq4_ld_nt(sc + 32 * (NS == 2 ? i : sh));
    w.sc[4 * i] = v.x; w.sc[4 * i + 1] = v.y; w.sc[4 * i + 2] = v.z; w.sc[4 * i + 3] = v.w;
  }
  const uint4 *src = reinterpret_cast<const uint4 *>(chunk) + lane;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const uint4 v = kq4_ld_nt(src + 64 * (u0 + u));
    w.n[4 * u] = v.x; w.n[4 * u + 1] = v.y; w.n[4 * u + 2] = v.z; w.n[4 * u + 3] = v.w;
  }
}

// Terms t[b][v] = fl(fl(sc*xd) * S) of the chunk's 2*NU blocks for this lane's row (lane%32) and
// pair VT*(lane/32)+v (VT = 2 or 4; 2*VT pairs): the pair's codes sit in MFMA token row
// 4*(lane/32)+v, i.e. A row rho = 4*i+v holds pair VT*i+v (i < 2, v < VT; other rows: any codes).
// The activation codes are at slab[pair*qts + qpos(b)], scales sx[b*2*VT + pair].
// PIPE: every block's activation scales are read first, the A fragments two blocks ahead, and
// two MFMAs are in flight, so LDS and MFMA latencies are not paid block by block (the scale read
// of each block used to wait for all outstanding LDS reads); for kernels with the registers to
// spare. VTC: the pairs computed (1 in one-token launches; t[b][v] = 0 for the others).
template <int NU, int NS, int VT, bool PIPE = false, int VTC = VT>
KQ4_DEV void kq4_moe_terms(const KQ4MoeW<NU, NS> &w, const uint8_t *slab, int qts,
                           const float *sx, int lane, float (*t)[VT]) {
  const int h = lane >> 5, r = lane & 31;
  const int pr = (r < 8 && (r & 3) < VT) ? VT * (r >> 2) + (r & 3) : 0;
  const uint8_t *qb = slab + pr * qts + 16 * h;
  if constexpr (PIPE) {
    constexpr int NB = 2 * NU;
    float xsv[NB][VTC];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int v = 0; v < VTC; ++v) xsv[b][v] = sx[b * 2 * VT + VT * h + v];
    auto rd = [&](int b) { return *reinterpret_cast<const kq4_v4i *>(qb + kq4_moe_qpos(b)); };
    auto mf = [&](int b, kq4_v4i A) {
      uint32_t o[4];
      kq4_unpack_half(w.n[2 * b], w.n[2 * b + 1], o);
      const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      return kq4_moe_mfma(A, B);
    };
    kq4_v4i Aq[3];
    Aq[0] = rd(0);
    if (NB > 1) Aq[1] = rd(1);
    kq4_v16i C = mf(0, Aq[0]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + 2 < NB) Aq[(b + 2) % 3] = rd(b + 2);
      kq4_v16i Cn = C;
      if (b + 1 < NB) Cn = mf(b + 1, Aq[(b + 1) % 3]);
      // block b+1's MFMA is issued before block b's result is read (two result sets live)
      __builtin_amdgcn_sched_barrier(0);
      // C = 16*S: fl(fl((sc/16)*xd) * 16S) = fl(fl(sc*xd) * S), every step scaled by a power of
      // two far from underflow (sc >= 2^-24, xd >= 1e-10/127)
      const float sc = kq4_h2f(w.sc[b >> 1] >> (16 * (b & 1))) * 0.0625f;
#pragma unroll
      for (int v = 0; v < VT; ++v) {
        t[b][v] = v < VTC ? (sc * xsv[b][v < VTC ? v : 0]) * (float)C[v] : 0.0f;
        kq4_moe_pin(t[b][v]);
      }
      C = Cn;
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < 2 * NU; ++b) {
    uint32_t o[4];
    kq4_unpack_half(w.n[2 * b], w.n[2 * b + 1], o);
    const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    const kq4_v4i A = *reinterpret_cast<const kq4_v4i *>(qb + kq4_moe_qpos(b));
    const kq4_v16i C = kq4_moe_mfma(A, B);
    const float sc = kq4_h2f(w.sc[b >> 1] >> (16 * (b & 1))) * 0.0625f;   // C = 16*S (as above)
    const float *xs = sx + b * 2 * VT + VT * h;
#pragma unroll
    for (int v = 0; v < VT; ++v) {
      t[b][v] = (sc * xs[v]) * (float)C[v];
      kq4_moe_pin(t[b][v]);
    }
    // one block's MFMA in flight at a time: each holds 16 result registers
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---- gate/up + SiLU + av quantization ----------------------------------------------------------
// grid: min(ne, pairs) expert slots x (ef/32) row sets; block: 2*nst waves, wave k < nst streams
// stage k of G, wave nst + k stage k of U (the same rows). Per pass of up to 4 pairs: the gate
// wave of stage k stages the pairs' codes of stage k in slab k; every wave computes its terms;
// then nst phases add them to the gate and up chains in block order; then one lane per (pair,
// row) forms av, and the 32 rows of the set (one av block) are quantized together.
// T1 (one token): slot j is rank j, expert sel[j] with the single pair j, and the gate waves
// quantize X themselves, so the launch needs no prep kernel (the grouping is trivial).
template <bool T1>
__global__ __launch_bounds__(1024) void kq4_moe_gu_kernel(
    const uint8_t *__restrict__ G, const uint8_t *__restrict__ U, const int8_t *__restrict__ xq,
    const float *__restrict__ xd, const int *__restrict__ rec, const int *__restrict__ ex_pair,
    int8_t *__restrict__ avq, float *__restrict__ avd,
    float *__restrict__ g_out, float *__restrict__ u_out, float *__restrict__ av_out, int d,
    int ef, int tk, const int *__restrict__ sel, const float *__restrict__ X, int ne) {
  extern __shared__ __align__(16) uint8_t kq4_moe_lds[];
  constexpr int PC = KQ4_MOE_PCG, VT = PC / 2;
  constexpr int SLAB = kq4_moe_slab(16, PC);
  const int rbs = ef / 32;
  const int slot = blockIdx.x / rbs, rs = blockIdx.x - slot * rbs;
  const int nb = d / 32, nst = (nb + 15) / 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = wave >= nst ? 1 : 0;                  // 0 = gate, 1 = up
  const int k = wave - m * nst;                       // stage
  const int nblk = nb - 16 * k < 16 ? nb - 16 * k : 16;
  // T1: a gate wave's share of X (lane quad per block, 8 values per lane), loaded before the
  // routing and the weights, so that its quantization waits only for these loads (the loads
  // complete in issue order)
  float4 x0 = make_float4(0, 0, 0, 0), x1 = x0;
  if (T1 && m == 0 && (lane >> 2) < nblk) {
    const float4 *src = reinterpret_cast<const float4 *>(X + (size_t)(16 * k + (lane >> 2)) * 32 +
                                                         8 * (lane & 3));
    x0 = src[0];
    x1 = src[1];
  }
  KQ4MoeSlot<0> sr{};   // header only: inline ids spill here
  int e, cnt;
  if (T1) {
    e = __builtin_amdgcn_readfirstlane(sel[slot]);
    if (e < 0 || e >= ne) return;                     // no expert at this rank
    cnt = 1;
  } else {
    sr = kq4_moe_slot<0>(rec, slot);
    e = sr.r[0];
    if (e < 0) return;                                // no expert in this slot (whole workgroup)
    cnt = sr.r[2];
  }
  auto pair = [&](int j) { return T1 ? slot : kq4_moe_pair<0>(sr, ex_pair, j); };
  const int h = lane >> 5, r = lane & 31;
  uint8_t *slab = kq4_moe_lds + k * SLAB;
  float *sx = reinterpret_cast<float *>(slab + PC * KQ4_MOE_QTS);     // [16][PC]
  float *accb = reinterpret_cast<float *>(kq4_moe_lds + nst * SLAB);   // [2][PC][32]
  // Several tokens: a gate wave stages stage k's codes and scales of a pass's pairs (zeros past
  // them and past K): 4 pairs x 16 blocks x 2 halves = 128 units of 16 B (two per lane) and 64
  // scales (one per lane). The first pass's are loaded before the weights (their pair ids from
  // the slot record), so that staging them waits only for these loads: the loads complete in
  // issue order, and issued after the weights they held the stage barrier until every weight
  // load was in.
  uint4 pv[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  float px = 0.0f;
  auto stage_load = [&](int c0, auto &&pid) {
    const int np = cnt - c0 < PC ? cnt - c0 : PC;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = lane + 64 * u;
      const int p = i >> 5, bb = (i >> 1) & 15, hh = i & 1;
      pv[u] = make_uint4(0, 0, 0, 0);
      if (p < np && bb < nblk) {
        const int tok = pid(c0 + p) / tk;
        pv[u] = *reinterpret_cast<const uint4 *>(xq + (size_t)tok * d + (size_t)(16 * k + bb) * 32 +
                                                 16 * hh);
      }
    }
    // a buffer load with a 32-bit offset: a 64-bit per-lane address of this read, hoisted out of
    // the passes' loop by the compiler, spilled
    const int p = lane >> 4, bb = lane & 15;
    px = p < np && bb < nblk
             ? __uint_as_float(kq4_bload4(kq4_rsrc(xd, 0xFFFFFFFFu),
                                          4u * (uint32_t)((pid(c0 + p) / tk) * nb + 16 * k + bb)))
             : 0.0f;
  };
  if (!T1 && m == 0) {
    const KQ4MoeSlot<4> s4 = kq4_moe_slot<4>(rec, slot);
    stage_load(0, [&](int j) { return kq4_moe_pair<4>(s4, ex_pair, j); });
  }
  KQ4MoeW<8, 2> w;
  kq4_moe_wload<8, 2>(w, (m ? U : G) + ((size_t)((e * ef) / 32 + rs) * nst + k) * KQ4_STREAM_CHUNK,
                      lane, 0, 0);

  // one pass of up to PC pairs; the first pass is a call of its own, so that its staged values
  // are not kept live around the loop of the later ones
  auto run_pass = [&](int c0, auto first) {
    const int np = cnt - c0 < PC ? cnt - c0 : PC;
    if (m == 0 && T1) {
      // token 0's stage k quantized here, a lane quad per block (8 values per lane), as the prep
      // kernel's quantizer does it: amax floored at 1e-10, dq = amax/127, q = (int)(x/dq + 0.5)
      // clamped to +-127; pairs 1-3 and blocks past K get zero codes and scales
      const int bb = lane >> 2, qq = lane & 3;
      const bool live = bb < nblk;
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      float am = 1e-10f;
#pragma unroll
      for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(xv[i]));
      am = kq4_quad_max(am);
      const float dq = am / 127.0f;
      uint32_t pk[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int q = (int)(xv[i] / dq + 0.5f);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        pk[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
      }
      *reinterpret_cast<uint2 *>(slab + kq4_moe_qpos(bb) + 8 * qq) = make_uint2(pk[0], pk[1]);
      if (qq == 0) sx[bb * PC] = live ? dq : 0.0f;
#pragma unroll
      for (int u = 0; u < 2; ++u) {   // pairs 1-3: 96 units of 16 B
        const int i = lane + 64 * u;
        const int p = i >> 5, b2 = (i >> 1) & 15, hh = i & 1;
        if (p >= 1)
          *reinterpret_cast<uint4 *>(slab + p * KQ4_MOE_QTS + kq4_moe_qpos(b2) + 16 * hh) =
              make_uint4(0, 0, 0, 0);
      }
      if (lane >= 16) sx[(lane & 15) * PC + (lane >> 4)] = 0.0f;
    } else if (m == 0) {
      if constexpr (!decltype(first)::value) stage_load(c0, pair);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = lane + 64 * u;
        const int p = i >> 5, bb = (i >> 1) & 15, hh = i & 1;
        *reinterpret_cast<uint4 *>(slab + p * KQ4_MOE_QTS + kq4_moe_qpos(bb) + 16 * hh) = pv[u];
      }
      sx[(lane & 15) * PC + (lane >> 4)] = px;
    }
    __syncthreads();
    float t[16][VT];
    kq4_moe_touch(w.n);
    kq4_moe_terms<8, 2, VT, T1, T1 ? 1 : VT>(w, slab, KQ4_MOE_QTS, sx, lane, t);
    if (T1) {
      // one pair: every wave puts its blocks' terms (pair 0: lanes 0-31, v = 0) in LDS, then one
      // lane per (gate/up, row) adds all of them in block order, the same chain in one pass
      float *tb = reinterpret_cast<float *>(kq4_moe_lds + nst * SLAB) + 2 * PC * 32;   // [2][32][pitch]
      const int pitch = 16 * nst + 1;
      if (h == 0) {
#pragma unroll
        for (int b = 0; b < 16; ++b) tb[(m * 32 + r) * pitch + 16 * k + b] = t[b][0];
      }
      __syncthreads();
      if (threadIdx.x < 64) {
        const int mm = threadIdx.x >> 5, rr = threadIdx.x & 31;
        const float *src = tb + (mm * 32 + rr) * pitch;
        float acc = 0.0f;
        for (int b0 = 0; b0 < nb; b0 += 16) {   // 16 reads, then 16 adds (every stage's 16 are set)
          float v[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = src[b0 + j];
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (b0 + j < nb) acc = acc + v[j];
        }
        accb[(mm * PC) * 32 + rr] = acc;
      }
      __syncthreads();
    } else
    // the chains: stage kk's waves add their blocks' terms in order, then hand the sums on
    for (int kk = 0; kk < nst; ++kk) {
      if (k == kk) {
        float acc[VT];
#pragma unroll
        for (int v = 0; v < VT; ++v) acc[v] = kk ? accb[(m * PC + VT * h + v) * 32 + r] : 0.0f;
#pragma unroll
        for (int b = 0; b < 16; ++b)
          if (b < nblk)
#pragma unroll
            for (int v = 0; v < VT; ++v) acc[v] = acc[v] + t[b][v];
#pragma unroll
        for (int v = 0; v < VT; ++v) accb[(m * PC + VT * h + v) * 32 + r] = acc[v];
      }
      __syncthreads();
    }
    // av = fl(fl(g / fl(1 + exp(-g))) * u), quantized over the set's 32 rows (one av block)
    for (int i = threadIdx.x; i < PC * 32; i += blockDim.x) {
      const int p = i >> 5, rw = i & 31;
      const float g = accb[p * 32 + rw], u = accb[(PC + p) * 32 + rw];
      const float a = (g / (1.0f + kq4_expf(-g))) * u;
      const float amax = kq4_max32(fmaxf(fabsf(a), 1e-10f));
      const float dq = amax / 127.0f;
      int qv = (int)(a / dq + 0.5f);
      qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
      if (p < np) {
        const int pi = pair(c0 + p);
        const size_t o = (size_t)pi * ef + (size_t)rs * 32 + rw;
        avq[o] = (int8_t)qv;
        if (rw == 0) avd[(size_t)pi * rbs + rs] = dq;
        if (g_out) { g_out[o] = g; u_out[o] = u; }
        if (av_out) av_out[o] = a;
      }
    }
    __syncthreads();   // before the next pass overwrites the slabs and sums
  };
  run_pass(0, std::true_type{});
  for (int c0 = PC; c0 < cnt; c0 += PC) run_pass(c0, std::false_type{});
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

// ---- down projection: unweighted partials -------------------------------------------------------
// grid: expert slots x groups of RSG row sets of D; block: RSG x NH waves. Wave (g, w) takes row
// set g of the group and half stage qa + w of D's blocks (8 blocks; qa = the first half stage that
// meets the expert's column band [e*ef/32, e*ef/32 + ef/32)); blocks outside the band are
// skipped, waves past the band only join the barriers. Per pass of up to 8 pairs the workgroup
// stages the band's av codes once (shared by its row sets), each wave computes its terms, and for
// every row set the waves add them in block order.
// T1 (one token): slot j is rank j, expert sel[j], its single pair j.
template <bool T1>
__global__ __launch_bounds__(1024) void kq4_moe_down_kernel(
    const uint8_t *__restrict__ D, const int8_t *__restrict__ avq, const float *__restrict__ avd,
    const int *__restrict__ rec, const int *__restrict__ ex_pair, float *__restrict__ P, int ne,
    int d, int ef, int rsg, int nhl, const int *__restrict__ sel) {
  extern __shared__ __align__(16) uint8_t kq4_moe_lds[];
  constexpr int PC = KQ4_MOE_PCD, VT = PC / 2;
  const int nrs = d / 32, ngrp = (nrs + rsg - 1) / rsg;
  const int slot = blockIdx.x / ngrp, grp = blockIdx.x - slot * ngrp;
  KQ4MoeSlot<PC> sr{};
  int e, cnt;
  if (T1) {
    e = __builtin_amdgcn_readfirstlane(sel[slot]);
    if (e < 0 || e >= ne) return;
    cnt = 1;
  } else {
    sr = kq4_moe_slot<PC>(rec, slot);
    e = sr.r[0];
    if (e < 0) return;
    cnt = sr.r[2];
  }
  auto pair = [&](int j) { return T1 ? slot : kq4_moe_pair<PC>(sr, ex_pair, j); };
  const int cbe = ef / 32, nbD = ne * cbe, nstD = (nbD + 15) / 16;
  const int b0 = e * cbe;                              // first block of the band
  const int qa = b0 >> 3, nh = ((b0 + cbe - 1) >> 3) - qa + 1;
  const int qts = ((cbe + 1) >> 1) * 80;               // pair pitch of the staged band codes
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave / nhl, w = wave - g * nhl;        // row set in the group, half stage
  const int rs = grp * rsg + g;
  const int h = lane >> 5, r = lane & 31;
  const int hq = qa + w;
  const bool live = w < nh && rs < nrs;
  uint8_t *codes = kq4_moe_lds;                                         // [PC][qts]
  float *sxb = reinterpret_cast<float *>(kq4_moe_lds + PC * qts);       // [cbe][PC]
  float *accb = sxb + cbe * PC + g * PC * 32;                           // per row set [PC][32]
  KQ4MoeW<4, 1> wt;
  if (live)
    kq4_moe_wload<4, 1>(wt, D + ((size_t)rs * nstD + (hq >> 1)) * KQ4_STREAM_CHUNK, lane,
                        4 * (hq & 1), hq & 1);
  // band-relative block of local block j, or -1 outside the band
  auto cbof = [&](int j) {
    const int gb = 8 * hq + j;
    return (gb >= b0 && gb < b0 + cbe) ? gb - b0 : -1;
  };
  const int pr = (r < 8 && (r & 3) < VT) ? VT * (r >> 2) + (r & 3) : 0;   // A row -> pair

  for (int c0 = 0; c0 < cnt; c0 += PC) {
    const int np = cnt - c0 < PC ? cnt - c0 : PC;
    // the band's codes and scales of the pass's pairs, once for all row sets
    for (int i = threadIdx.x; i < PC * cbe * 2; i += blockDim.x) {
      const int p = i / (2 * cbe), rem = i - p * 2 * cbe, cb = rem >> 1, hh = rem & 1;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (p < np)
        v = *reinterpret_cast<const uint4 *>(avq + (size_t)pair(c0 + p) * ef +
                                             (size_t)cb * 32 + 16 * hh);
      *reinterpret_cast<uint4 *>(codes + p * qts + kq4_moe_qpos(cb) + 16 * hh) = v;
    }
    for (int i = threadIdx.x; i < PC * cbe; i += blockDim.x) {
      const int cb = i / PC, p = i - cb * PC;
      sxb[i] = p < np ? avd[(size_t)pair(c0 + p) * cbe + cb] : 0.0f;
    }
    __syncthreads();
    float t[8][VT];
    if (live && T1) {
      // one pair: the pipelined form of the loop below (scales first, A fragments two blocks
      // ahead, two MFMAs in flight), pair 0's terms only
      kq4_moe_touch(wt.n);
      float xs0[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int cb = cbof(j);
        xs0[j] = sxb[(cb < 0 ? 0 : cb) * PC + VT * h];
      }
      auto rd = [&](int j) {
        const int cb = cbof(j);
        return *reinterpret_cast<const kq4_v4i *>(codes + pr * qts + kq4_moe_qpos(cb < 0 ? 0 : cb) +
                                                  16 * h);
      };
      auto mf = [&](int j, kq4_v4i A) {
        uint32_t o[4];
        kq4_unpack_half(wt.n[2 * j], wt.n[2 * j + 1], o);
        const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        return kq4_moe_mfma(A, B);
      };
      kq4_v4i Aq[3];
      Aq[0] = rd(0);
      Aq[1] = rd(1);
      kq4_v16i C = mf(0, Aq[0]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j + 2 < 8) Aq[(j + 2) % 3] = rd(j + 2);
        kq4_v16i Cn = C;
        if (j + 1 < 8) Cn = mf(j + 1, Aq[(j + 1) % 3]);
        __builtin_amdgcn_sched_barrier(0);
        // C = 16*S: fl(fl((sc/16)*xd) * 16S) = fl(fl(sc*xd) * S), as in kq4_moe_terms
        const float sc = kq4_h2f(wt.sc[j >> 1] >> (16 * (j & 1))) * 0.0625f;
        t[j][0] = (sc * xs0[j]) * (float)C[0];
        kq4_moe_pin(t[j][0]);
#pragma unroll
        for (int v = 1; v < VT; ++v) t[j][v] = 0.0f;
        C = Cn;
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (live) {
      kq4_moe_touch(wt.n);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int cb = cbof(j);
        const int cbs = cb < 0 ? 0 : cb;
        uint32_t o[4];
        kq4_unpack_half(wt.n[2 * j], wt.n[2 * j + 1], o);
        const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        const kq4_v4i A =
            *reinterpret_cast<const kq4_v4i *>(codes + pr * qts + kq4_moe_qpos(cbs) + 16 * h);
        const kq4_v16i C = kq4_moe_mfma(A, B);
        const float sc = kq4_h2f(wt.sc[j >> 1] >> (16 * (j & 1))) * 0.0625f;   // C = 16*S
        const float *xs = sxb + cbs * PC + VT * h;
#pragma unroll
        for (int v = 0; v < VT; ++v) {
          t[j][v] = (sc * xs[v]) * (float)C[v];
          kq4_moe_pin(t[j][v]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // the chains over the band's blocks, one per row set: wave by wave, block by block
    for (int ww = 0; ww < nh; ++ww) {
      if (w == ww && rs < nrs) {
        float acc[VT];
#pragma unroll
        for (int v = 0; v < VT; ++v) acc[v] = ww ? accb[(VT * h + v) * 32 + r] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (cbof(j) >= 0)
#pragma unroll
            for (int v = 0; v < VT; ++v) acc[v] = acc[v] + t[j][v];
#pragma unroll
        for (int v = 0; v < VT; ++v) {
          if (ww + 1 < nh) {
            accb[(VT * h + v) * 32 + r] = acc[v];
          } else if (VT * h + v < np) {
            P[(size_t)pair(c0 + VT * h + v) * d + (size_t)rs * 32 + r] = acc[v];
          }
        }
      }
      __syncthreads();
    }
  }
}

// ---- down projection, one wave per (expert slot, row set) -------------------------------------
// For bands of whole 8-block half stages (cbe % 8 == 0, up to 32 blocks; Qwen3-30B-A3B: 24
// blocks, 3 half stages) from two tokens on. A wave holds its row set's whole band: NH half
// stages of 4 stream units and 8 scales each, loaded at the start. Each output's chain over the
// band runs in the lane's registers in block order: acc = fl(acc + fl(fl(sc*xd)*S)), the V4
// chain. No LDS hand-off and no barrier between waves is needed. A workgroup's W waves take W
// consecutive row sets of one expert. They share the staging of each pass's av codes and scales
// (one barrier per pass). kq4_moe_down_kernel instead spreads the band's half stages over NH
// waves of one workgroup and passes the chain between them through LDS; here a CU holds NH
// times as many (expert, row set) items. PC: pairs per pass, 8 (4 per wave half) or 4 (2 per
// half, half the epilogue's VALU work; chosen when the launch averages at most 4 pairs per
// expert, the band's weights staying in registers across the passes).
template <int NH, int PC>
__global__ __launch_bounds__(256) void kq4_moe_downw_kernel(
    const uint8_t *__restrict__ D, const int8_t *__restrict__ avq, const float *__restrict__ avd,
    const int *__restrict__ rec, const int *__restrict__ ex_pair, float *__restrict__ P, int ne,
    int d) {
  extern __shared__ __align__(16) uint8_t kq4_moe_lds[];
  constexpr int VT = PC / 2, CBE = 8 * NH, QTS = (CBE / 2) * 80;
  const int W = blockDim.x >> 6;
  const int nrs = d / 32, ngrp = (nrs + W - 1) / W;
  const int slot = blockIdx.x / ngrp, grp = blockIdx.x - slot * ngrp;
  const KQ4MoeSlot<PC> sr = kq4_moe_slot<PC>(rec, slot);
  const int e = sr.r[0];
  if (e < 0) return;   // uniform over the workgroup
  const int cnt = sr.r[2];
  auto pair = [&](int j) { return kq4_moe_pair<PC>(sr, ex_pair, j); };
  const int nstD = (ne * CBE + 15) / 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rs = grp * W + wave;
  const bool live = rs < nrs;
  const int h = lane >> 5, r = lane & 31;
  uint8_t *codes = kq4_moe_lds;                                     // [PC][QTS]
  float *sxb = reinterpret_cast<float *>(kq4_moe_lds + PC * QTS);   // [CBE][PC]
  // the band's half stages e*NH .. e*NH + NH - 1 of row set rs
  KQ4MoeW<4, 1> wt[NH];
  if (live) {
#pragma unroll
    for (int k = 0; k < NH; ++k) {
      const int hq = e * NH + k;
      kq4_moe_wload<4, 1>(wt[k], D + ((size_t)rs * nstD + (hq >> 1)) * KQ4_STREAM_CHUNK, lane,
                          4 * (hq & 1), hq & 1);
    }
  }
  const int pr = (r < 8 && (r & 3) < VT) ? VT * (r >> 2) + (r & 3) : 0;   // A row 4i+v: pair VT*i+v
  for (int c0 = 0; c0 < cnt; c0 += PC) {
    const int np = cnt - c0 < PC ? cnt - c0 : PC;
    if (c0) __syncthreads();   // every wave is done with the previous pass's codes
    for (int i = threadIdx.x; i < PC * CBE * 2; i += blockDim.x) {
      const int p = i / (2 * CBE), rem = i - p * 2 * CBE, cb = rem >> 1, hh = rem & 1;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (p < np)
        v = *reinterpret_cast<const uint4 *>(avq + (size_t)pair(c0 + p) * (32 * CBE) +
                                             (size_t)cb * 32 + 16 * hh);
      *reinterpret_cast<uint4 *>(codes + p * QTS + kq4_moe_qpos(cb) + 16 * hh) = v;
    }
    for (int i = threadIdx.x; i < PC * CBE; i += blockDim.x) {
      const int cb = i / PC, p = i - cb * PC;
      sxb[i] = p < np ? avd[(size_t)pair(c0 + p) * CBE + cb] : 0.0f;
    }
    __syncthreads();
    if (!live) continue;
    float acc[VT];
#pragma unroll
    for (int v = 0; v < VT; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int k = 0; k < NH; ++k) {
      kq4_moe_touch(wt[k].n);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int cb = 8 * k + j;
        uint32_t o[4];
        kq4_unpack_half(wt[k].n[2 * j], wt[k].n[2 * j + 1], o);
        const kq4_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        const kq4_v4i A =
            *reinterpret_cast<const kq4_v4i *>(codes + pr * QTS + kq4_moe_qpos(cb) + 16 * h);
        const kq4_v16i C = kq4_moe_mfma(A, B);
        // C = 16*S: fl(fl((sc/16)*xd) * 16S) = fl(fl(sc*xd) * S), every step scaled by a power
        // of two far from underflow (sc >= 2^-24, xd >= 1e-10/127)
        const float sc = kq4_h2f(wt[k].sc[j >> 1] >> (16 * (j & 1))) * 0.0625f;
        const float *xs = sxb + cb * PC + VT * h;
#pragma unroll
        for (int v = 0; v < VT; ++v) {
          acc[v] = acc[v] + (sc * xs[v]) * (float)C[v];
          kq4_moe_pin(acc[v]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < VT; ++v)
      if (VT * h + v < np) P[(size_t)pair(c0 + VT * h + v) * d + (size_t)rs * 32 + r] = acc[v];
  }
}

// ---- one token: down projection and combine in one launch ------------------------------------
// A workgroup takes 8 rows of Y (a quarter row set) and every rank: wave w handles ranks w,
// w + nw, .., so the combine's rank order is within the workgroup and needs no cross-workgroup
// step. For rank j (expert e, band of cbe blocks from B0 = e*cbe, B0 even): lane (k, r) =
// (lane/8, lane%8) takes row r's 16-B stream lines L = k, k+8, .. (unit L/2 of the band, K half
// L%2: the halves of two blocks), 8 rows' lines of one unit being 128 contiguous bytes. Its
// integer dots (v_dot4 on the 16*(n-8) operand against the rank's av codes) give half-block
// sums; the partner lane (k+1, same row) holds the other half, one DPP add makes the exact block
// sums, and the even-k lanes form the terms fl(fl(sc*xs) * S) as the down kernel does. The
// terms go to LDS and lane r of the wave adds them in block order from 0 (the reference's
// chain, v4_row), giving P[j][row]; after a barrier wave 0's lanes 0..7 run the combine
// y = fl(y + fl(p * P)) over the ranks in order, skipping invalid expert ids, as
// kq4_moe_combine_kernel does.
#define KQ4_MOE_D1_ROWS 8
#define KQ4_MOE_D1_MAXL 4   // lines per lane (NL): cbe <= 32
template <int NL>
__global__ __launch_bounds__(1024) void kq4_moe_down1_kernel(
    float *__restrict__ Y, const uint8_t *__restrict__ D, const int8_t *__restrict__ avq,
    const float *__restrict__ avd, const int *__restrict__ sel, const float *__restrict__ pr,
    int tk, int ne, int d, int ef) {
  extern __shared__ __align__(16) uint8_t kq4_moe_lds[];
  const int cbe = ef / 32, nstD = (ne * cbe + 15) / 16;
  const int row0 = blockIdx.x * KQ4_MOE_D1_ROWS;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int r = lane & 7, k = lane >> 3;
  const int n = row0 + r;
  float *terms = reinterpret_cast<float *>(kq4_moe_lds) + wave * KQ4_MOE_D1_ROWS * cbe;
  float *sP = reinterpret_cast<float *>(kq4_moe_lds) + nw * KQ4_MOE_D1_ROWS * cbe;   // [tk][8]
  for (int j = wave; j < tk; j += nw) {
    const int e = __builtin_amdgcn_readfirstlane(sel[j]);
    if (e < 0 || e >= ne) continue;                  // skipped by the combine
    const int B0 = e * cbe;
    const int8_t *aq = avq + (size_t)j * ef;
    const float *ad = avd + (size_t)j * cbe;
    // all loads first: the lane's lines, their two blocks' scales and av codes and scales.
    // Unconditional (a line past the band reloads the band's last line, not used): loads behind
    // a branch made the wait counts at its join hold for both paths, and line 0's dots waited
    // for nearly every load of the later lines.
    uint4 wl[NL], a0[NL], a1[NL];
    uint32_t sw[NL];
    float2 xs[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int L = k + 8 * i < cbe ? k + 8 * i : cbe - 1;
      const int uu = L >> 1, h = L & 1, Bu = B0 + 2 * uu;
      wl[i] = *reinterpret_cast<const uint4 *>(D + kq4_stream_nib(n, Bu, h, nstD));
      sw[i] = *reinterpret_cast<const uint32_t *>(D + kq4_stream_scale(n, Bu, nstD));
      a0[i] = *reinterpret_cast<const uint4 *>(aq + 64 * uu + 16 * h);
      a1[i] = *reinterpret_cast<const uint4 *>(aq + 64 * uu + 32 + 16 * h);
      xs[i] = *reinterpret_cast<const float2 *>(ad + 2 * uu);
      asm volatile("" ::: "memory");   // the lines' loads in line order, as they are consumed
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int L = k + 8 * i;
      {   // every lane takes part in the exchange; a lane and its partner (L, L+1, cbe even)
          // are both inside the band or both past it
        // half-block sums 16*S of the two blocks: bytes 0-7 block 2uu, 8-15 block 2uu+1
        int s0 = 0, s1 = 0;
        if (L < cbe) {
          const uint32_t q0[4] = {a0[i].x, a0[i].y, a0[i].z, a0[i].w};
          const uint32_t q1[4] = {a1[i].x, a1[i].y, a1[i].z, a1[i].w};
          uint32_t o[4];
          kq4_unpack_half(wl[i].x, wl[i].y, o);
#pragma unroll
          for (int c = 0; c < 4; ++c) s0 = kq4_dot4(o[c], q0[c], s0);
          kq4_unpack_half(wl[i].z, wl[i].w, o);
#pragma unroll
          for (int c = 0; c < 4; ++c) s1 = kq4_dot4(o[c], q1[c], s1);
        }
        // the other K half from lane (k ^ 1, r): DPP row_ror:8 within each 16-lane row
        const int p0 = __builtin_amdgcn_update_dpp(0, s0, 0x128, 0xf, 0xf, false);
        const int p1 = __builtin_amdgcn_update_dpp(0, s1, 0x128, 0xf, 0xf, false);
        if ((k & 1) == 0 && L < cbe) {
          const int uu = L >> 1;
          const int S0 = (s0 + p0) >> 4, S1 = (s1 + p1) >> 4;   // exact: 16*S
          terms[r * cbe + 2 * uu] = (kq4_h2f(sw[i]) * xs[i].x) * (float)S0;
          terms[r * cbe + 2 * uu + 1] = (kq4_h2f(sw[i] >> 16) * xs[i].y) * (float)S1;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (k == 0) {
      float acc = 0.0f;
      for (int b = 0; b < cbe; ++b) acc = acc + terms[r * cbe + b];
      sP[j * KQ4_MOE_D1_ROWS + r] = acc;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");   // terms reused by the next rank
  }
  __syncthreads();
  if (wave == 0 && lane < KQ4_MOE_D1_ROWS) {
    float y = 0.0f;
    for (int j = 0; j < tk; ++j) {
      const int e = sel[j];
      if (e >= 0 && e < ne) y = y + pr[j] * sP[j * KQ4_MOE_D1_ROWS + lane];
    }
    Y[row0 + lane] = y;
  }
}

// y = fl(y + fl(p * P)) over the ranks in order, skipping invalid expert ids. The loads of all
// ranks are issued before the chain (P rows of skipped ranks are read but not used).
__global__ __launch_bounds__(256) void kq4_moe_combine_kernel(float *__restrict__ Y,
                                                              const float *__restrict__ P,
                                                              const int *__restrict__ sel,
                                                              const float *__restrict__ pr,
                                                              int T, int tk, int d, int ne) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)T * d) return;
  const int t = (int)(i / d), n = (int)(i - (long)t * d);
  float y = 0.0f;
  for (int j0 = 0; j0 < tk; j0 += 8) {
    float pv[8], wv[8];
    int ev[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = t * tk + j0 + j;
      const bool in = j0 + j < tk;
      ev[j] = in ? sel[s] : -1;
      wv[j] = in ? pr[s] : 0.0f;
      pv[j] = in ? P[(size_t)s * d + n] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (ev[j] >= 0 && ev[j] < ne) y = y + wv[j] * pv[j];
  }
  Y[i] = y;
}

int kq4_launch_moe_route(int *sel, float *pr, const float *logits, int T, int ne, int tk,
                         hipStream_t s) {
  if (tk > KQ4_MOE_MAXTK || ne > KQ4_MOE_MAXNE) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kq4_moe_route_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, sel,
                     pr, logits, T, ne, tk);
  return (int)hipGetLastError();
}

int kq4_moe_shape_ok(int d, int ef) {
  if (d <= 0 || ef <= 0 || d % 32 || ef % 32) return 0;
  const int nst = (d / 32 + 15) / 16;
  return nst <= 8 && (ef / 32) / 8 + 2 <= 16 && ef <= 4096;   // 2*nst and <= 16 waves; LDS
}

int kq4_launch_moe_dbg(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                       const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d,
                       int ef, const KQ4MoeWs &ws, float *g_out, float *u_out, float *av_out,
                       const float *av_in, hipStream_t s) {
  if (!kq4_moe_shape_ok(d, ef) || T <= 0 || tk <= 0) return (int)hipErrorInvalidValue;
  const int n_pairs = T * tk;
  const int nb = d / 32, nst = (nb + 15) / 16, cbe = ef / 32;
  const long qblk = (long)T * nb;
  // one token: every slot is a rank with one pair, the kernels take sel directly (no prep)
  const bool t1 = T == 1;
  const int slots = t1 ? tk : (ne < n_pairs ? ne : n_pairs);
  if (!t1)
    hipLaunchKernelGGL(kq4_moe_prep_kernel, dim3((unsigned)(1 + (qblk + 7) / 8)), dim3(256),
                       (3 * ne + 2 * 256) * sizeof(int), s, ws.ex_off, ws.ex_pair, ws.rec, slots,
                       sel, n_pairs, ne, X, ws.xq, ws.xd, T, d);
  const size_t lds_gu = (size_t)nst * kq4_moe_slab(16, KQ4_MOE_PCG) +
                        2 * KQ4_MOE_PCG * 32 * sizeof(float) +
                        (t1 ? (size_t)2 * 32 * (16 * nst + 1) * sizeof(float) : 0);   // T1 terms
  hipLaunchKernelGGL(t1 ? kq4_moe_gu_kernel<true> : kq4_moe_gu_kernel<false>,
                     dim3((unsigned)(slots * cbe)), dim3(128 * nst), lds_gu, s, G, U, ws.xq, ws.xd,
                     ws.rec, ws.ex_pair, ws.avq, ws.avd, g_out, u_out, av_out, d, ef, tk, sel, X, ne);
  if (av_in) {
    const long nblk = (long)n_pairs * cbe;
    hipLaunchKernelGGL(kq4_moe_avq_kernel, dim3((unsigned)((nblk + 7) / 8)), dim3(256), 0, s,
                       av_in, ws.avq, ws.avd, nblk);
  }
  // one token with an even band (every band starts on a stream unit) and at most 16 ranks: down
  // and combine in one launch
  const int cbe_ = ef / 32;
  if (t1 && cbe_ % 2 == 0 && cbe_ <= 8 * KQ4_MOE_D1_MAXL && tk <= 16) {
    const int nw = tk;
    const size_t lds = ((size_t)nw * KQ4_MOE_D1_ROWS * cbe_ + (size_t)tk * KQ4_MOE_D1_ROWS) *
                       sizeof(float);
    const dim3 grid((unsigned)(d / KQ4_MOE_D1_ROWS)), block(64 * nw);
    switch ((cbe_ + 7) / 8) {
      case 1: hipLaunchKernelGGL(kq4_moe_down1_kernel<1>, grid, block, lds, s, Y, D, ws.avq,
                                 ws.avd, sel, pr, tk, ne, d, ef); break;
      case 2: hipLaunchKernelGGL(kq4_moe_down1_kernel<2>, grid, block, lds, s, Y, D, ws.avq,
                                 ws.avd, sel, pr, tk, ne, d, ef); break;
      case 3: hipLaunchKernelGGL(kq4_moe_down1_kernel<3>, grid, block, lds, s, Y, D, ws.avq,
                                 ws.avd, sel, pr, tk, ne, d, ef); break;
      default: hipLaunchKernelGGL(kq4_moe_down1_kernel<4>, grid, block, lds, s, Y, D, ws.avq,
                                  ws.avd, sel, pr, tk, ne, d, ef); break;
    }
    return (int)hipGetLastError();
  }
  // bands of whole half stages, two tokens on: one wave per (slot, row set), W row sets per
  // workgroup (KQ4_MOE_DOWNW: W; 0 = the kernel below)
  static const int downw = [] {
    const char *v = getenv("KQ4_MOE_DOWNW");
    return v ? atoi(v) : KQ4_MOE_DOWNW_DEFAULT;
  }();
  if (!t1 && cbe % 8 == 0 && cbe <= 32 && downw >= 1 && downw <= 4) {
    const int W = downw, nrs = d / 32, ngrp = (nrs + W - 1) / W;
    // 4 pairs per pass when the pairs average at most 4 per expert slot (Qwen3-30B-A3B: T = 8
    // and 64; 8 from T = 256 on, where the extra passes' staging costs more than the smaller
    // epilogue saves); KQ4_MOE_DOWNW_PC = 4 / 8 forces one (for measurement)
    static const int pc_force = [] {
      const char *v = getenv("KQ4_MOE_DOWNW_PC");
      return v ? atoi(v) : 0;
    }();
    const int pc = pc_force == 4 || pc_force == 8 ? pc_force : (n_pairs <= 4 * slots ? 4 : 8);
    const size_t lds = (size_t)pc * ((cbe / 2) * 80) + (size_t)cbe * pc * 4;
    const dim3 grid((unsigned)(slots * ngrp)), block(64 * W);
#define KQ4_DOWNW(NH, PC)                                                                       \
  {                                                                                             \
    auto kern = kq4_moe_downw_kernel<NH, PC>;                                                   \
    hipLaunchKernelGGL(kern, grid, block, lds, s, D, ws.avq, ws.avd, ws.rec, ws.ex_pair, ws.P,  \
                       ne, d);                                                                  \
  }
    switch (cbe / 8 * 16 + pc) {
      case 1 * 16 + 4: KQ4_DOWNW(1, 4); break;
      case 1 * 16 + 8: KQ4_DOWNW(1, 8); break;
      case 2 * 16 + 4: KQ4_DOWNW(2, 4); break;
      case 2 * 16 + 8: KQ4_DOWNW(2, 8); break;
      case 3 * 16 + 4: KQ4_DOWNW(3, 4); break;
      case 3 * 16 + 8: KQ4_DOWNW(3, 8); break;
      case 4 * 16 + 4: KQ4_DOWNW(4, 4); break;
      default: KQ4_DOWNW(4, 8); break;
    }
#undef KQ4_DOWNW
    const long n = (long)T * d;
    hipLaunchKernelGGL(kq4_moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       s, Y, ws.P, sel, pr, T, tk, d, ne);
    return (int)hipGetLastError();
  }
  // half stages a band can meet (the most over the experts), and row sets per workgroup
  int nhl = 1;
  for (int e = 0; e < ne; ++e) {
    const int b0 = e * cbe, nh = ((b0 + cbe - 1) >> 3) - (b0 >> 3) + 1;
    nhl = nh > nhl ? nh : nhl;
  }
  // row sets per workgroup: as many as fit 16 waves, keeping about two workgroups per CU
  const int nrs = d / 32;
  int rsg = 16 / nhl;
  const int spread = (slots * nrs) / (2 * (ws.ncu > 0 ? ws.ncu : 256));
  rsg = rsg < spread ? rsg : spread;
  // Capped at 1 by default: one row set per workgroup (nhl waves) measured fastest at every T
  // (Qwen3-30B-A3B T = 64: 114.5 us at up to 4 row sets per workgroup, 16 waves, against 108.1 us;
  // small workgroups let a CU overlap one's loads with another's chain), although each then
  // stages the band's codes for itself. KQ4_MOE_RSG sets the cap (for measurement).
  static const int rsg_max = [] {
    const char *v = getenv("KQ4_MOE_RSG");
    return v ? atoi(v) : 1;
  }();
  rsg = rsg < rsg_max ? rsg : rsg_max;
  rsg = rsg < 1 ? 1 : (rsg > nrs ? nrs : rsg);
  const int ngrp = (nrs + rsg - 1) / rsg;
  const size_t lds_dn = (size_t)KQ4_MOE_PCD * (((cbe + 1) / 2) * 80) +
                        (size_t)cbe * KQ4_MOE_PCD * sizeof(float) +
                        (size_t)rsg * KQ4_MOE_PCD * 32 * sizeof(float);
  hipLaunchKernelGGL(t1 ? kq4_moe_down_kernel<true> : kq4_moe_down_kernel<false>,
                     dim3((unsigned)(slots * ngrp)), dim3(64 * rsg * nhl), lds_dn, s, D, ws.avq,
                     ws.avd, ws.rec, ws.ex_pair, ws.P, ne, d, ef, rsg, nhl, sel);
  const long n = (long)T * d;
  hipLaunchKernelGGL(kq4_moe_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     Y, ws.P, sel, pr, T, tk, d, ne);
  return (int)hipGetLastError();
}

int kq4_launch_moe(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                   const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                   const KQ4MoeWs &ws, hipStream_t s) {
  return kq4_launch_moe_dbg(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, ws, nullptr, nullptr,
                            nullptr, nullptr, s);
}
