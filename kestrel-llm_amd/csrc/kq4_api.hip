// kq4_api.hip - C ABI of libkq4.so (declared in include/kq4.h): argument checks, per-device
// workspaces, the weight cache of the host-pointer drop-in API, and kernel dispatch.
#include "../../include/kq4.h"
#include "kq4_common.h"
#include "kq4_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

// Error reporting for the library's C host files (kq4_err.h).
extern "C" __attribute__((visibility("hidden"))) int kq4_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

namespace {

#define KQ4_HIP(call)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess) return fail(KQ4_EHIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

struct Buf {
  void *p = nullptr;
  size_t cap = 0;
};

struct WEntry {
  uint8_t *p;
  size_t bytes;
  uint64_t fp;   // fingerprint of the host bytes it was uploaded from
};

const int kMaxDev = 16;

struct DevState {
  bool ready = false;
  int ncu = 256;        // compute units (sizes the GEMV grid)
  Buf ws;    // device-API workspace: quantized activations, MoE routing and staging
  std::vector<void *> retired;   // outgrown device-API workspaces, freed by kq4_shutdown
  Buf hx, hu, hres, hout, hw, hsel, hpr, hstage;   // staging for the host-pointer API
  std::unordered_map<uint64_t, WEntry> wcache;
  uint8_t *scratch = nullptr;   // this device's address of kq4_scratch (set by kq4_init)
};

DevState g_dev[kMaxDev];

// Scratch of kq4_matmul_noalloc_dev, the entry point that allocates nothing: a file-scope device
// array, one copy per GPU at its own address, held until the process ends. Host code never
// passes `kq4_scratch` itself to a kernel (on the host that name is a stand-in, not a device
// address): kq4_init looks up each device's address with hipGetSymbolAddress and the entry point
// carves its buffers from DevState::scratch.
__device__ __align__(256) uint8_t kq4_scratch[KQ4_NOALLOC_SCRATCH_BYTES];
std::mutex g_mu;   // guards lazy init / cache maps (the op itself is single-caller)

inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

int cur_dev(DevState **out) {
  int d = 0;
  KQ4_HIP(hipGetDevice(&d));
  if (d < 0 || d >= kMaxDev) return fail(KQ4_ENODEV, "device %d out of range", d);
  if (!g_dev[d].ready) {
    int rc = kq4_init(d);
    if (rc != KQ4_OK) return rc;
  }
  *out = &g_dev[d];
  return KQ4_OK;
}

size_t grow_size(size_t bytes) { return al256(bytes > 4096 ? bytes + bytes / 4 : 4096); }

// Staging buffers of the host-pointer API, whose calls are synchronous and cannot be captured
// (they copy from and to host memory): grown by freeing the old buffer once the device is idle.
int ensure(Buf &b, size_t bytes) {
  if (b.cap >= bytes) return KQ4_OK;
  const size_t n = grow_size(bytes);
  if (b.p) {
    KQ4_HIP(hipDeviceSynchronize());   // in-flight kernels may still read the old buffer
    KQ4_HIP(hipFree(b.p));
    b.p = nullptr;
    b.cap = 0;
  }
  if (hipMalloc(&b.p, n) != hipSuccess) {
    b.p = nullptr;
    return fail(KQ4_ENOMEM, "hipMalloc(%zu) failed", n);
  }
  b.cap = n;
  return KQ4_OK;
}

// A device-API call's workspace: the device's growable one, or a fixed buffer it must fit in.
struct Ws {
  Buf *b;
  DevState *ds;   // nullptr: fixed (never grows)
};

// Makes ws hold at least `bytes`. A HIP graph captured around a device-API call keeps the
// workspace address it was recorded with, so a workspace is never freed while the library runs:
// growth allocates a larger one and retires the old one (freed by kq4_shutdown), which graphs
// captured before the growth go on using. Growth needs hipMalloc, which stream capture does not
// allow, so a call on a capturing stream that would grow the workspace fails with KQ4_EINVAL
// before it launches anything (kq4_workspace_reserve sizes it beforehand).
int ensure_ws(const Ws &ws, size_t payload, hipStream_t s) {
  Buf &b = *ws.b;
  const size_t bytes = payload;
  if (b.cap >= bytes) return KQ4_OK;
  if (!ws.ds)
    return fail(KQ4_EINVAL, "the call needs %zu B of workspace; its fixed buffer holds %zu B",
                bytes, b.cap);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  KQ4_HIP(hipStreamIsCapturing(s, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(KQ4_EINVAL, "the workspace must grow to %zu B (it holds %zu B) while the stream "
                "is being captured; call kq4_workspace_reserve before capturing", bytes, b.cap);
  const size_t n = grow_size(bytes);
  void *p = nullptr;
  if (hipMalloc(&p, n) != hipSuccess) return fail(KQ4_ENOMEM, "hipMalloc(%zu) failed", n);
  if (b.p) ws.ds->retired.push_back(b.p);
  b.p = p;
  b.cap = n;
  return KQ4_OK;
}

struct Carve {   // bump allocator over a workspace
  char *base;
  size_t off = 0;
  template <class T>
  T *take(size_t count) {
    T *p = reinterpret_cast<T *>(base + off);
    off += al256(count * sizeof(T));
    return p;
  }
};

// Bytes of a matmul's quantized activations (int8 codes + f32 scales, token-major) in the
// workspace, and of the fp8 GEMM's operand pairs (64 B per token and block) + scales.
size_t qa_bytes(int n, int cols) {
  return al256((size_t)n * cols) + al256((size_t)n * (cols / 32) * sizeof(float));
}
size_t f8_bytes(int n, int cols) {
  return al256((size_t)n * (cols / 32) * 64) + al256((size_t)n * (cols / 32) * sizeof(float));
}

bool shape_ok(int rows, int cols) { return rows > 0 && rows % 4 == 0 && cols > 0 && cols % 32 == 0; }

int env_int(const char *name, int dflt) {
  const char *e = getenv(name);
  return e ? atoi(e) : dflt;
}

// Tuning options (measurement and tests): initial values from the environment variable of each
// (KQ4_ + the name in upper case), changed at run time by kq4_set_option. -1 = the planner's
// choice where a planner chooses.
enum OptId {
  kGemvKind, kGemvMfmaFrom, kGemvHs, kGemvRps, kGemvWaves, kGemvWpcu, kGemvMaxw,
  kGemvFq, kGemvFqWork, kGemvSiluFqWork, kGemvChunkMax, kGemmKind, kGemmTile, kGemmSplit,
  kGemmPrio, kOptCount
};
struct OptDef {
  const char *name, *env;
  int dflt;
};
const OptDef kOpts[kOptCount] = {
    {"gemv_kind", "KQ4_GEMV_KIND", -1},          {"gemv_mfma_from", "KQ4_GEMV_MFMA_FROM", 2},
    {"gemv_hs", "KQ4_GEMV_HS", -1},              {"gemv_rps", "KQ4_GEMV_RPS", -1},
    {"gemv_waves", "KQ4_GEMV_WAVES", -1},
    {"gemv_wpcu", "KQ4_GEMV_WPCU", 64},          {"gemv_maxw", "KQ4_GEMV_MAXW", 16},
    {"gemv_fq", "KQ4_GEMV_FQ", -1},              {"gemv_fq_work", "KQ4_GEMV_FQ_WORK", 50000},
    {"gemv_silu_fq_work", "KQ4_GEMV_SILU_FQ_WORK", 15000},
    {"gemv_chunk_max", "KQ4_GEMV_CHUNK_MAX", 16},
    {"gemm_kind", "KQ4_GEMM_KIND", -1},          {"gemm_tile", "KQ4_GEMM_TILE", 0},
    {"gemm_split", "KQ4_GEMM_SPLIT", -1},        {"gemm_prio", "KQ4_GEMM_PRIO", -1},
};
std::atomic<int> g_opt[kOptCount];
int g_opt_init[kOptCount];   // each option's value at load: its environment variable or default
std::once_flag g_opt_once;

int opt(OptId i) {
  std::call_once(g_opt_once, [] {
    for (int k = 0; k < kOptCount; ++k) {
      g_opt_init[k] = env_int(kOpts[k].env, kOpts[k].dflt);
      g_opt[k] = g_opt_init[k];
    }
  });
  return g_opt[i].load(std::memory_order_relaxed);
}

int asm_tokens_for(int chain, int n) {
  if (chain == KQ4_CHAIN_ASM) return n;
  if (chain == KQ4_CHAIN_AUTO) return n > 3 ? (n & ~3) : 0;
  return 0;
}

// Integer-dot kind of the GEMV: per-lane v_dot4 for one token, v_mfma from two tokens on (the
// dot4 work grows with M, the MFMA's does not; at one token both measure the same).
// Option gemv_kind = 0/1 forces one (for measurement).
// Most q4 tokens the GEMV takes (its 16-token kernel from 9 on): option gemv_chunk_max, at most 16.
int gemv_q4_max() {
  const int c = opt(kGemvChunkMax);
  return c < KQ4_GEMV_WIDE_M ? c : KQ4_GEMV_WIDE_M;
}

int gemv_kind(int n) {
  const int force = opt(kGemvKind);
  if (force == 1 || (force == 0 && n <= KQ4_GEMV_DOT4_MAX_M)) return force;
  return n >= opt(kGemvMfmaFrom) || n > KQ4_GEMV_DOT4_MAX_M ? 1 : 0;
}

// GEMV launch shape (kq4_gemv_impl.h). A group of output rows is R whole 32-row sets (rps), or
// half (hs = 1) or a quarter (hs = 2) of one set, one workgroup each, of nw waves that take the
// K stages (16 blocks of q4) in turn. Chosen from a
// sweep of every combination over the Qwen3-8B and Qwen3-VL-2B decode shapes at M = 1, 2, 4, 8
// on MI355X (graph replay, weights streamed from HBM):
//   * hs: quarter sets when the launch has at most one set per 4 CUs, half sets below two sets
//     per CU, whole sets beyond - and whole sets from two tokens on when K has at least 8
//     stages and there are at least 3 sets per 4 CUs (Qwen3-8B QKV, 192 sets: 6.97 against
//     7.85 us at M = 4);
//   * rps: 3 sets per workgroup from 4 tokens on when whole sets fill the chip, with the
//     activations quantized in the kernel, once for the 3 sets (Qwen3-8B gate/up pair at M = 4:
//     14.7 against 16.0 us); 1 otherwise (at fewer tokens the lower wave count costs more);
//   * waves: about gemv_wpcu (64) per CU over the launch, at most one per stage and 16 per
//     workgroup (8 with rps > 1), balanced so that no wave has more stages than another by more
//     than one.
// Options gemv_hs / _rps / _waves / _maxw / _wpcu override it (measurement, tests).
struct GemvPlan {
  int hs, rps, nw, groups;
};

GemvPlan plan_gemv(int n_mats, const int *rows, int nst, int ncu, int n) {
  const int force_hs = opt(kGemvHs), force_r = opt(kGemvRps);
  const int force_w = opt(kGemvWaves), per_cu = opt(kGemvWpcu);
  const int max_w = opt(kGemvMaxw) >= 1 && opt(kGemvMaxw) <= 16 ? opt(kGemvMaxw) : 16;
  int sets = 0;
  for (int i = 0; i < n_mats; ++i) sets += (rows[i] + 31) / 32;
  GemvPlan p;
  p.hs = force_hs >= 0 && force_hs <= 2                  ? force_hs
         : 4 * sets <= ncu                                   ? 2
         : sets >= 2 * ncu || (n >= 2 && nst >= 8 && 4 * sets >= 3 * ncu) ? 0
                                                             : 1;
  p.rps = force_r >= 1 && force_r <= KQ4_GEMV_MAX_RPS ? force_r
          : n >= 4 && sets >= 2 * ncu                 ? 3
                                                      : 1;
  if (p.hs) p.rps = 1;
  if (n > KQ4_GEMV_MAX_M && p.hs > 1) p.hs = 1;   // the 16-token kernel: whole or half sets
  p.groups = 0;
  for (int i = 0; i < n_mats; ++i) p.groups += ((rows[i] + 31) / 32 + p.rps - 1) / p.rps << p.hs;
  const int wgs = p.groups;
  int want = force_w > 0 ? force_w : (per_cu * ncu + wgs - 1) / wgs;
  int mw = p.rps > 1 && max_w > KQ4_GEMV_RPS_MAX_WAVES ? KQ4_GEMV_RPS_MAX_WAVES : max_w;
  const int lds_w = (160 * 1024 - 64) / kq4_gemv_slab_bytes(n);   // slabs that fit a CU's LDS
  mw = mw < lds_w ? mw : lds_w;
  const int cap = nst < mw ? nst : mw;
  want = want < 1 ? 1 : (want > cap ? cap : want);
  const int spw = (nst + want - 1) / want;   // stages per wave
  p.nw = (nst + spw - 1) / spw;
  return p;
}

// Whether the GEMV quantizes its fp32 activations itself (one launch per op) or reads them from
// a separate quantize launch (about 2 us more per op in a graph). Every workgroup quantizes its
// K slice of the activation for itself, so a CU spends VALU time on that many elements per
// workgroup it runs: work = n * (K slice) * ceil(workgroups / CUs). From the sweep above, the
// in-kernel path is faster up to about 50K such elements at 1-4 tokens and 33K at 5-8 (two
// quantization passes), always with several sets per workgroup, and with the SiLU product
// (about 30 more instructions per element) up to about 15K. (Re-measured with the faster
// quantizer launch: raising the limits from 45K / 20K moved Qwen3-8B QKV at 5-8 tokens and
// down at 4, Qwen3-VL-2B gate/up and down at 5 into the kernel, each 0.4-1.6 us faster.)
// Option gemv_fq = 0 / 1 forces it off / on; gemv_fq_work (the 1-4-token limit; 2/3 of it
// from 5 tokens) and gemv_silu_fq_work set the limits.
bool gemv_fq(long work, int n, int rps, bool silu) {
  const int force = opt(kGemvFq);
  if (force == 0 || force == 1) return force;
  if (silu) return work <= opt(kGemvSiluFqWork);
  return rps > 1 || work <= (n <= 4 ? opt(kGemvFqWork) : opt(kGemvFqWork) * 2 / 3);
}

// Tile and K slices of each matrix's prefill GEMM (kq4_gemm_plan) into pl[], and the workspace
// bytes of their partial sums: one buffer for the largest, reused matrix after matrix (the
// launches are stream-ordered).
size_t split_bytes(int n_mats, const int *rows, int cols, int n, int wf, int chain, int ncu,
                   KQ4GemmPlan *pl) {
  size_t mx = 0;
  for (int i = 0; i < n_mats; ++i) {
    const int ft = opt(kGemmTile);
    pl[i] = kq4_gemm_plan(n, rows[i], cols, wf, chain, ncu, ft >= 1 && ft <= 4 ? ft : -1,
                          opt(kGemmSplit));
    const size_t b = (size_t)(pl[i].ksplit - 1) * n * rows[i] * sizeof(float);
    mx = b > mx ? b : mx;
  }
  return al256(mx);
}

// GEMV over n_mats matrices for n tokens (n <= 8; q4 up to 16 in the 16-token kernel): from fp32
// x (quantized in the kernel or by a separate launch; with xu the activation is
// silu_mul(x, xu), quantized apart beyond 8 tokens) or from token-major xq/xd.
int run_gemv(DevState *ds, const Ws &wsp, int n_mats, float *const *out, const float *const *res,
             const uint8_t *const *w, const int *rows, int cols, const float *x, const float *xu,
             const int8_t *xq, const float *xd, int n, int asm_tokens, hipStream_t s,
             int wf = 0) {
  const int nb = cols / 32;
  const int cb = wf ? KQ8_STREAM_CB : KQ4_STREAM_CB;   // q8 stages hold 8 blocks
  const int nst = (nb + cb - 1) / cb;
  int rc;
  KQ4GemvArgs a;
  memset(&a, 0, sizeof(a));
  GemvPlan pl = plan_gemv(n_mats, rows, nst, ds->ncu, n);
  const int kind = wf ? 1 : gemv_kind(n);
  // the quantized activations (when quantized apart) in the workspace
  const int wgs = pl.groups;
  bool fq = false;
  if (x) {
    const long per_cu = ((long)wgs + ds->ncu - 1) / ds->ncu;
    // Q8_0 stages stream twice the weight bytes per element, which leaves the in-kernel
    // quantization less time to hide in: its work counts 5/3 (Qwen3-8B q8 gate / down at M = 4,
    // 32K / 49K elements: 16.3 / 14.6 us in the kernel against 15.4 / 14.3 us with the quantizer
    // launch; at M = 2 the kernel form 13.3 / 12.6 against 14.9 / 14.0 us)
    fq = gemv_fq(per_cu * n * cols * (wf ? 5 : 3) / 3, n, pl.rps, xu != nullptr);
    if (n > KQ4_GEMV_MAX_M && xu) fq = false;   // the 16-token kernel quantizes plain x only
  }
  const size_t qbytes = x && !fq ? qa_bytes(n, cols) : 0;
  if (qbytes && (rc = ensure_ws(wsp, qbytes, s))) return rc;
  Carve cv{static_cast<char *>(wsp.b->p)};
  if (x) {
    if (fq) {
      a.xf = x;
      a.xu = xu;
    } else {
      int8_t *q = cv.take<int8_t>((size_t)n * cols);
      float *d = cv.take<float>((size_t)n * nb);
      KQ4_HIP((hipError_t)kq4_launch_quantize(x, q, d, nullptr, n, cols, 0, s, 0, xu));
      xq = q;
      xd = d;
    }
  }
  a.nmat = n_mats;
  a.xq = xq;
  a.xd = xd;
  a.asm_tokens = asm_tokens;
  a.cols = cols;
  a.nb = nb;
  a.wf = wf;
  a.nw = pl.nw;
  a.ntok = n;
  int g = 0;
  for (int i = 0; i < n_mats; ++i) {
    KQ4GemvMat &m = a.mat[i];
    m.w = w[i];
    m.out = out[i];
    m.res = res ? res[i] : nullptr;
    m.rows = rows[i];
    m.wg_begin = g;
    g += ((rows[i] + 31) / 32 + pl.rps - 1) / pl.rps << pl.hs;
  }
  KQ4_HIP((hipError_t)kq4_launch_gemv(a, n, kind, pl.hs, pl.rps, wgs, s));
  return KQ4_OK;
}

// x (fp32; with xu the activation is silu_mul(x, xu)) or xq_in/xd_in (pre-quantized).
// wsp (may be null): the workspace to carve instead of the device's growable one.
int matmul_impl(int n_mats, float *const *out, const float *const *res, const uint8_t *const *w,
                const int *rows, int cols, const float *x, const int8_t *xq_in,
                const float *xd_in, int n, int chain, hipStream_t s, const float *xu = nullptr,
                int wf = 0, const Ws *wsp = nullptr) {
  if (n_mats < 1 || n_mats > KQ4_MAX_MATS) return fail(KQ4_EINVAL, "n_mats=%d", n_mats);
  if (wf ? (chain != KQ4_CHAIN_AUTO && chain != KQ4_CHAIN_GEMV32 && chain != KQ4_CHAIN_Q8GEMM)
         : (chain < KQ4_CHAIN_AUTO || chain > KQ4_CHAIN_ASM))
    return fail(KQ4_EINVAL, "chain=%d", chain);
  if (wf && xu) return fail(KQ4_EINVAL, "the SiLU form takes q4 weights");
  if (n < 0) return fail(KQ4_EINVAL, "n_batch=%d", n);
  for (int i = 0; i < n_mats; ++i) {
    if (!shape_ok(rows[i], cols))
      return fail(KQ4_EINVAL, "rows=%d cols=%d: need rows%%4==0, cols%%32==0", rows[i], cols);
    if (!w[i] || !out[i]) return fail(KQ4_EINVAL, "null weight/output pointer");
    if ((uintptr_t)w[i] % 16) return fail(KQ4_EINVAL, "weights not 16-byte aligned");
  }
  if (n == 0) return KQ4_OK;
  if ((x && (uintptr_t)x % 16) || (xu && (uintptr_t)xu % 16) || (xq_in && (uintptr_t)xq_in % 16) ||
      (xd_in && (uintptr_t)xd_in % 4))
    return fail(KQ4_EINVAL, "activations not aligned (x, up, xq: 16 B; xd: 4 B)");
  if (xu && !x) return fail(KQ4_EINVAL, "up without gate");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  const Ws ws = wsp ? *wsp : Ws{&ds->ws, ds};
  const int nb = cols / 32;
  const size_t qbytes = qa_bytes(n, cols);

  // q4 weights, 9 to gemv_chunk_max tokens (16): the decode GEMV's 16-token kernel, one launch
  // that reads the weights once (the rows past n padding): below ~24 tokens the prefill GEMM's
  // per-tile stage chain is latency-bound and slower. Its int8 work is the MFMA's 32 rows
  // either way, so 16 tokens cost about what 8 do. The AUTO chain puts the first n & ~3 tokens on
  // the ASM scale rounding, as the reference's dispatch over the whole batch does. Outputs as the
  // GEMV's: within 1e-5 of the reference chain, not bit-identical to it. Q8_0 weights stay on the
  // GEMM (their 8-token GEMV launches at twice the bytes measured slower there).
  if (!wf && n > KQ4_GEMV_MAX_M && n <= gemv_q4_max())
    return run_gemv(ds, ws, n_mats, out, res, w, rows, cols, x, xu, xq_in, xd_in, n,
                    asm_tokens_for(chain, n), s);

  if (wf) {
    // Q8_0: the VDOT chain (f32 activation scale, fused) or the GEMM chain (f16-rounded scale,
    // unfused) for every token; AUTO takes VDOT for one token and GEMM from two on, as the
    // reference's q8 wrappers dispatch (vllm_safetensors.c:5977-6001, :6071-6091)
    const bool gchain = chain == KQ4_CHAIN_Q8GEMM || (chain == KQ4_CHAIN_AUTO && n >= 2);
    if (n <= KQ4_GEMV_MAX_M)
      return run_gemv(ds, ws, n_mats, out, res, w, rows, cols, x, nullptr, xq_in, xd_in, n,
                      gchain ? n : 0, s, gchain ? 2 : 1);
    const int qc = gchain ? KQ4_CHAIN_Q8GEMM : KQ4_CHAIN_GEMV32;
    KQ4GemmPlan pl[KQ4_MAX_MATS];
    const size_t pbytes = split_bytes(n_mats, rows, cols, n, 1, qc, ds->ncu, pl);
    if ((rc = ensure_ws(ws, qbytes + pbytes, s))) return rc;
    Carve cv{static_cast<char *>(ws.b->p)};
    KQ4GemmAct act{xq_in, cols, 32, xd_in, nb, 1};
    if (x) {
      int8_t *q = cv.take<int8_t>((size_t)n * cols);
      float *d = cv.take<float>((size_t)n * nb);
      KQ4_HIP((hipError_t)kq4_launch_quantize(x, q, d, nullptr, n, cols, 0, s, 0));
      act = KQ4GemmAct{q, cols, 32, d, nb, 1};
    } else {
      cv.off = qbytes;
    }
    float *part = pbytes ? cv.take<float>(pbytes / sizeof(float)) : nullptr;
    for (int i = 0; i < n_mats; ++i)
      KQ4_HIP((hipError_t)kq4_launch_gemm(out[i], res ? res[i] : nullptr, w[i], act, rows[i],
                                          cols, n, qc, ds->ncu, s, 1, pl[i].tile, pl[i].ksplit,
                                          part, opt(kGemmPrio)));
    return KQ4_OK;
  }

  if (n <= KQ4_GEMV_MAX_M)
    return run_gemv(ds, ws, n_mats, out, res, w, rows, cols, x, xu, xq_in, xd_in, n,
                    asm_tokens_for(chain, n), s);

  // prefill: MFMA GEMM on the main segment, GEMV on the 1..3-token CTILE tail (AUTO)
  const int main_n = chain == KQ4_CHAIN_AUTO ? (n & ~3) : n;
  const int tail = n - main_n;
  const int main_chain = chain == KQ4_CHAIN_AUTO ? KQ4_CHAIN_ASM : chain;
  if (x && (main_chain == KQ4_CHAIN_ASM || main_chain == KQ4_CHAIN_GEMV32) && opt(kGemmKind) == 1) {
    // fp8 operands (kq4_launch_gemm_f8): the main segment's activations quantized once into
    // e4m3 operand pairs, the tail tokens by the GEMV from their fp32 rows
    if ((rc = ensure_ws(ws, f8_bytes(main_n, cols), s))) return rc;
    Carve cv{static_cast<char *>(ws.b->p)};
    uint8_t *xp = cv.take<uint8_t>((size_t)main_n * nb * 64);
    float *d = cv.take<float>((size_t)main_n * nb);
    KQ4_HIP((hipError_t)kq4_launch_quantize(x, reinterpret_cast<int8_t *>(xp), d, nullptr, main_n,
                                            cols, 0, s, 2, xu));
    for (int i = 0; i < n_mats; ++i)
      KQ4_HIP((hipError_t)kq4_launch_gemm_f8(out[i], res ? res[i] : nullptr, w[i], xp, d,
                                             rows[i], cols, main_n, main_chain, ds->ncu, s,
                                             opt(kGemmTile)));
    if (!tail) return KQ4_OK;
    float *o2[KQ4_MAX_MATS];
    const float *r2[KQ4_MAX_MATS];
    for (int i = 0; i < n_mats; ++i) {
      o2[i] = out[i] + (size_t)main_n * rows[i];
      r2[i] = (res && res[i]) ? res[i] + (size_t)main_n * rows[i] : nullptr;
    }
    return run_gemv(ds, ws, n_mats, o2, r2, w, rows, cols, x + (size_t)main_n * cols,
                    xu ? xu + (size_t)main_n * cols : nullptr, nullptr, nullptr, tail, 0, s);
  }
  KQ4GemmPlan pl[KQ4_MAX_MATS];
  const size_t pbytes = split_bytes(n_mats, rows, cols, main_n, 0, main_chain, ds->ncu, pl);
  if ((rc = ensure_ws(ws, qbytes + pbytes, s))) return rc;
  Carve cv{static_cast<char *>(ws.b->p)};
  KQ4GemmAct act;
  const int8_t *xq_t = nullptr;
  const float *xd_t = nullptr;
  if (x) {
    // every token at once, token-major (contiguous stores; the GEMM's staging reads 32-byte
    // token rows per block at a stride, and the tail GEMV reads its rows as they are)
    int8_t *q = cv.take<int8_t>((size_t)n * cols);
    float *d = cv.take<float>((size_t)n * nb);
    KQ4_HIP((hipError_t)kq4_launch_quantize(x, q, d, nullptr, n, cols, 0, s, 0, xu));
    act = KQ4GemmAct{q, cols, 32, d, nb, 1};
    xq_t = q + (size_t)main_n * cols;
    xd_t = d + (size_t)main_n * nb;
  } else {
    cv.off = qbytes;
    act = KQ4GemmAct{xq_in, cols, 32, xd_in, nb, 1};
    xq_t = xq_in + (size_t)main_n * cols;
    xd_t = xd_in + (size_t)main_n * nb;
  }
  float *part = pbytes ? cv.take<float>(pbytes / sizeof(float)) : nullptr;
  for (int i = 0; i < n_mats; ++i)
    KQ4_HIP((hipError_t)kq4_launch_gemm(out[i], res ? res[i] : nullptr, w[i], act, rows[i], cols,
                                        main_n, main_chain, ds->ncu, s, 0, pl[i].tile,
                                        pl[i].ksplit, part, opt(kGemmPrio)));
  if (tail) {
    float *o2[KQ4_MAX_MATS];
    const float *r2[KQ4_MAX_MATS];
    for (int i = 0; i < n_mats; ++i) {
      o2[i] = out[i] + (size_t)main_n * rows[i];
      r2[i] = (res && res[i]) ? res[i] + (size_t)main_n * rows[i] : nullptr;
    }
    return run_gemv(ds, ws, n_mats, o2, r2, w, rows, cols, nullptr, nullptr, xq_t, xd_t, tail, 0,
                    s);
  }
  return KQ4_OK;
}

// Workspace bytes of the expert FFN's staging (expert CSR, slot records, quantized X and av,
// unweighted partials) and of the fused layer's routing (logits, sel, pr) carved before it.
size_t moe_stage_bytes(int T, int tk, int ne, int d, int ef) {
  const size_t np = (size_t)T * tk;
  return al256((ne + 1) * sizeof(int)) + al256(np * sizeof(int)) +
         al256((size_t)ne * KQ4_MOE_REC * sizeof(int)) + al256((size_t)T * d) +
         al256((size_t)T * (d / 32) * sizeof(float)) + al256(np * ef) +
         al256(np * (ef / 32) * sizeof(float)) + al256(np * d * sizeof(float));
}

size_t moe_route_bytes(int T, int tk, int ne) {
  const size_t np = (size_t)T * tk;
  return al256((size_t)T * ne * sizeof(float)) + al256(np * sizeof(int)) +
         al256(np * sizeof(float));
}

// The expert FFN; its staging is carved from the workspace at byte offset `off` (the fused
// layer call keeps its routing below it).
int moe_impl(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
             const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
             float *g_out, float *u_out, float *av_out, const float *av_in, hipStream_t s,
             size_t off = 0) {
  if (T < 0 || tk < 1 || tk > 32 || ne < 1 || !kq4_moe_shape_ok(d, ef))
    return fail(KQ4_EINVAL, "moe: T=%d tk=%d ne=%d d=%d ef=%d (need d, ef %% 32 == 0, "
                "d <= 4096, ef <= 3840)", T, tk, ne, d, ef);
  if (!G || !U || !D || (uintptr_t)G % 16 || (uintptr_t)U % 16 || (uintptr_t)D % 16)
    return fail(KQ4_EINVAL, "moe: null or misaligned (16 B) weights");
  if (T == 0) return KQ4_OK;
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  const size_t np = (size_t)T * tk;
  if ((rc = ensure_ws(Ws{&ds->ws, ds}, off + moe_stage_bytes(T, tk, ne, d, ef), s))) return rc;
  Carve cv{static_cast<char *>(ds->ws.p), off};
  KQ4MoeWs ws;
  ws.ex_off = cv.take<int>(ne + 1);
  ws.ex_pair = cv.take<int>(np);
  ws.rec = cv.take<int>((size_t)ne * KQ4_MOE_REC);
  ws.xq = cv.take<int8_t>((size_t)T * d);
  ws.xd = cv.take<float>((size_t)T * (d / 32));
  ws.avq = cv.take<int8_t>(np * ef);
  ws.avd = cv.take<float>(np * (ef / 32));
  ws.P = cv.take<float>(np * d);
  ws.ncu = ds->ncu;
  KQ4_HIP((hipError_t)kq4_launch_moe_dbg(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, ws, g_out,
                                         u_out, av_out, av_in, s));
  return KQ4_OK;
}

// ---- host-pointer API helpers --------------------------------------------------------------

size_t wbytes(int rows, int cols) { return (size_t)(rows / 4) * (cols / 32) * 72; }

// Fingerprint of a host weight buffer: FNV-1a over the size and 64 spans of 64 bytes spread
// evenly from the first byte to the last (4 KB read per call; every byte when the buffer is at
// most 4 KB). A cache entry whose key was reused for different weights (e.g. a freed and
// reallocated host buffer) is re-uploaded instead of served stale whenever one sampled span
// differs. The key is the caller's promise, as it is for the reference's NPU weight cache
// (include/npu/vllm_npu.h:135-159); the fingerprint catches a broken promise for any two
// different matrices (they differ throughout), not a change confined to unsampled bytes.
uint64_t fingerprint(const uint8_t *w, size_t bytes) {
  constexpr size_t kSpans = 64, kSpan = 64;
  uint64_t h = 1469598103934665603ull;
  for (int i = 0; i < 8; ++i) h = (h ^ ((bytes >> (8 * i)) & 0xFF)) * 1099511628211ull;
  auto mix = [&](size_t o, size_t n) {
    for (size_t i = 0; i < n; ++i) h = (h ^ w[o + i]) * 1099511628211ull;
  };
  if (bytes <= kSpans * kSpan) {
    mix(0, bytes);
    return h;
  }
  for (size_t k = 0; k < kSpans; ++k)   // span k starts at k/(kSpans-1) of the way to the end
    mix((bytes - kSpan) / (kSpans - 1) * k, kSpan);
  return h;
}

// Device copy of host VQF weights in the stream layout: from the cache under wkey (uploaded and
// repacked once), or for wkey == 0 repacked into `tmp` for this call only. The VQF bytes go
// through the staging buffer hstage; everything runs on the null stream, so it is ordered before
// the kernels that read the copy.
// g = 0: q4 VQF 4x4 tiles; g = 8 / 4: Q8_0 tiles of g rows (kept under wkey with bit 63 set, so
// a layer's q4 and q8 copies of one projection do not collide).
int dev_weights(DevState *ds, uint64_t wkey, const uint8_t *w, int rows, int cols, Buf &tmp,
                const uint8_t **dev, int g = 0) {
  const size_t bytes = g ? (size_t)rows * (cols / 32) * 34 : wbytes(rows, cols);
  const size_t sbytes = g ? kq8_stream_bytes(rows, cols) : kq4_stream_bytes(rows, cols);
  if (wkey && g) wkey |= 1ull << 63;
  const uint64_t fp = wkey ? fingerprint(w, bytes) : 0;
  if (wkey) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = ds->wcache.find(wkey);
    if (it != ds->wcache.end() && it->second.bytes == bytes && it->second.fp == fp) {
      *dev = it->second.p;
      return KQ4_OK;
    }
  }
  int rc = ensure(ds->hstage, bytes);
  if (rc) return rc;
  KQ4_HIP(hipMemcpy(ds->hstage.p, w, bytes, hipMemcpyHostToDevice));
  uint8_t *dst = nullptr;
  if (wkey) {
    void *p = nullptr;
    if (hipMalloc(&p, sbytes) != hipSuccess) return fail(KQ4_ENOMEM, "weights %zu B", sbytes);
    dst = static_cast<uint8_t *>(p);
  } else {
    if ((rc = ensure(tmp, sbytes))) return rc;
    dst = static_cast<uint8_t *>(tmp.p);
  }
  const uint8_t *src = static_cast<const uint8_t *>(ds->hstage.p);
  hipError_t e = (hipError_t)(g ? kq8_launch_repack(dst, src, g, rows, cols, nullptr)
                                : kq4_launch_repack(dst, src, rows, cols, nullptr));
  if (e != hipSuccess) {
    if (wkey) (void)hipFree(dst);
    return fail(KQ4_EHIP, "weight repack: %s", hipGetErrorString(e));
  }
  if (wkey) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = ds->wcache.find(wkey);
    if (it != ds->wcache.end()) {
      (void)hipDeviceSynchronize();   // the stale copy may still be read by queued work
      (void)hipFree(it->second.p);
    }
    ds->wcache[wkey] = WEntry{dst, bytes, fp};
  }
  *dev = dst;
  return KQ4_OK;
}

}  // namespace

extern "C" {

const char *kq4_version(void) { return "kq4 0.1 (gfx950)"; }

const char *kq4_last_error(void) { return g_err; }

int kq4_init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(KQ4_ENODEV, "no HIP device");
  if (device < 0 || device >= n || device >= kMaxDev)
    return fail(KQ4_ENODEV, "device %d of %d", device, n);
  KQ4_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  KQ4_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(KQ4_ENODEV, "device %d is %s; libkq4 is built for gfx950", device,
                prop.gcnArchName);
  std::lock_guard<std::mutex> lk(g_mu);
  DevState &ds = g_dev[device];
  ds.ncu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  if (!ds.scratch) {   // once per device, with that device current
    void *p = nullptr;
    KQ4_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(kq4_scratch)));
    if (!p) return fail(KQ4_EHIP, "device %d: no address for the no-allocation scratch", device);
    ds.scratch = static_cast<uint8_t *>(p);
  }
  ds.ready = true;
  return KQ4_OK;
}

void kq4_shutdown(void) {
  int cur = 0;
  (void)hipGetDevice(&cur);
  for (int d = 0; d < kMaxDev; ++d) {
    DevState &s = g_dev[d];
    if (!s.ready) continue;
    (void)hipSetDevice(d);
    (void)hipDeviceSynchronize();
    Buf *bufs[] = {&s.ws, &s.hx, &s.hu, &s.hres, &s.hout, &s.hw, &s.hsel, &s.hpr, &s.hstage};
    for (Buf *b : bufs) {
      if (b->p) (void)hipFree(b->p);
      *b = Buf();
    }
    for (void *p : s.retired) (void)hipFree(p);
    s.retired.clear();
    for (auto &kv : s.wcache) (void)hipFree(kv.second.p);
    s.wcache.clear();
    s.ready = false;
  }
  (void)hipSetDevice(cur);
}

size_t kq4_matmul_workspace_bytes(int n_batch, int cols) {
  if (n_batch < 0 || cols <= 0 || cols % 32) return 0;
  // quantized activations (int8 or the fp8 GEMM's operand pairs) and the one-token RMSNorm row;
  // beyond the GEMV's tokens the planner's K-split partial sums, at most KQ4_SPLIT_PART_MAX
  const size_t q = qa_bytes(n_batch, cols), f = f8_bytes(n_batch, cols);
  const size_t part = n_batch > KQ4_GEMV_MAX_M ? (size_t)KQ4_SPLIT_PART_MAX : 0;
  return (q + part > f ? q + part : f) + al256((size_t)cols * sizeof(float));
}

size_t kq4_moe_workspace_bytes(int T, int tk, int ne, int d, int ef) {
  if (T < 0 || tk < 1 || tk > 32 || ne < 1 || !kq4_moe_shape_ok(d, ef)) return 0;
  return moe_route_bytes(T, tk, ne) + moe_stage_bytes(T, tk, ne, d, ef);
}

int kq4_workspace_reserve(size_t bytes) {
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  return ensure_ws(Ws{&ds->ws, ds}, bytes, nullptr);
}

int kq4_workspace_trim(void) {
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  if (ds->retired.empty()) return KQ4_OK;
  KQ4_HIP(hipDeviceSynchronize());   // work queued before the call may still read them
  hipError_t e = hipSuccess;
  for (void *p : ds->retired) {
    const hipError_t f = hipFree(p);
    if (e == hipSuccess) e = f;
  }
  ds->retired.clear();   // freed or not, never freed again
  if (e != hipSuccess) return fail(KQ4_EHIP, "workspace_trim: hipFree: %s", hipGetErrorString(e));
  return KQ4_OK;
}

int kq4_get_option(const char *name, int *value) {
  if (!name || !value) return fail(KQ4_EINVAL, "get_option: null argument");
  for (int k = 0; k < kOptCount; ++k)
    if (strcmp(name, kOpts[k].name) == 0) {
      *value = opt(static_cast<OptId>(k));
      return KQ4_OK;
    }
  return fail(KQ4_EINVAL, "get_option: unknown option %s", name);
}

int kq4_gemm_plan_info(int n_batch, int rows, int cols, int q8, int chain, int ncu, int *tile,
                       int *ksplit) {
  if (!tile || !ksplit || n_batch < 1 || !shape_ok(rows, cols))
    return fail(KQ4_EINVAL, "gemm_plan_info: n_batch=%d rows=%d cols=%d", n_batch, rows, cols);
  if (q8 ? (chain != KQ4_CHAIN_AUTO && chain != KQ4_CHAIN_GEMV32 && chain != KQ4_CHAIN_Q8GEMM)
         : (chain < KQ4_CHAIN_AUTO || chain > KQ4_CHAIN_ASM))
    return fail(KQ4_EINVAL, "gemm_plan_info: chain=%d", chain);
  if (n_batch <= KQ4_GEMV_MAX_M || (!q8 && n_batch <= gemv_q4_max())) {
    *tile = *ksplit = 0;
    return KQ4_OK;
  }
  if (ncu <= 0) {
    DevState *ds = nullptr;
    int rc = cur_dev(&ds);
    if (rc) return rc;
    ncu = ds->ncu;
  }
  // the GEMM's operands as matmul_impl forms them: q8 takes one chain for every token; q4's AUTO
  // runs ASM on the first n & ~3 tokens (the rest on the GEMV)
  const bool gchain = chain == KQ4_CHAIN_Q8GEMM || (chain == KQ4_CHAIN_AUTO && n_batch >= 2);
  const int main_n = !q8 && chain == KQ4_CHAIN_AUTO ? (n_batch & ~3) : n_batch;
  const int mc = q8 ? (gchain ? KQ4_CHAIN_Q8GEMM : KQ4_CHAIN_GEMV32)
                    : (chain == KQ4_CHAIN_AUTO ? KQ4_CHAIN_ASM : chain);
  KQ4GemmPlan pl;
  split_bytes(1, &rows, cols, main_n, q8 ? 1 : 0, mc, ncu, &pl);
  *tile = pl.tile;
  *ksplit = pl.ksplit;
  return KQ4_OK;
}

int kq4_set_option(const char *name, int value) {
  if (!name) return fail(KQ4_EINVAL, "set_option: null name");
  (void)opt(kGemvKind);   // the environment's values first
  for (int k = 0; k < kOptCount; ++k)
    if (strcmp(name, kOpts[k].name) == 0) {
      g_opt[k] = value < 0 ? g_opt_init[k] : value;
      return KQ4_OK;
    }
  return fail(KQ4_EINVAL, "set_option: unknown option %s", name);
}

int kq4_quantize_dev(int8_t *xq, float *xd, float *xde, const float *x, int n_batch, int cols,
                     int chain, void *stream) {
  if (n_batch < 0 || cols <= 0 || cols % 32 || !xq || !xd || (!x && n_batch))
    return fail(KQ4_EINVAL, "quantize: n_batch=%d cols=%d", n_batch, cols);
  if ((uintptr_t)x % 16 || (uintptr_t)xq % 8 || (uintptr_t)xd % 4 || (uintptr_t)xde % 4)
    return fail(KQ4_EINVAL, "quantize: x must be 16-byte, xq 8-byte aligned");
  KQ4_HIP((hipError_t)kq4_launch_quantize(x, xq, xd, xde, n_batch, cols,
                                          asm_tokens_for(chain, n_batch),
                                          (hipStream_t)stream, 0));
  return KQ4_OK;
}

size_t kq4_weights_stream_bytes(int rows, int cols) {
  return shape_ok(rows, cols) ? kq4_stream_bytes(rows, cols) : 0;
}

int kq4_weights_prepare_dev(uint8_t *dst, const uint8_t *w4x4, int rows, int cols,
                            void *stream) {
  if (!shape_ok(rows, cols)) return fail(KQ4_EINVAL, "prepare: rows=%d cols=%d", rows, cols);
  if (!dst || !w4x4 || (uintptr_t)dst % 16 || (uintptr_t)w4x4 % 8)
    return fail(KQ4_EINVAL, "prepare: null pointer, dst not 16-byte or w4x4 not 8-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  KQ4_HIP((hipError_t)kq4_launch_repack(dst, w4x4, rows, cols, (hipStream_t)stream));
  return KQ4_OK;
}

size_t kq4_q8_weights_stream_bytes(int rows, int cols) {
  return shape_ok(rows, cols) ? kq8_stream_bytes(rows, cols) : 0;
}

int kq4_q8_weights_prepare_dev(uint8_t *dst, const uint8_t *w_tiles, int g, int rows, int cols,
                               void *stream) {
  if ((g != 8 && g != 4) || !shape_ok(rows, cols) || rows % g)
    return fail(KQ4_EINVAL, "q8 prepare: g=%d rows=%d cols=%d", g, rows, cols);
  if (!dst || !w_tiles || (uintptr_t)dst % 16 || (uintptr_t)w_tiles % 4)
    return fail(KQ4_EINVAL, "q8 prepare: null pointer, dst not 16-byte or tiles not 4-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  KQ4_HIP((hipError_t)kq8_launch_repack(dst, w_tiles, g, rows, cols, (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_q8_weights_prepare_host(uint8_t *dst, const uint8_t *w_tiles_host, int g, int rows,
                                int cols, void *stream) {
  if ((g != 8 && g != 4) || !shape_ok(rows, cols) || rows % g)
    return fail(KQ4_EINVAL, "q8 prepare: g=%d rows=%d cols=%d", g, rows, cols);
  if (!dst || !w_tiles_host || (uintptr_t)dst % 16)
    return fail(KQ4_EINVAL, "q8 prepare: null pointer or dst not 16-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  const size_t n = (size_t)rows * (cols / 32) * 34;
  if ((rc = ensure(ds->hstage, n))) return rc;
  hipStream_t s = (hipStream_t)stream;
  KQ4_HIP(hipMemcpyAsync(ds->hstage.p, w_tiles_host, n, hipMemcpyHostToDevice, s));
  KQ4_HIP((hipError_t)kq8_launch_repack(dst, static_cast<const uint8_t *>(ds->hstage.p), g, rows,
                                        cols, s));
  KQ4_HIP(hipStreamSynchronize(s));   // the staging buffer is reused by the next call
  return KQ4_OK;
}

int kq4_q8_matmul_dev(float *out, const float *x, const float *residual, const uint8_t *w,
                      int rows, int cols, int n_batch, int chain, void *stream) {
  if (!x && n_batch) return fail(KQ4_EINVAL, "null x");
  const float *res[1] = {residual};
  return matmul_impl(1, &out, res, &w, &rows, cols, x, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream, nullptr, 1);
}

int kq4_q8_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                            const uint8_t *const *w, const int *rows, int cols, const float *x,
                            int n_batch, int chain, void *stream) {
  if (!x && n_batch) return fail(KQ4_EINVAL, "null x");
  if (!out || !w || !rows) return fail(KQ4_EINVAL, "null array argument");
  return matmul_impl(n_mats, out, residual, w, rows, cols, x, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream, nullptr, 1);
}

int kq4_weights_prepare_host(uint8_t *dst, const uint8_t *w4x4_host, int rows, int cols,
                             void *stream) {
  if (!shape_ok(rows, cols)) return fail(KQ4_EINVAL, "prepare: rows=%d cols=%d", rows, cols);
  if (!dst || !w4x4_host || (uintptr_t)dst % 16)
    return fail(KQ4_EINVAL, "prepare: null pointer or dst not 16-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  const size_t n = wbytes(rows, cols);
  if ((rc = ensure(ds->hstage, n))) return rc;
  hipStream_t s = (hipStream_t)stream;
  KQ4_HIP(hipMemcpyAsync(ds->hstage.p, w4x4_host, n, hipMemcpyHostToDevice, s));
  KQ4_HIP((hipError_t)kq4_launch_repack(dst, static_cast<const uint8_t *>(ds->hstage.p), rows,
                                        cols, s));
  KQ4_HIP(hipStreamSynchronize(s));   // the staging buffer is reused by the next call
  return KQ4_OK;
}

int kq4_matmul_dev(float *out, const float *x, const float *residual, const uint8_t *w, int rows,
                   int cols, int n_batch, int chain, void *stream) {
  if (!x && n_batch) return fail(KQ4_EINVAL, "null x");
  const float *res[1] = {residual};
  return matmul_impl(1, &out, res, &w, &rows, cols, x, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream);
}

int kq4_matmul_noalloc_dev(float *out, const float *x, const float *residual, const uint8_t *w,
                           int rows, int cols, int n_batch, int chain, void *stream) {
  if (!x && n_batch) return fail(KQ4_EINVAL, "null x");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  size_t need = 0;
  if (n_batch > 0 && cols > 0 && cols % 32 == 0) {
    if (n_batch <= KQ4_GEMV_MAX_M) {
      need = qa_bytes(n_batch, cols);
    } else {   // fp8 operands, or int8 operands and the K-split partial sums
      const int main_n = chain == KQ4_CHAIN_AUTO ? (n_batch & ~3) : n_batch;
      const int mc = chain == KQ4_CHAIN_AUTO ? KQ4_CHAIN_ASM : chain;
      KQ4GemmPlan pl;
      const size_t q = qa_bytes(n_batch, cols) + split_bytes(1, &rows, cols, main_n, 0, mc,
                                                             ds->ncu, &pl);
      const size_t f = f8_bytes(n_batch, cols);
      need = q > f ? q : f;
    }
  }
  if (need > (size_t)KQ4_NOALLOC_SCRATCH_BYTES)
    return fail(KQ4_EINVAL, "matmul_noalloc: %d tokens x %d columns need %zu B of scratch; the "
                "maximum is %u B", n_batch, cols, need, (unsigned)KQ4_NOALLOC_SCRATCH_BYTES);
  Buf b;   // the device's copy of kq4_scratch, fixed: matmul_impl carves it and never grows it
  b.p = ds->scratch;
  b.cap = KQ4_NOALLOC_SCRATCH_BYTES;
  const Ws ws{&b, nullptr};
  const float *res[1] = {residual};
  return matmul_impl(1, &out, res, &w, &rows, cols, x, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream, nullptr, 0, &ws);
}

int kq4_matmul_silu_dev(float *out, const float *gate, const float *up, const float *residual,
                        const uint8_t *w, int rows, int cols, int n_batch, int chain,
                        void *stream) {
  if ((!gate || !up) && n_batch) return fail(KQ4_EINVAL, "null gate/up");
  const float *res[1] = {residual};
  return matmul_impl(1, &out, res, &w, &rows, cols, gate, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream, up);
}

int kq4_rms_norm_dev(float *out, const float *x, const float *w, int n_batch, int d, float eps,
                     int order, void *stream) {
  if (n_batch < 0 || d <= 0 || d % 8 || d > 16384 ||
      (order != KQ4_RMS_CHUNKED && order != KQ4_RMS_SERIAL) || (n_batch && (!out || !x || !w)))
    return fail(KQ4_EINVAL, "rms_norm: n_batch=%d d=%d order=%d (d %% 8 == 0, d <= 16384)",
                n_batch, d, order);
  if ((uintptr_t)out % 16 || (uintptr_t)x % 16 || (uintptr_t)w % 16)
    return fail(KQ4_EINVAL, "rms_norm: out, x and w must be 16-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  KQ4_HIP((hipError_t)kq4_launch_rms_norm(x, w, out, nullptr, nullptr, n_batch, d, eps,
                                          order == KQ4_RMS_SERIAL, (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_rmsnorm_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                                 const uint8_t *const *w, const int *rows, int cols,
                                 const float *x, const float *norm_w, float eps, int order,
                                 float *normed, int n_batch, int chain, void *stream) {
  if (n_batch < 0 || cols > 16384 || (order != KQ4_RMS_CHUNKED && order != KQ4_RMS_SERIAL) ||
      (n_batch && (!x || !norm_w)))
    return fail(KQ4_EINVAL, "rmsnorm_matmul: n_batch=%d cols=%d order=%d", n_batch, cols, order);
  if (!out || !w || !rows) return fail(KQ4_EINVAL, "null array argument");
  if ((uintptr_t)x % 16 || (uintptr_t)norm_w % 16 || (uintptr_t)normed % 16)
    return fail(KQ4_EINVAL, "rmsnorm_matmul: x, norm_w and normed must be 16-byte aligned");
  if (n_mats < 1 || n_mats > KQ4_MAX_MATS) return fail(KQ4_EINVAL, "n_mats=%d", n_mats);
  for (int i = 0; i < n_mats; ++i)
    if (!shape_ok(rows[i], cols))
      return fail(KQ4_EINVAL, "rows=%d cols=%d: need rows%%4==0, cols%%32==0", rows[i], cols);
  if (n_batch == 0) return KQ4_OK;
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  // the normalised activations are quantized where they are formed; the matmul then reads the
  // codes (the same workspace carve matmul_impl makes for its own quantization, so it stays)
  const size_t qbytes = qa_bytes(n_batch, cols);
  // Where the GEMV would quantize fp32 activations in its own kernel (gemv_fq: one to a few
  // tokens), the norm is written in fp32 and the matmul quantizes it there (the same codes):
  // measured faster than reading the norm kernel's codes (Qwen3-8B QKV, graph replay: M = 1 by
  // 0.2-0.3 us, M = 2 9.98 -> 9.46 us, M = 4 10.47 -> 10.27 us). Where it would take a separate
  // quantizer launch instead (Qwen3-8B QKV from 5 tokens on), the norm kernel writes the codes
  // and saves that launch (M = 8 12.15 -> 10.48 us).
  bool fp32_path = false;
  // up to 4 tokens: from 5 the norm kernel's codes measured faster even where the GEMV would
  // quantize in its own kernel (Qwen3-8B QKV, M = 5 / 6 / 8: 11.1 / 11.1 / 11.1 against
  // 11.5 / 11.9 / 12.7 us)
  if (n_batch <= 4) {
    const GemvPlan pl = plan_gemv(n_mats, rows, (cols / 32 + KQ4_STREAM_CB - 1) / KQ4_STREAM_CB,
                                  ds->ncu, n_batch);
    const long per_cu = ((long)pl.groups + ds->ncu - 1) / ds->ncu;
    fp32_path = gemv_fq(per_cu * n_batch * cols, n_batch, pl.rps, false);
  }
  if (fp32_path) {
    // Without a caller buffer the fp32 rows sit above the carve matmul_impl makes for its own
    // quantization, reserved first so that matmul_impl does not reallocate.
    float *nx = normed;
    if (!nx) {
      if ((rc = ensure_ws(Ws{&ds->ws, ds},
                          qbytes + al256((size_t)n_batch * cols * sizeof(float)),
                          (hipStream_t)stream)))
        return rc;
      nx = reinterpret_cast<float *>(static_cast<char *>(ds->ws.p) + qbytes);
    }
    KQ4_HIP((hipError_t)kq4_launch_rms_norm(x, norm_w, nx, nullptr, nullptr, n_batch, cols, eps,
                                            order == KQ4_RMS_SERIAL, (hipStream_t)stream));
    return matmul_impl(n_mats, out, residual, w, rows, cols, nx, nullptr, nullptr, n_batch,
                       chain, (hipStream_t)stream);
  }
  if ((rc = ensure_ws(Ws{&ds->ws, ds}, qbytes, (hipStream_t)stream))) return rc;
  Carve cv{static_cast<char *>(ds->ws.p)};
  int8_t *q = cv.take<int8_t>((size_t)n_batch * cols);
  float *dq = cv.take<float>((size_t)n_batch * (cols / 32));
  hipStream_t s = (hipStream_t)stream;
  KQ4_HIP((hipError_t)kq4_launch_rms_norm(x, norm_w, normed, q, dq, n_batch, cols, eps,
                                          order == KQ4_RMS_SERIAL, s));
  return matmul_impl(n_mats, out, residual, w, rows, cols, nullptr, q, dq, n_batch, chain, s);
}

int kq4_silu_mul_dev(float *gate, const float *up, long n, void *stream) {
  if (n < 0 || (n && (!gate || !up))) return fail(KQ4_EINVAL, "silu_mul: n=%ld", n);
  if ((uintptr_t)gate % 16 || (uintptr_t)up % 16)
    return fail(KQ4_EINVAL, "silu_mul: gate and up must be 16-byte aligned");
  KQ4_HIP((hipError_t)kq4_launch_silu_mul(gate, up, n, (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_matmul_multi_dev(int n_mats, float *const *out, const float *const *residual,
                         const uint8_t *const *w, const int *rows, int cols, const float *x,
                         int n_batch, int chain, void *stream) {
  if (!x && n_batch) return fail(KQ4_EINVAL, "null x");
  if (!out || !w || !rows) return fail(KQ4_EINVAL, "null array argument");
  return matmul_impl(n_mats, out, residual, w, rows, cols, x, nullptr, nullptr, n_batch, chain,
                     (hipStream_t)stream);
}

int kq4_matmul_q_dev(float *out, const int8_t *xq, const float *xd, const float *residual,
                     const uint8_t *w, int rows, int cols, int n_batch, int chain, void *stream) {
  if ((!xq || !xd) && n_batch) return fail(KQ4_EINVAL, "null xq/xd");
  const float *res[1] = {residual};
  return matmul_impl(1, &out, res, &w, &rows, cols, nullptr, xq, xd, n_batch, chain,
                     (hipStream_t)stream);
}

int kq4_matmul_multi_q_dev(int n_mats, float *const *out, const float *const *residual,
                           const uint8_t *const *w, const int *rows, int cols, const int8_t *xq,
                           const float *xd, int n_batch, int chain, void *stream) {
  if ((!xq || !xd) && n_batch) return fail(KQ4_EINVAL, "null xq/xd");
  if (!out || !w || !rows) return fail(KQ4_EINVAL, "null array argument");
  return matmul_impl(n_mats, out, residual, w, rows, cols, nullptr, xq, xd, n_batch, chain,
                     (hipStream_t)stream);
}

int kq4_block_sums_dev(int32_t *s_lo, int32_t *s_hi, const int8_t *xq, const uint8_t *w, int rows,
                       int cols, int n_batch, void *stream) {
  if (!shape_ok(rows, cols) || n_batch < 0) return fail(KQ4_EINVAL, "block_sums shape");
  KQ4_HIP((hipError_t)kq4_launch_block_sums(s_lo, s_hi, xq, w, rows, cols, n_batch,
                                            (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_moe_route_dev(int *sel, float *pr, const float *logits, int T, int ne, int tk,
                      void *stream) {
  if (T < 0 || ne < 1 || ne > 2048 || tk < 1 || tk > 32 || tk > ne)
    return fail(KQ4_EINVAL, "route: T=%d ne=%d tk=%d", T, ne, tk);
  if (T == 0) return KQ4_OK;
  KQ4_HIP((hipError_t)kq4_launch_moe_route(sel, pr, logits, T, ne, tk, (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_moe_router_logits_dev(float *logits, const float *router, const float *X, int T, int ne,
                              int d, void *stream) {
  if (T < 0 || ne < 1 || d <= 0 || d % 32 || (T && (!logits || !router || !X)))
    return fail(KQ4_EINVAL, "router_logits: T=%d ne=%d d=%d (d %% 32 == 0)", T, ne, d);
  if ((uintptr_t)router % 16 || (uintptr_t)X % 16)
    return fail(KQ4_EINVAL, "router_logits: router and X must be 16-byte aligned");
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  KQ4_HIP((hipError_t)kq4_launch_moe_logits(logits, router, X, T, ne, d, (hipStream_t)stream));
  return KQ4_OK;
}

int kq4_moe_layer_dev(float *Y, const float *X, const float *router, const uint8_t *G,
                      const uint8_t *U, const uint8_t *D, int T, int ne, int tk, int d, int ef,
                      int *sel_out, float *pr_out, void *stream) {
  if (T < 0 || ne < 1 || ne > 2048 || tk < 1 || tk > 32 || tk > ne || !kq4_moe_shape_ok(d, ef) ||
      (T && (!Y || !X || !router)))
    return fail(KQ4_EINVAL, "moe_layer: T=%d ne=%d tk=%d d=%d ef=%d", T, ne, tk, d, ef);
  if ((uintptr_t)router % 16 || (uintptr_t)X % 16)
    return fail(KQ4_EINVAL, "moe_layer: router and X must be 16-byte aligned");
  if (T == 0) return KQ4_OK;
  DevState *ds = nullptr;
  int rc = cur_dev(&ds);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  const size_t np = (size_t)T * tk;
  const size_t rbytes = moe_route_bytes(T, tk, ne);
  // the routing sits below the expert FFN's staging, so the FFN does not overwrite it
  if ((rc = ensure_ws(Ws{&ds->ws, ds}, rbytes + moe_stage_bytes(T, tk, ne, d, ef), s))) return rc;
  Carve cv{static_cast<char *>(ds->ws.p)};
  float *lg = cv.take<float>((size_t)T * ne);
  int *sel = sel_out ? sel_out : cv.take<int>(np);
  float *pr = pr_out ? pr_out : cv.take<float>(np);
  KQ4_HIP((hipError_t)kq4_launch_moe_logits(lg, router, X, T, ne, d, s));
  KQ4_HIP((hipError_t)kq4_launch_moe_route(sel, pr, lg, T, ne, tk, s));
  return moe_impl(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, nullptr, nullptr, nullptr, nullptr, s,
                  rbytes);
}

int kq4_moe_ffn_dev(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                    const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                    void *stream) {
  return moe_impl(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, nullptr, nullptr, nullptr, nullptr,
                  (hipStream_t)stream);
}

int kq4_moe_ffn_stages_dev(float *Y, const float *X, const int *sel, const float *pr, int T,
                           int tk, const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne,
                           int d, int ef, float *gate_out, float *up_out, float *av_out,
                           const float *av_in, void *stream) {
  if ((gate_out == nullptr) != (up_out == nullptr))
    return fail(KQ4_EINVAL, "gate_out and up_out go together");
  return moe_impl(Y, X, sel, pr, T, tk, G, U, D, ne, d, ef, gate_out, up_out, av_out, av_in,
                  (hipStream_t)stream);
}

// ---- host-pointer drop-in API ----------------------------------------------------------------

int kq4_weights_upload(uint64_t wkey, const uint8_t *w4x4, int rows, int cols) {
  if (!wkey || !w4x4 || !shape_ok(rows, cols)) {
    fail(KQ4_EINVAL, "weights_upload: key=%llu rows=%d cols=%d", (unsigned long long)wkey, rows,
         cols);
    return 0;
  }
  DevState *ds = nullptr;
  if (cur_dev(&ds)) return 0;
  const uint8_t *dev = nullptr;
  Buf unused;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = ds->wcache.find(wkey);
    if (it != ds->wcache.end()) {
      (void)hipFree(it->second.p);
      ds->wcache.erase(it);
    }
  }
  return dev_weights(ds, wkey, w4x4, rows, cols, unused, &dev) == KQ4_OK ? 1 : 0;
}

int kq4_weights_evict(uint64_t wkey) {
  DevState *ds = nullptr;
  if (cur_dev(&ds)) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = ds->wcache.find(wkey);
  if (it == ds->wcache.end()) return 0;
  (void)hipDeviceSynchronize();
  (void)hipFree(it->second.p);
  ds->wcache.erase(it);
  return 1;
}

int kq4_weights_clear(void) {
  DevState *ds = nullptr;
  if (cur_dev(&ds)) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  const int n = (int)ds->wcache.size();
  (void)hipDeviceSynchronize();
  for (auto &kv : ds->wcache) (void)hipFree(kv.second.p);
  ds->wcache.clear();
  return n;
}

}  // extern "C"

namespace {

// The host-pointer matmul: stage x (and up) and the residuals, run on the device, read back.
int host_matmul(int n_mats, float *const *out, const float *const *residual,
                const uint8_t *const *w4x4, const int *rows, int cols, const float *x,
                const float *xu, int n_batch, int chain, const uint64_t *wkeys, int g = 0) {
  if (n_mats < 1 || n_mats > KQ4_MAX_MATS || !out || !w4x4 || !rows || !x || n_batch < 1) {
    fail(KQ4_EINVAL, "matmul: n_mats=%d n_batch=%d", n_mats, n_batch);
    return 0;
  }
  for (int i = 0; i < n_mats; ++i)
    if (!out[i] || !w4x4[i] || !shape_ok(rows[i], cols) || (g && rows[i] % g)) {
      fail(KQ4_EINVAL, "matmul: rows=%d cols=%d", rows[i], cols);
      return 0;
    }
  DevState *ds = nullptr;
  if (cur_dev(&ds)) return 0;
  // one staging buffer for x, all outputs and all residuals
  size_t ob[KQ4_MAX_MATS], total_o = 0;
  for (int i = 0; i < n_mats; ++i) {
    ob[i] = (size_t)n_batch * rows[i] * sizeof(float);
    total_o += al256(ob[i]);
  }
  const size_t xb = (size_t)n_batch * cols * sizeof(float);
  Buf tw[KQ4_MAX_MATS];
  const uint8_t *dw[KQ4_MAX_MATS];
  int rc = KQ4_OK;
  for (int i = 0; i < n_mats && !rc; ++i)
    rc = dev_weights(ds, wkeys ? wkeys[i] : 0, w4x4[i], rows[i], cols,
                     i == 0 ? ds->hw : tw[i], &dw[i], g);
  int ok = 0;
  if (!rc && !ensure(ds->hx, xb) && !ensure(ds->hout, total_o) && !ensure(ds->hres, total_o) &&
      (!xu || !ensure(ds->hu, xb))) {
    float *dout[KQ4_MAX_MATS];
    const float *dres[KQ4_MAX_MATS];
    char *po = static_cast<char *>(ds->hout.p), *pr = static_cast<char *>(ds->hres.p);
    bool good = hipMemcpy(ds->hx.p, x, xb, hipMemcpyHostToDevice) == hipSuccess &&
                (!xu || hipMemcpy(ds->hu.p, xu, xb, hipMemcpyHostToDevice) == hipSuccess);
    for (int i = 0; i < n_mats && good; ++i) {
      dout[i] = reinterpret_cast<float *>(po);
      dres[i] = nullptr;
      if (residual && residual[i]) {
        dres[i] = reinterpret_cast<const float *>(pr);
        good = hipMemcpy(pr, residual[i], ob[i], hipMemcpyHostToDevice) == hipSuccess;
      }
      po += al256(ob[i]);
      pr += al256(ob[i]);
    }
    if (good &&
        matmul_impl(n_mats, dout, dres, dw, rows, cols, static_cast<const float *>(ds->hx.p),
                    nullptr, nullptr, n_batch, chain, nullptr,
                    xu ? static_cast<const float *>(ds->hu.p) : nullptr, g ? 1 : 0) == KQ4_OK) {
      ok = 1;
      for (int i = 0; i < n_mats && ok; ++i)
        if (hipMemcpy(out[i], dout[i], ob[i], hipMemcpyDeviceToHost) != hipSuccess) {
          fail(KQ4_EHIP, "matmul readback failed");
          ok = 0;
        }
    }
  }
  bool any_tmp = false;
  for (int i = 1; i < n_mats; ++i) any_tmp = any_tmp || tw[i].p;
  if (any_tmp) (void)hipDeviceSynchronize();
  for (int i = 1; i < n_mats; ++i)
    if (tw[i].p) (void)hipFree(tw[i].p);
  return ok;
}

}  // namespace

extern "C" {

int kq4_matmul_multi(int n_mats, float *const *out, const float *const *residual,
                     const uint8_t *const *w4x4, const int *rows, int cols, const float *x,
                     int n_batch, int chain, const uint64_t *wkeys) {
  return host_matmul(n_mats, out, residual, w4x4, rows, cols, x, nullptr, n_batch, chain, wkeys);
}

int kq4_matmul(float *out, const float *x, const float *residual, const uint8_t *w4x4, int rows,
               int cols, int n_batch, int chain, uint64_t wkey) {
  const float *res[1] = {residual};
  return host_matmul(1, &out, res, &w4x4, &rows, cols, x, nullptr, n_batch, chain, &wkey);
}

int kq4_q8_matmul_multi(int n_mats, float *const *out, const float *const *residual,
                        const uint8_t *const *w_tiles, int g, const int *rows, int cols,
                        const float *x, int n_batch, int chain, const uint64_t *wkeys) {
  if (g != 8 && g != 4) {
    fail(KQ4_EINVAL, "q8 matmul: tile rows %d (8 or 4)", g);
    return 0;
  }
  return host_matmul(n_mats, out, residual, w_tiles, rows, cols, x, nullptr, n_batch, chain,
                     wkeys, g);
}

int kq4_q8_matmul(float *out, const float *x, const float *residual, const uint8_t *w_tiles,
                  int g, int rows, int cols, int n_batch, int chain, uint64_t wkey) {
  const float *res[1] = {residual};
  return kq4_q8_matmul_multi(1, &out, res, &w_tiles, g, &rows, cols, x, n_batch, chain, &wkey);
}

int kq4_matmul_silu(float *out, const float *gate, const float *up, const float *residual,
                    const uint8_t *w4x4, int rows, int cols, int n_batch, int chain,
                    uint64_t wkey) {
  if (!up) {
    fail(KQ4_EINVAL, "matmul_silu: null up");
    return 0;
  }
  const float *res[1] = {residual};
  return host_matmul(1, &out, res, &w4x4, &rows, cols, gate, up, n_batch, chain, &wkey);
}

int kq4_moe_ffn(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                uint64_t wkey) {
  if (!Y || !X || !sel || !pr || !G || !U || !D || T < 1) {
    fail(KQ4_EINVAL, "moe_ffn: null argument or T<1");
    return 0;
  }
  DevState *ds = nullptr;
  if (cur_dev(&ds)) return 0;
  if (ne < 1 || !kq4_moe_shape_ok(d, ef)) {
    fail(KQ4_EINVAL, "moe_ffn: ne=%d d=%d ef=%d", ne, d, ef);
    return 0;
  }
  const uint8_t *dG, *dU, *dD;
  Buf tg, tu, td;
  int rc = dev_weights(ds, wkey, G, ne * ef, d, tg, &dG);
  if (!rc) rc = dev_weights(ds, wkey ? wkey + 1 : 0, U, ne * ef, d, tu, &dU);
  if (!rc) rc = dev_weights(ds, wkey ? wkey + 2 : 0, D, d, ne * ef, td, &dD);
  int ok = 0;
  const size_t xb = (size_t)T * d * sizeof(float), sb = (size_t)T * tk * sizeof(int);
  if (!rc && !ensure(ds->hx, xb) && !ensure(ds->hout, xb) && !ensure(ds->hsel, sb) &&
      !ensure(ds->hpr, sb) &&
      hipMemcpy(ds->hx.p, X, xb, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(ds->hsel.p, sel, sb, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(ds->hpr.p, pr, sb, hipMemcpyHostToDevice) == hipSuccess &&
      kq4_moe_ffn_dev(static_cast<float *>(ds->hout.p), static_cast<const float *>(ds->hx.p),
                      static_cast<const int *>(ds->hsel.p), static_cast<const float *>(ds->hpr.p),
                      T, tk, dG, dU, dD, ne, d, ef, nullptr) == KQ4_OK &&
      hipMemcpy(Y, ds->hout.p, xb, hipMemcpyDeviceToHost) == hipSuccess)
    ok = 1;
  if (tg.p || tu.p || td.p) (void)hipDeviceSynchronize();
  if (tg.p) (void)hipFree(tg.p);
  if (tu.p) (void)hipFree(tu.p);
  if (td.p) (void)hipFree(td.p);
  return ok;
}

}  // extern "C"
