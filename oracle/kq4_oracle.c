/* kq4_oracle.c - scalar C restatement of kestrel-llm's Q4_0 x int8 matmul (the parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY (see kq4_oracle.h). Compiled with -O2 -ffp-contract=off and without
 * fast-math so every fp32 step below is exactly one IEEE binary32 operation; fmaf() is a single
 * fused multiply-add (the reference's vfmaq_f32 / fmla).
 *
 * The reference computes this path only in AArch64 NEON code (src/model/vllm_safetensors.c
 * "#if ST_HAVE_NEON" sections), which cannot be built here; every step below restates that
 * source text. Notation in comments: fl() = one binary32 rounding, S = integer block sum.
 *
 * The four fp32 chains (all start from 0, blocks b ascending):
 *   V1 C-tile  (q4x4_dot1_group16 vllm_safetensors.c:4180-4216, worker :4516-4557):
 *        s = fl(wd*xd); lo = fma(S_lo, s, lo); hi = fma(S_hi, s, hi); out = fl(lo+hi)
 *   V2 M4f     (q4x4_dot1_group16_gemv :4229-4251, worker :6107-6121):
 *        acc = fma(S, fl(wd*xd), acc); out = acc
 *   V3 asm     (llama_gemm_q4_0_4x4_asm.c:151-161 via repack_q8_0_4x4 :4086-4119):
 *        as V2 with xd replaced by f32(f16_rne(xd))
 *   V4 MoE int8 (q4x4_gup_actq_neon :11861-11903, moe_q4_down_group_actq_neon :11927-11968):
 *        acc = fl(acc + fl(fl(sc*xd) * S))
 *   residual (fused O / down): out = fl(resid + out)  (:4544-4549, :4317-4326, :6428-6431)
 * Dispatch (q4x4_gemm_batched :4593-4631): n_batch <= 3 -> V1 for all tokens;
 *   n_batch > 3 -> V3 on the first n_batch & ~3 tokens, V1 on the remaining 1..3.
 */
#include "kq4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 <-> f32 */

/* Exact f16 -> f32 bit pattern, subnormals normalised (vllm_safetensors.c:3614-3631; the MoE
 * decoder vq_f16 :10976-10998 computes the same value). Pinned exhaustively against numpy's
 * float16 -> float32 conversion over all 65536 codes. */
uint32_t kqo_f16_to_f32_bits(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t ex = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    if (ex == 0) {
        if (mant == 0) return sign << 31;
        int shift = 0;
        while (mant < 0x400u) { mant <<= 1; shift++; }
        return (sign << 31) | ((uint32_t)(113 - shift) << 23) | ((mant & 0x3FFu) << 13);
    }
    if (ex == 0x1F) return (sign << 31) | (0xFFu << 23) | (mant << 13);
    return (sign << 31) | ((ex + 112u) << 23) | (mant << 13);
}

float kqo_f16_to_f32(uint16_t h) {
    uint32_t b = kqo_f16_to_f32_bits(h);
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* f32 -> f16, round-to-nearest-even incl. subnormals, overflow -> inf
 * (vllm_safetensors.c:3639-3670). Pinned against numpy float32 -> float16 (IEEE RNE) over
 * every f16 midpoint, its neighbours and random bit patterns. */
uint16_t kqo_f32_to_f16_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ef = (u >> 23) & 0xFFu;
    uint32_t mant = u & 0x7FFFFFu;
    if (ef == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int32_t e = (int32_t)ef - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        uint32_t sh = (uint32_t)(14 - e);
        uint32_t half = 1u << (sh - 1);
        uint32_t rem = mant & ((1u << sh) - 1u);
        mant >>= sh;
        if (rem > half || (rem == half && (mant & 1u))) mant++;
        return (uint16_t)(sign | mant);
    }
    uint32_t rem = mant & 0x1FFFu;
    mant >>= 13;
    if (rem > 0x1000u || (rem == 0x1000u && (mant & 1u))) {
        if (++mant == 0x400u) {
            mant = 0;
            if (++e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | mant);
}

/* ---------------------------------------------------------------- weight codec */

/* Legacy Q4_0 encoder: d = (signed max)/-8, nib = clamp((int)(x*(1/d) + 8.5), 0, 15)
 * (vqf_convert/src/quant_kernels.c:118-151). Element j -> low nibble of qs[j], element
 * 16+j -> high nibble. Pinned against the reference encoder built in oracle/_ref. */
void kqo_f32_to_q4_0(uint8_t *q4_out, const float *f32_in, int n_elements) {
    int n_blocks = n_elements / 32;
    for (int b = 0; b < n_blocks; b++) {
        const float *xb = f32_in + (size_t)b * 32;
        float amax = 0.0f, maxv = 0.0f;
        for (int i = 0; i < 32; i++) {
            float av = fabsf(xb[i]);
            if (av > amax) { amax = av; maxv = xb[i]; }
        }
        float d = maxv / -8.0f;
        if (d == 0.0f) d = 1.0f;
        float id = 1.0f / d;
        uint16_t h = kqo_f32_to_f16_bits(d);
        memcpy(q4_out + (size_t)b * 18, &h, 2);
        uint8_t *qs = q4_out + (size_t)b * 18 + 2;
        for (int j = 0; j < 16; j++) {
            volatile float x0 = xb[j] * id;
            volatile float x1 = xb[16 + j] * id;
            int i0 = (int)(x0 + 8.5f), i1 = (int)(x1 + 8.5f);
            if (i0 > 15) i0 = 15;
            if (i0 < 0) i0 = 0;
            if (i1 > 15) i1 = 15;
            if (i1 < 0) i1 = 0;
            qs[j] = (uint8_t)(i0 | (i1 << 4));
        }
    }
}

/* Legacy (4 rows x 18 B per block) -> 4x4 tile (72 B): bytes [0,8) = 4 row scales (f16, row
 * order); chunk c (c = 0..15) at 8 + 4c = legacy qs bytes [(c>>2)*4, +4) of row (c&3), each
 * byte XOR 0x88 (vqf_convert/src/qk_repack.c:19-46). Pinned against the reference repack
 * built in oracle/_ref and by the round trip with kqo_unpack_4x4_to_q4_0. */
int kqo_repack_q4_0_4x4(const uint8_t *legacy, uint8_t *tiles, int rows, int cols) {
    if (rows % 4 != 0 || cols % 32 != 0) return -1;
    int nb = cols / 32;
    size_t row_stride = (size_t)nb * 18;
    for (int g = 0; g < rows / 4; g++) {
        const uint8_t *src = legacy + (size_t)g * 4 * row_stride;
        for (int b = 0; b < nb; b++) {
            uint8_t *out = tiles + ((size_t)g * nb + b) * 72;
            for (int r = 0; r < 4; r++) memcpy(out + 2 * r, src + r * row_stride + (size_t)b * 18, 2);
            for (int c = 0; c < 16; c++)
                for (int i = 0; i < 4; i++)
                    out[8 + 4 * c + i] =
                        (uint8_t)(src[(c & 3) * row_stride + (size_t)b * 18 + 2 + (c >> 2) * 4 + i] ^ 0x88u);
        }
    }
    return 0;
}

int kqo_unpack_4x4_to_q4_0(const uint8_t *tiles, uint8_t *legacy, int rows, int cols) {
    if (rows % 4 != 0 || cols % 32 != 0) return -1;
    int nb = cols / 32;
    size_t row_stride = (size_t)nb * 18;
    for (int g = 0; g < rows / 4; g++) {
        uint8_t *dst = legacy + (size_t)g * 4 * row_stride;
        for (int b = 0; b < nb; b++) {
            const uint8_t *t = tiles + ((size_t)g * nb + b) * 72;
            for (int r = 0; r < 4; r++) memcpy(dst + r * row_stride + (size_t)b * 18, t + 2 * r, 2);
            for (int c = 0; c < 16; c++)
                for (int i = 0; i < 4; i++)
                    dst[(c & 3) * row_stride + (size_t)b * 18 + 2 + (c >> 2) * 4 + i] =
                        (uint8_t)(t[8 + 4 * c + i] ^ 0x88u);
        }
    }
    return 0;
}

/* Element e (0..31) of row r (0..3) in one tile, as the signed weight n-8 in [-8, 7]:
 * byte j = e & 15 sits at 8 + (j>>2)*16 + r*4 + (j&3); low nibble for e < 16, high otherwise;
 * the stored nibble is n^8, i.e. the 4-bit two's complement of n-8 (layout doc
 * vllm_safetensors.c:4121-4132, MoE accessor vq4x4_w :11000-11011). */
int kqo_tile_weight(const uint8_t *tile, int r, int e) {
    int j = e & 15;
    uint8_t byte = tile[8 + (j >> 2) * 16 + r * 4 + (j & 3)];
    int nib = (e < 16) ? (byte & 15) : (byte >> 4);
    return ((nib ^ 8) & 15) - 8;
}

/* ---------------------------------------------------------------- activation quantizer */

/* quantize_row_q8_0_act (vllm_safetensors.c:7893-7920; NEON twin q8q32_block_neon :7858-7883):
 *   amax = max(1e-10f, max|x|); d = fl(amax/127); q = clamp((int)fl(fl(x/d) + 0.5f), -127, 127)
 * (int) truncates toward zero, so -amax maps to -126. True IEEE division, never a reciprocal.
 * Pinned against the reference quantizer built in oracle/_ref and by closed-form special
 * cases (all-zero block, +-amax, .5 ties, saturation) in tests/test_oracle_quant.py. */
void kqo_quantize_row_q8_0_act(const float *x, int8_t *q, float *d, int cols) {
    int nb = cols / 32;
    for (int b = 0; b < nb; b++) {
        const float *xb = x + (size_t)b * 32;
        float amax = 1e-10f;
        for (int i = 0; i < 32; i++) {
            float av = fabsf(xb[i]);
            if (av > amax) amax = av;
        }
        float scale = amax / 127.0f;
        d[b] = scale;
        for (int i = 0; i < 32; i++) {
            int v = (int)(xb[i] / scale + 0.5f);
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            q[(size_t)b * 32 + i] = (int8_t)v;
        }
    }
}

void kqo_quantize_rows(const float *x, int8_t *q, float *d, int n_batch, int cols) {
    int nb = cols / 32;
    for (int t = 0; t < n_batch; t++)
        kqo_quantize_row_q8_0_act(x + (size_t)t * cols, q + (size_t)t * cols, d + (size_t)t * nb, cols);
}

/* ---------------------------------------------------------------- integer block sums */

/* S_lo = sum_{e<16}(n_e-8) q_e, S_hi = sum_{e>=16}: what the sdot lanes produce before the
 * exact /16 (vllm_safetensors.c:4133-4151, :4190-4216). Pinned by brute force through
 * kqo_tile_weight on tiny inputs and the int32 bound |S| <= 32*8*127. */
static void tile_sums(const uint8_t *tile, int r, const int8_t *q, int32_t *lo, int32_t *hi) {
    int32_t a = 0, c = 0;
    for (int e = 0; e < 16; e++) a += kqo_tile_weight(tile, r, e) * (int32_t)q[e];
    for (int e = 16; e < 32; e++) c += kqo_tile_weight(tile, r, e) * (int32_t)q[e];
    *lo = a;
    *hi = c;
}

void kqo_block_sums(const uint8_t *w, const int8_t *xq, int rows, int cols, int n_batch,
                    int32_t *s_lo, int32_t *s_hi) {
    int nb = cols / 32;
    for (int t = 0; t < n_batch; t++)
        for (int n = 0; n < rows; n++)
            for (int b = 0; b < nb; b++) {
                const uint8_t *tile = w + ((size_t)(n >> 2) * nb + b) * 72;
                size_t o = ((size_t)t * rows + n) * nb + b;
                tile_sums(tile, n & 3, xq + (size_t)t * cols + (size_t)b * 32, &s_lo[o], &s_hi[o]);
            }
}

/* ---------------------------------------------------------------- fp32 chains */

static int token_chain(int chain, int t, int n_batch) {
    if (chain != KQO_CHAIN_AUTO) return chain;
    if (n_batch > 3 && t < (n_batch & ~3)) return KQO_CHAIN_ASM;
    return KQO_CHAIN_CTILE;
}

static float f16r(float x) { return kqo_f16_to_f32(kqo_f32_to_f16_bits(x)); }

/* One output (token t, row n) under chain c. */
static float chain_out(const uint8_t *w, const int8_t *xq_t, const float *xd_t, int n, int nb,
                       int c) {
    const uint8_t *grp = w + (size_t)(n >> 2) * nb * 72;
    int r = n & 3;
    if (c == KQO_CHAIN_CTILE) {
        float lo = 0.0f, hi = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t *tile = grp + (size_t)b * 72;
            int32_t sl, sh;
            tile_sums(tile, r, xq_t + (size_t)b * 32, &sl, &sh);
            uint16_t h;
            memcpy(&h, tile + 2 * r, 2);
            float s = kqo_f16_to_f32(h) * xd_t[b];
            lo = fmaf((float)sl, s, lo);
            hi = fmaf((float)sh, s, hi);
        }
        return lo + hi;
    }
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *tile = grp + (size_t)b * 72;
        int32_t sl, sh;
        tile_sums(tile, r, xq_t + (size_t)b * 32, &sl, &sh);
        uint16_t h;
        memcpy(&h, tile + 2 * r, 2);
        float xs = (c == KQO_CHAIN_ASM) ? f16r(xd_t[b]) : xd_t[b];
        float s = kqo_f16_to_f32(h) * xs;
        acc = fmaf((float)(sl + sh), s, acc);
    }
    return acc;
}

int kqo_matmul_q(float *out, const int8_t *xq, const float *xd, const float *residual,
                 const uint8_t *w, int rows, int cols, int n_batch, int chain) {
    if (rows <= 0 || rows % 4 || cols <= 0 || cols % 32 || n_batch < 0) return -1;
    int nb = cols / 32;
    for (int t = 0; t < n_batch; t++) {
        int c = token_chain(chain, t, n_batch);
        for (int n = 0; n < rows; n++) {
            float v = chain_out(w, xq + (size_t)t * cols, xd + (size_t)t * nb, n, nb, c);
            if (residual) v = residual[(size_t)t * rows + n] + v;
            out[(size_t)t * rows + n] = v;
        }
    }
    return 0;
}

int kqo_matmul_q_sample(float *out, const int8_t *xq, const float *xd, const float *residual,
                        const uint8_t *w, int rows, int cols, int n_batch, int chain,
                        const int *tok, const int *row, int n_sample) {
    if (rows <= 0 || rows % 4 || cols <= 0 || cols % 32) return -1;
    int nb = cols / 32;
    for (int i = 0; i < n_sample; i++) {
        int t = tok[i], n = row[i];
        if (t < 0 || t >= n_batch || n < 0 || n >= rows) return -1;
        float v = chain_out(w, xq + (size_t)t * cols, xd + (size_t)t * nb, n, nb,
                            token_chain(chain, t, n_batch));
        if (residual) v = residual[(size_t)t * rows + n] + v;
        out[i] = v;
    }
    return 0;
}

int kqo_matmul(float *out, const float *x, const float *residual, const uint8_t *w, int rows,
               int cols, int n_batch, int chain) {
    if (rows <= 0 || rows % 4 || cols <= 0 || cols % 32 || n_batch < 0) return -1;
    int nb = cols / 32;
    int8_t *xq = (int8_t *)malloc((size_t)n_batch * cols + 1);
    float *xd = (float *)malloc(((size_t)n_batch * nb + 1) * sizeof(float));
    if (!xq || !xd) { free(xq); free(xd); return -1; }
    kqo_quantize_rows(x, xq, xd, n_batch, cols);
    int rc = kqo_matmul_q(out, xq, xd, residual, w, rows, cols, n_batch, chain);
    free(xq);
    free(xd);
    return rc;
}

/* ---------------------------------------------------------------- dense SiLU * up */

static float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* exp_neon4 (vllm_safetensors.c:4041-4068), one lane: clamp to [-87, 87]; n = vrndnq(x*log2e)
 * (round to nearest even); r = vfmsq(x, n, ln2) = x - n*ln2 fused; p = Horner over the Taylor
 * coefficients 1/6!, 1/5!, .., 1/2, 1, 1 with vfmaq(c, p, r) = c + p*r fused; result bits =
 * bits(p) + (int(n) << 23). Pinned: exp(0) = 1 exactly, relative error against libm exp below
 * 2.5e-7 over [-87, 87] (a dropped or mis-ordered coefficient is far outside it), and an
 * independent float64 emulation of the instruction sequence (tests/test_oracle_silu.py). */
float kqo_exp_neon(float x) {
    x = fmaxf(x, -87.0f);
    x = fminf(x, 87.0f);
    float n = rintf(x * 1.4426950408889634f);
    float r = fmaf(-n, 0.6931471805599453f, x);
    float p = 0.001388888888888889f;
    p = fmaf(p, r, 0.008333333333333333f);
    p = fmaf(p, r, 0.041666666666666664f);
    p = fmaf(p, r, 0.16666666666666666f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return f32_from_bits(f32_bits(p) + ((uint32_t)(int32_t)n << 23));
}

/* vrecpeq_f32 / FRECPE, single precision, as the ARMv8 Architecture Reference Manual's
 * FPRecipEstimate and RecipEstimate pseudocode define it (no FEAT_RPRES; the RK3588's
 * Cortex-A76/A55 have none), for positive normal inputs below 2^126 - the range of the SiLU
 * denominator 1 + exp_neon4(-g), which lies in [1, 6.1e37]: scaled = 256 + the top 8 fraction
 * bits; a = 2*scaled + 1; b = 2^19 DIV a; r = (b + 1) DIV 2; result = 2^(253 - e - 127) *
 * (1 + (r - 256)/256). Pinned: FRECPE(1.0) = 0.998046875 (the documented value), every
 * estimate within 2^-8 relative of 1/x, monotone in x, exponent symmetry. Returns NaN outside
 * the domain. */
float kqo_frecpe(float x) {
    uint32_t b = f32_bits(x);
    uint32_t e = (b >> 23) & 0xFFu;
    if ((b >> 31) || e == 0 || e >= 253) return NAN;
    int a = 2 * (256 + (int)((b >> 15) & 0xFFu)) + 1;
    int q = (1 << 19) / a;
    uint32_t r = (uint32_t)((q + 1) / 2);
    return f32_from_bits(((253u - e) << 23) | ((r & 0xFFu) << 15));
}

/* One element of vllm_silu_mul_worker's NEON loop (vllm_safetensors.c:10941-10950):
 * ex = exp_neon4(-g); den = ex + 1; rec = FRECPE(den); twice rec = rec * FRECPS(den, rec) with
 * FRECPS(d, r) = 2 - d*r fused (FPRecipStepFused); out = fl(fl(g * rec) * u). */
float kqo_silu_mul_neon(float g, float u) {
    float den = kqo_exp_neon(-g) + 1.0f;
    float rec = kqo_frecpe(den);
    rec = rec * fmaf(-den, rec, 2.0f);
    rec = rec * fmaf(-den, rec, 2.0f);
    return (g * rec) * u;
}

/* fast_silu (vllm_safetensors.c:3685-3696), the worker's scalar tail and its non-NEON body. */
float kqo_fast_silu(float x) {
    if (x <= 0.0f) {
        if (x < -20.0f) return 0.0f;
        float ex = expf(x);
        return x * ex / (1.0f + ex);
    }
    if (x > 20.0f) return x;
    return x / (1.0f + expf(-x));
}

/* vllm_silu_mul_worker over a flat array of n elements, in place, as the parfor of 16-element
 * tasks covers it (:10932-10958, callers :16735, :17233): within every task the first
 * (count & ~3) elements take the NEON form, the rest fast_silu(g) * u. Since tasks start at
 * multiples of 16, that is: element i < (n & ~3) NEON, the last n % 4 elements scalar. */
void kqo_silu_mul_rows(float *g, const float *u, long n) {
    long nv = n & ~3L;
    for (long i = 0; i < nv; i++) g[i] = kqo_silu_mul_neon(g[i], u[i]);
    for (long i = nv; i < n; i++) g[i] = kqo_fast_silu(g[i]) * u[i];
}

/* The dense FFN's second half: av = silu_mul(gate, up) over [n_batch][cols], then
 * out = [residual +] down . av with the chain `chain` (dyn_matvec_q4_q8_fused_down_residual*
 * :8663, :8762 after vllm_silu_mul_worker; dense decode :16756-16767). */
int kqo_matmul_silu(float *out, const float *gate, const float *up, const float *residual,
                    const uint8_t *w, int rows, int cols, int n_batch, int chain) {
    if (rows <= 0 || rows % 4 || cols <= 0 || cols % 32 || n_batch < 0) return -1;
    size_t n = (size_t)n_batch * cols;
    float *av = (float *)malloc((n + 1) * sizeof(float));
    if (!av) return -1;
    memcpy(av, gate, n * sizeof(float));
    kqo_silu_mul_rows(av, up, (long)n);
    int rc = kqo_matmul(out, av, residual, w, rows, cols, n_batch, chain);
    free(av);
    return rc;
}

/* ---------------------------------------------------------------- Q8_0 weights */

/* Legacy Q8_0 encoder, 34-B blocks {f16 d; int8 qs[32]} (vqf_convert/src/quant_kernels.c:64-107):
 * scale = max(1e-10f, max|x|) / 127 (true division), stored as f16 (RNE); qs = round half away
 * from zero of fl(x * fl(1/scale)) (the f32 scale), clamped to [-127, 127]. Pinned byte for byte
 * against the reference's f32_to_q8_0 built in oracle/_ref. */
void kqo_f32_to_q8_0(uint8_t *q8_out, const float *f32_in, int n_elements) {
    int n_blocks = n_elements / 32;
    for (int b = 0; b < n_blocks; b++) {
        const float *xb = f32_in + (size_t)b * 32;
        float amax = 1e-10f;
        for (int i = 0; i < 32; i++) {
            float av = fabsf(xb[i]);
            if (av > amax) amax = av;
        }
        volatile float c127 = 127.0f;
        float scale = amax / c127;
        if (scale < 1e-10f) scale = 1e-10f;
        uint16_t h = kqo_f32_to_f16_bits(scale);
        memcpy(q8_out + (size_t)b * 34, &h, 2);
        int8_t *qs = (int8_t *)(q8_out + (size_t)b * 34 + 2);
        float rscale = 1.0f / scale;
        for (int i = 0; i < 32; i++) {
            volatile float qv = xb[i] * rscale;
            int q = (int)(qv < 0.0f ? qv - 0.5f : qv + 0.5f);
            qs[i] = (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
        }
    }
}

/* Legacy -> tiled Q8_0 (vqf_convert/src/qk_repack.c:51-103): per group of g rows (g = 8: the
 * 272-B block_q8_0x8, VQF_FLAG_Q8_8X8; g = 4: the 136-B block_q8_0x4) and block b: the g row
 * scales (f16, row order), then qs[k*4g + m*4 + i] = row m's element 4k+i (k = 0..7). Pinned byte
 * for byte against the reference's repack_q8_0_8x8_inplace / repack_q8_0_4x4_inplace. */
int kqo_repack_q8_0_tiled(const uint8_t *legacy, uint8_t *tiles, int g, int rows, int cols) {
    if ((g != 8 && g != 4) || rows % g != 0 || cols % 32 != 0) return -1;
    int nb = cols / 32;
    size_t row_stride = (size_t)nb * 34, tb = (size_t)34 * g;
    for (int r0 = 0; r0 < rows; r0 += g) {
        const uint8_t *src = legacy + (size_t)r0 * row_stride;
        for (int b = 0; b < nb; b++) {
            uint8_t *out = tiles + ((size_t)(r0 / g) * nb + b) * tb;
            for (int m = 0; m < g; m++) memcpy(out + 2 * m, src + m * row_stride + (size_t)b * 34, 2);
            for (int k = 0; k < 8; k++)
                for (int m = 0; m < g; m++)
                    memcpy(out + 2 * g + (size_t)k * 4 * g + 4 * m,
                           src + m * row_stride + (size_t)b * 34 + 2 + 4 * k, 4);
        }
    }
    return 0;
}

/* Code of element e (0..31) of (row, block b) in a tiled matrix, and its row scale (f32). */
static int q8_code(const uint8_t *w, int g, int nb, int row, int b, int e) {
    const uint8_t *t = w + ((size_t)(row / g) * nb + b) * (size_t)(34 * g);
    return (int8_t)t[2 * g + (e >> 2) * 4 * g + (row % g) * 4 + (e & 3)];
}
static float q8_scale(const uint8_t *w, int g, int nb, int row, int b) {
    const uint8_t *t = w + ((size_t)(row / g) * nb + b) * (size_t)(34 * g);
    uint16_t h;
    memcpy(&h, t + 2 * (row % g), 2);
    return kqo_f16_to_f32(h);
}

/* Q8_0 matmul from quantized activations, per token the reference's chain (AArch64, weights
 * repacked):
 *   VDOT (KQO_CHAIN_GEMV32; q8x8_dot_rows vllm_safetensors.c:5178-5225, single-token decode
 *     :5410-5421): acc = fma(f32(S), fl(wd * xd), acc), S = the exact int32 block dot;
 *   GEMM (KQO_CHAIN_Q8GEMM; gemm_q8_0_8x8_neon :4973-5050 and its 8x4 tail, batched
 *     n_batch >= 2 :5323-5331, activation scales through repack_q8_0_8x8_act :4937-4965):
 *     acc = fl(acc + fl(fl(wd * f32(f16_rne(xd))) * f32(S))) (vmlaq_f32 is an unfused
 *     multiply-add under the reference's -ffp-contract=off);
 *   AUTO: n_batch == 1 -> VDOT, n_batch >= 2 -> GEMM for every token
 *     (dyn_matvec_q8_*_batched_neon :5977-6001, :6071-6091).
 * out = fl(residual + acc) when fused (:5219-5224, vllm_q8x4_res_worker :4806-4814). g = 8 or 4
 * (tile rows). Pinned by exact cases and planted differences (tests/test_oracle_q8.py). */
int kqo_q8_matmul_q(float *out, const int8_t *xq, const float *xd, const float *residual,
                    const uint8_t *w, int g, int rows, int cols, int n_batch, int chain) {
    if ((g != 8 && g != 4) || rows <= 0 || rows % g || cols <= 0 || cols % 32 || n_batch < 0)
        return -1;
    int nb = cols / 32;
    int gemm = chain == KQO_CHAIN_Q8GEMM || (chain == KQO_CHAIN_AUTO && n_batch >= 2);
    if (!gemm && chain != KQO_CHAIN_GEMV32 && chain != KQO_CHAIN_AUTO) return -1;
    for (int t = 0; t < n_batch; t++) {
        const int8_t *q = xq + (size_t)t * cols;
        for (int n = 0; n < rows; n++) {
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                int32_t s = 0;
                for (int e = 0; e < 32; e++) s += q8_code(w, g, nb, n, b, e) * (int32_t)q[b * 32 + e];
                float wd = q8_scale(w, g, nb, n, b);
                float xs = xd[(size_t)t * nb + b];
                if (gemm) {
                    float sc = wd * kqo_f16_to_f32(kqo_f32_to_f16_bits(xs));
                    acc = acc + sc * (float)s;
                } else {
                    acc = fmaf((float)s, wd * xs, acc);
                }
            }
            float r = residual ? residual[(size_t)t * rows + n] + acc : acc;
            out[(size_t)t * rows + n] = r;
        }
    }
    return 0;
}

int kqo_q8_matmul(float *out, const float *x, const float *residual, const uint8_t *w, int g,
                  int rows, int cols, int n_batch, int chain) {
    if (cols <= 0 || cols % 32 || n_batch < 0) return -1;
    int nb = cols / 32;
    int8_t *xq = (int8_t *)malloc((size_t)n_batch * cols + 1);
    float *xd = (float *)malloc(((size_t)n_batch * nb + 1) * sizeof(float));
    if (!xq || !xd) { free(xq); free(xd); return -1; }
    kqo_quantize_rows(x, xq, xd, n_batch, cols);
    int rc = kqo_q8_matmul_q(out, xq, xd, residual, w, g, rows, cols, n_batch, chain);
    free(xq);
    free(xd);
    return rc;
}

/* ---------------------------------------------------------------- RMSNorm */

/* hsum8_f32 (vllm_safetensors.c:8803-8809): ((v0+v4) + (v1+v5)) + ((v2+v6) + (v3+v7)). */
static float hsum8(const float *v) {
    float lo[4];
    for (int i = 0; i < 4; i++) lo[i] = v[i] + v[4 + i];
    return (lo[0] + lo[1]) + (lo[2] + lo[3]);
}

/* Sum of squares of one row in the reference's two orders:
 *   chunked (dyn_rms_norm :8811-8822, and the batch worker under VLLM_SPEC_VNORM=1 :8854-8861):
 *     ss = serial sum over 8-element chunks of hsum8(x^2), then the d % 8 tail serially;
 *   serial (the batch worker's default, :8862-8863): ss = serial sum of x[i]^2.
 * Every square and every sum is one binary32 rounding (the reference builds with
 * -ffp-contract=off). */
static float rms_ss(const float *x, int d, int chunked) {
    float ss = 0.0f;
    int i = 0;
    if (chunked) {
        int d8 = d & ~7;
        for (; i < d8; i += 8) {
            float v[8];
            for (int k = 0; k < 8; k++) v[k] = x[i + k] * x[i + k];
            ss += hsum8(v);
        }
    }
    for (; i < d; i++) ss += x[i] * x[i];
    return ss;
}

/* out[t] = fl(fl(x[t][i] * rms) * w[i]), rms = fl(1 / fl(sqrt(fl(fl(ss / d) + eps)))), for
 * n_batch rows of d: dyn_rms_norm (:8811-8827, chunked = 1) and dyn_rms_norm_batch's worker
 * (:8849-8867, chunked = 0, or 1 under VLLM_SPEC_VNORM=1). Pinned bit for bit against both
 * reference functions built in oracle/_ref, and by exact cases (tests/test_oracle_rmsnorm.py). */
void kqo_rms_norm(float *out, const float *x, const float *w, int n_batch, int d, float eps,
                  int chunked) {
    for (int t = 0; t < n_batch; t++) {
        const float *xr = x + (size_t)t * d;
        float *orow = out + (size_t)t * d;
        float rms = 1.0f / sqrtf(rms_ss(xr, d, chunked) / (float)d + eps);
        for (int i = 0; i < d; i++) orow[i] = xr[i] * rms * w[i];
    }
}

void kqo_matmul_f64(double *out, const int8_t *xq, const float *xd, const uint8_t *w, int rows,
                    int cols, int n_batch) {
    int nb = cols / 32;
    for (int t = 0; t < n_batch; t++)
        for (int n = 0; n < rows; n++) {
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t *tile = w + ((size_t)(n >> 2) * nb + b) * 72;
                int32_t sl, sh;
                tile_sums(tile, n & 3, xq + (size_t)t * cols + (size_t)b * 32, &sl, &sh);
                uint16_t h;
                memcpy(&h, tile + 2 * (n & 3), 2);
                acc += (double)kqo_f16_to_f32(h) * (double)xd[(size_t)t * nb + b] * (double)(sl + sh);
            }
            out[(size_t)t * rows + n] = acc;
        }
}

/* ---------------------------------------------------------------- MoE */

/* Router logit: serial fp32 dot s = fl(s + fl(w*x)), i ascending (st_moe_ffn_sparse_q4
 * vllm_safetensors.c:12961-12967; the reference build uses -ffp-contract=off). */
void kqo_router_logits(const float *router, const float *x, int ne, int d, float *logits) {
    for (int e = 0; e < ne; e++) {
        const float *rw = router + (size_t)e * d;
        float s = 0.0f;
        for (int i = 0; i < d; i++) s += rw[i] * x[i];
        logits[e] = s;
    }
}

/* Deterministic top-k by insertion, ties -> smaller expert id; softmax over the k selected:
 * p = fl(expf(l - max) * fl(1/sum)), sum accumulated k ascending
 * (vllm_safetensors.c:12968-12984; batched twin :14963-14989). Pinned by closed-form cases
 * (ties, equal logits -> uniform 1/k) and by the reference's own x86 MoE built in oracle/_ref. */
void kqo_moe_route(const float *lg, int ne, int tk, int *sel, float *pr) {
    float sv[64];
    for (int k = 0; k < tk; k++) { sel[k] = -1; sv[k] = -INFINITY; }
    for (int e = 0; e < ne; e++) {
        for (int k = 0; k < tk; k++) {
            if (lg[e] > sv[k] || (lg[e] == sv[k] && (sel[k] < 0 || e < sel[k]))) {
                for (int j = tk - 1; j > k; j--) { sel[j] = sel[j - 1]; sv[j] = sv[j - 1]; }
                sel[k] = e;
                sv[k] = lg[e];
                break;
            }
        }
    }
    float mx = -INFINITY;
    for (int k = 0; k < tk; k++) if (sv[k] > mx) mx = sv[k];
    float sum = 0.0f;
    for (int k = 0; k < tk; k++) { pr[k] = expf(sv[k] - mx); sum += pr[k]; }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int k = 0; k < tk; k++) pr[k] *= inv;
}

/* av = fl(fl(g / fl(1 + expf(-g))) * u)  (vllm_safetensors.c:12671-12675, :14752). The expf
 * bits come from this host's libm; the reference's on-board libm is not reachable here, which
 * is why the down stage is pinned stage-wise (kqo_moe_ffn av_in). */
float kqo_silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

/* V4 tile step for one row: S over all 32 elements, acc = fl(acc + fl(fl(sc*xd) * S))
 * (q4x4_gup_actq_neon :11893-11902, moe_q4_down_group_actq_neon :11947-11963). */
static float v4_row(const uint8_t *tiles, int ntile, int r, const int8_t *q, const float *qd) {
    float acc = 0.0f;
    for (int cb = 0; cb < ntile; cb++) {
        const uint8_t *tile = tiles + (size_t)cb * 72;
        int32_t sl, sh;
        tile_sums(tile, r, q + (size_t)cb * 32, &sl, &sh);
        uint16_t h;
        memcpy(&h, tile + 2 * r, 2);
        float sc = kqo_f16_to_f32(h) * qd[cb];
        acc = acc + sc * (float)(sl + sh);
    }
    return acc;
}

/* Grouped MoE FFN, int8 track (VLLM_ACTQ=1): per (token t, rank j) with expert e = sel:
 *   gate/up rows [e*ef, e*ef+ef) of G/U (4-row groups e*ef/4 ..), x quantized once per token;
 *   av = silu(g)*u, re-quantized per (t, j) with quantize_row_q8_0_act;
 *   down: rows 0..d-1 of D over the column band [e*ef, e*ef+ef) (tiles e*ef/32 .. +ef/32);
 *   y = fl(y + fl(p * acc)) for j = 0..tk-1 ascending from y = 0.
 * (st_moe_ffn_sparse_q4 :12921-13398 with arm_dn_actq_worker :12895-12902; batched
 * st_moe_ffn_sparse_q4_batch_arm :14894-15064 computes the same per (t, j) values.) */
int kqo_moe_ffn(float *Y, const float *X, const int *sel, const float *pr, int T, int tk,
                const uint8_t *G, const uint8_t *U, const uint8_t *D, int ne, int d, int ef,
                float *gate_o, float *up_o, float *av_o, int8_t *avq_o, float *avd_o, float *P_o,
                const float *av_in) {
    if (d <= 0 || d % 32 || ef <= 0 || ef % 32 || ne <= 0 || tk <= 0 || tk > 64) return -1;
    int nbG = d / 32, cbe = ef / 32, ff = ne * ef, nbD = ff / 32;
    size_t ggB = (size_t)nbG * 72, gdB = (size_t)nbD * 72;
    int8_t *xq = (int8_t *)malloc((size_t)d);
    float *xd = (float *)malloc((size_t)nbG * sizeof(float));
    float *gv = (float *)malloc((size_t)ef * sizeof(float));
    float *uv = (float *)malloc((size_t)ef * sizeof(float));
    float *av = (float *)malloc((size_t)ef * sizeof(float));
    int8_t *aq = (int8_t *)malloc((size_t)ef);
    float *ad = (float *)malloc((size_t)cbe * sizeof(float));
    if (!xq || !xd || !gv || !uv || !av || !aq || !ad) {
        free(xq); free(xd); free(gv); free(uv); free(av); free(aq); free(ad);
        return -1;
    }
    for (int t = 0; t < T; t++) {
        float *y = Y + (size_t)t * d;
        for (int i = 0; i < d; i++) y[i] = 0.0f;
        kqo_quantize_row_q8_0_act(X + (size_t)t * d, xq, xd, d);
        for (int j = 0; j < tk; j++) {
            int e = sel[(size_t)t * tk + j];
            size_t sj = (size_t)t * tk + j;
            if (e < 0 || e >= ne) continue;
            for (int n = 0; n < ef; n++) {
                size_t g = (size_t)(e * ef + n) >> 2;
                gv[n] = v4_row(G + g * ggB, nbG, n & 3, xq, xd);
                uv[n] = v4_row(U + g * ggB, nbG, n & 3, xq, xd);
                av[n] = kqo_silu_mul(gv[n], uv[n]);
            }
            if (gate_o) memcpy(gate_o + sj * ef, gv, (size_t)ef * sizeof(float));
            if (up_o) memcpy(up_o + sj * ef, uv, (size_t)ef * sizeof(float));
            if (av_o) memcpy(av_o + sj * ef, av, (size_t)ef * sizeof(float));
            const float *avs = av_in ? av_in + sj * ef : av;
            kqo_quantize_row_q8_0_act(avs, aq, ad, ef);
            if (avq_o) memcpy(avq_o + sj * ef, aq, (size_t)ef);
            if (avd_o) memcpy(avd_o + sj * cbe, ad, (size_t)cbe * sizeof(float));
            float p = pr[sj];
            size_t cb0 = (size_t)e * ef / 32;
            for (int n = 0; n < d; n++) {
                const uint8_t *band = D + (size_t)(n >> 2) * gdB + cb0 * 72;
                float acc = v4_row(band, cbe, n & 3, aq, ad);
                if (P_o) P_o[sj * d + n] = acc;
                y[n] = y[n] + p * acc;
            }
        }
    }
    free(xq); free(xd); free(gv); free(uv); free(av); free(aq); free(ad);
    return 0;
}
