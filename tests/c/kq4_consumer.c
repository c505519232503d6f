/* kq4_consumer.c - a C11 program that uses libkq4 the way kestrel-llm's engine would: it includes
 * include/kq4_ops.h, links -lkq4 and calls every wrapper with the argument lists of the reference
 * functions they replace (src/model/vllm_safetensors.c:8628-8786 for the q4 family, :8509-8610
 * for Q8_0, st_moe_ffn_sparse_q4 :12921 and its batch twin :14426). Built by
 * tests/test_c_consumer.py with the reference's C dialect (-std=gnu11 -D_GNU_SOURCE) and
 * -Wall -Wextra -Werror.
 *
 *   kq4_consumer DIR
 *
 * reads its inputs from raw files in DIR (the test writes them from tests/golden/ fixtures) and
 * writes each wrapper's output there as <name>.out; exits 0 when every wrapper returned 1. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kq4.h"
#include "kq4_ops.h"

enum { ROWS = 12, COLS = 96, NB = 5, ROWS8 = 16 };
enum { MOE_D = 64, MOE_NE = 8, MOE_TK = 2, MOE_EF = 32, MOE_T = 3 };

static const char *g_dir;
static int g_fail;

static void *load(const char *name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", g_dir, name);
    FILE *f = fopen(path, "rb");
    void *p = malloc(bytes);
    if (!f || !p || fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "cannot read %zu bytes of %s\n", bytes, path);
        exit(2);
    }
    fclose(f);
    return p;
}

static void save(const char *name, const float *p, size_t n) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s.out", g_dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, sizeof(float), n, f) != n) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

/* Each wrapper returns 1 = done on the GPU, 0 = not done (the engine would run its CPU body). */
static void check(const char *name, int done) {
    if (done != 1) {
        fprintf(stderr, "%s not done: %s\n", name, kq4_last_error());
        g_fail++;
    }
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s DIR\n", argv[0]);
        return 2;
    }
    g_dir = argv[1];
    const uint8_t *w = load("w.bin", ROWS / 4 * (COLS / 32) * 72);
    const uint8_t *w8 = load("w8.bin", ROWS8 * (COLS / 32) * 34);
    const float *x = load("x.bin", sizeof(float) * NB * COLS);
    const float *up = load("up.bin", sizeof(float) * NB * COLS);
    const float *res = load("res.bin", sizeof(float) * NB * ROWS);
    const float *res8 = load("res8.bin", sizeof(float) * NB * ROWS8);
    kq4_moe_layer L;
    L.router = load("router.bin", sizeof(float) * MOE_NE * MOE_D);
    L.G = load("G.bin", MOE_NE * MOE_EF / 4 * (MOE_D / 32) * 72);
    L.U = load("U.bin", MOE_NE * MOE_EF / 4 * (MOE_D / 32) * 72);
    L.D = load("D.bin", MOE_D / 4 * (MOE_NE * MOE_EF / 32) * 72);
    L.n_experts = MOE_NE;
    L.top_k = MOE_TK;
    L.dim = MOE_D;
    L.ef = MOE_EF;
    const float *X = load("X.bin", sizeof(float) * MOE_T * MOE_D);

    if (kq4_init(0) != KQ4_OK) {
        fprintf(stderr, "kq4_init: %s\n", kq4_last_error());
        return 2;
    }
    float a[NB * ROWS8], b[NB * ROWS8], c[NB * ROWS8];

    /* q4, one token (decode) */
    check("dyn_matvec_q4_q8", kq4_dyn_matvec_q4_q8(a, w, x, ROWS, COLS));
    save("mv", a, ROWS);
    check("fused_gate_up", kq4_dyn_matvec_q4_q8_fused_gate_up(a, b, w, w, x, ROWS, COLS));
    save("gu_gate", a, ROWS);
    save("gu_up", b, ROWS);
    check("fused_qkv", kq4_dyn_matvec_q4_q8_fused_qkv(a, b, c, w, w, w, x, ROWS, ROWS, COLS));
    save("qkv_q", a, ROWS);
    save("qkv_v", c, ROWS);
    check("fused_o_residual", kq4_dyn_matvec_q4_q8_fused_o_residual(a, res, w, x, ROWS, COLS));
    save("o_res", a, ROWS);
    check("fused_down_residual",
          kq4_dyn_matvec_q4_q8_fused_down_residual(a, res, w, x, ROWS, COLS));
    save("down_res", a, ROWS);
    check("silu_mul_down_residual", kq4_silu_mul_down_residual(a, res, w, x, up, ROWS, COLS));
    save("silu_down_res", a, ROWS);

    /* q4, batched (NB tokens; the x8_* prefill copies are unused, NULL as the engine may pass) */
    check("fused_qkv_batched", kq4_dyn_matvec_q4_q8_fused_qkv_batched(
                                   a, b, c, w, w, w, x, ROWS, ROWS, COLS, NB, NULL, NULL, NULL));
    save("qkv_b_q", a, NB * ROWS);
    save("qkv_b_k", b, NB * ROWS);
    check("fused_o_residual_batched",
          kq4_dyn_matvec_q4_q8_fused_o_residual_batched(a, res, w, x, ROWS, COLS, NB, NULL));
    save("o_res_b", a, NB * ROWS);
    check("fused_gate_up_batched", kq4_dyn_matvec_q4_q8_fused_gate_up_batched(
                                       a, b, w, w, x, ROWS, COLS, NB, NULL, NULL));
    save("gu_b_up", b, NB * ROWS);
    check("fused_down_residual_batched",
          kq4_dyn_matvec_q4_q8_fused_down_residual_batched(a, res, w, x, ROWS, COLS, NB, NULL));
    save("down_res_b", a, NB * ROWS);
    check("silu_mul_down_residual_batched",
          kq4_silu_mul_down_residual_batched(a, res, w, x, up, ROWS, COLS, NB));
    save("silu_down_res_b", a, NB * ROWS);

    /* Q8_0 (8x8 tiles: ROWS8 % 8 == 0) */
    check("dyn_matvec_q8", kq4_dyn_matvec_q8(a, w8, x, ROWS8, COLS));
    save("q8_mv", a, ROWS8);
    check("q8_fused_o_residual", kq4_dyn_matvec_q8_fused_o_residual(a, res8, w8, x, ROWS8, COLS));
    save("q8_o_res", a, ROWS8);
    check("q8_fused_down_residual",
          kq4_dyn_matvec_q8_fused_down_residual(a, res8, w8, x, ROWS8, COLS));
    save("q8_down_res", a, ROWS8);
    check("q8_fused_qkv_batched", kq4_dyn_matvec_q8_fused_qkv_batched(
                                      a, b, c, w8, w8, w8, x, ROWS8, ROWS8, COLS, NB));
    save("q8_qkv_b_q", a, NB * ROWS8);
    check("q8_fused_o_residual_batched",
          kq4_dyn_matvec_q8_fused_o_residual_batched(a, res8, w8, x, ROWS8, COLS, NB));
    save("q8_o_res_b", a, NB * ROWS8);
    check("q8_fused_gate_up_batched",
          kq4_dyn_matvec_q8_fused_gate_up_batched(a, b, w8, w8, x, ROWS8, COLS, NB));
    save("q8_gu_b_gate", a, NB * ROWS8);
    check("q8_fused_down_residual_batched",
          kq4_dyn_matvec_q8_fused_down_residual_batched(a, res8, w8, x, ROWS8, COLS, NB));
    save("q8_down_res_b", a, NB * ROWS8);

    /* MoE: one token, then the batch */
    float y[MOE_T * MOE_D];
    check("st_moe_ffn_sparse_q4", kq4_st_moe_ffn_sparse_q4(&L, X, y));
    save("moe_1", y, MOE_D);
    check("st_moe_ffn_sparse_q4_batch", kq4_st_moe_ffn_sparse_q4_batch(&L, MOE_T, X, y));
    save("moe_b", y, MOE_T * MOE_D);

    kq4_shutdown();
    printf("kq4_consumer: %d wrapper(s) not done\n", g_fail);
    return g_fail ? 1 : 0;
}
