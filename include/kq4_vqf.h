/* kq4_vqf.h - VQF model files as libkq4 reads them: mmap, header and directory validation, and
 * each layer's q4 / q8 weight matrix uploaded to HBM (in the stream layouts the kernels read).
 *
 * Restates the part of kestrel-llm's VQF loader the matmul needs (src/model/vqf.c vqf_load
 * :222-560, format include/model/vqf_format.h): the 448-byte header (or the legacy 432-byte one,
 * told apart by which (data_offset, file_len) pair is consistent with the file size,
 * vqf_header_normalize :160-220), the 64-byte directory entries after it, the FNV-1a checksum
 * trailer of plaintext files (:470-490), and the layout flags VQF_FLAG_Q4_4X4 (q4 tensors) and
 * VQF_FLAG_Q8_8X8 (q8 tensors). Per-layer matrices are stacked as the reference stacks them:
 * layer l of a tensor starts at Q4_BYTES(l * N * K) / Q8_BYTES(l * N * K)
 * (vllm_safetensors.c:2338, :16426). Encrypted files (VQF_FLAG_ENC,
 * SM4-CTR) are refused; signatures (VQF_FLAG_SIGNED) are not verified - both belong to the
 * reference's supply-chain layer, not to the matmul.
 *
 * Return convention: 0 = ok, negative KQ4_E* code (kq4.h) on failure; kq4_last_error() says why.
 */
#ifndef KQ4_VQF_H
#define KQ4_VQF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Projection ids: the reference's VLLM_NPU_PROJ_* (include/npu/vllm_npu.h:111-118), which also
 * form its weight-cache keys wkey = layer << 32 | proj. */
#define KQ4_PROJ_Q 0
#define KQ4_PROJ_K 1
#define KQ4_PROJ_V 2
#define KQ4_PROJ_O 3
#define KQ4_PROJ_GATE 4
#define KQ4_PROJ_UP 5
#define KQ4_PROJ_DOWN 6
#define KQ4_PROJ_LM 7

/* VQF flags (include/model/vqf_format.h:30-41) */
#define KQ4_VQF_FLAG_Q8_8X8 (1u << 0)
#define KQ4_VQF_FLAG_Q4_4X4 (1u << 1)
#define KQ4_VQF_FLAG_ENC (1u << 7)
#define KQ4_VQF_FLAG_SIGNED (1u << 8)
#define KQ4_VQF_FLAG_MOE (1u << 9)

typedef struct {
    uint32_t version, flags, n_tensors;
    uint32_t dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size;
    float rope_theta, norm_eps;
    uint32_t n_experts, moe_ffn, top_k; /* MoE (0 for dense files and legacy headers) */
    uint64_t data_offset, file_len;     /* file_len excludes the trailer (8 B FNV, 32 B HMAC) */
    int legacy_header;                  /* 1: the 41-field VQFArch header was normalised */
} kq4_vqf_info;

typedef struct kq4_vqf kq4_vqf;

/* Validates a header and its directory held in buf (buf_len bytes; 4096 covers both) for a
 * file of file_size bytes, as vqf_load does before mounting anything. */
int kq4_vqf_parse_header(const uint8_t *buf, size_t buf_len, uint64_t file_size,
                         kq4_vqf_info *info);

/* mmaps and validates a VQF file; verify_checksum = 1 also checks the FNV-1a trailer over the
 * directory and the data region (the reference's VLLM_VQF_CHECK=1). */
int kq4_vqf_open(const char *path, int verify_checksum, kq4_vqf **out);
void kq4_vqf_close(kq4_vqf *v);
const kq4_vqf_info *kq4_vqf_get_info(const kq4_vqf *v);

/* Directory entry i: name (NUL-terminated, <= 31 chars), qtype (VQF_QT_*), the diagnostic
 * geometry rows x cols, and where its bytes are in the mapped file. */
int kq4_vqf_entry(const kq4_vqf *v, int i, char name[32], uint32_t *qtype, uint32_t *rows,
                  uint32_t *cols, const uint8_t **data, uint64_t *bytes);
/* The entry called name, or KQ4_EINVAL when there is none. */
int kq4_vqf_find(const kq4_vqf *v, const char *name, const uint8_t **data, uint64_t *bytes);

/* Layer `layer` of the q4 matrix of projection proj (KQ4_PROJ_*): a pointer into the mapped
 * file to its VQF 4x4 tiles and its shape (N rows x K cols from the header's arch:
 * Q n_heads*head_dim x dim, K/V n_kv_heads*head_dim x dim, O dim x n_heads*head_dim, gate/up
 * ffn_dim x dim, down dim x ffn_dim, LM vocab x dim with layer 0). */
int kq4_vqf_q4_matrix(const kq4_vqf *v, int proj, int layer, const uint8_t **w4x4, int *rows,
                      int *cols);

/* The q4 matrix's stream-layout copy written to dst (device memory,
 * kq4_weights_stream_bytes(rows, cols) bytes, 16-byte aligned): what every kq4_*_dev call
 * takes as weights. Synchronous with respect to the host bytes. */
int kq4_vqf_prepare_dev(const kq4_vqf *v, int proj, int layer, uint8_t *dst, void *stream);

/* Uploads the q4 matrix into the host-pointer API's weight cache under the reference's key
 * wkey = layer << 32 | proj (st_npu_gw_get vllm_safetensors.c:2780-2800); returns 0 or
 * KQ4_E*. */
int kq4_vqf_upload(const kq4_vqf *v, int proj, int layer, uint64_t *wkey_out);

/* Layer `layer` of the Q8_0 matrix of projection proj (tensors q8_q .. q8_lm of dual / q8 VQF
 * files, stacked at Q8_BYTES(l * N * K), vqf.c:930): its tiles and shape as above, and g, the
 * tile rows: 8 (block_q8_0x8) when the file carries VQF_FLAG_Q8_8X8, else 4 (block_q8_0x4, the
 * reference's other repacked layout). */
int kq4_vqf_q8_matrix(const kq4_vqf *v, int proj, int layer, const uint8_t **w_tiles, int *rows,
                      int *cols, int *g);

/* The q8 matrix's stream-layout copy written to dst (kq4_q8_weights_stream_bytes(rows, cols)
 * bytes, 16-byte aligned): what the kq4_q8_*_dev calls take as weights. */
int kq4_vqf_prepare_q8_dev(const kq4_vqf *v, int proj, int layer, uint8_t *dst, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KQ4_VQF_H */
