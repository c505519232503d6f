/* kq4_vqf.c - VQF files for libkq4 (include/kq4_vqf.h): mmap, header/directory validation as
 * kestrel-llm's vqf_load does it (src/model/vqf.c:105-420), and per-layer q4 matrices handed to
 * the device. The on-disk structures are read field by field at their fixed offsets
 * (include/model/vqf_format.h: VQFHeader 448 B, VQFHeaderLegacy 432 B, VQFTensor 64 B). */
#define _GNU_SOURCE
#include "kq4_vqf.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "kq4.h"
#include "kq4_err.h"

#define VQF_MAGIC 0x57465146u   /* "VQFW" */
#define VQF_ALIGN 64
#define VQF_QT_Q4_0 0x03
#define HDR_BYTES 448           /* sizeof(VQFHeader); the directory starts here */
#define ENT_BYTES 64            /* sizeof(VQFTensor) */
/* field offsets in the header: the 45-field VQFArch (180 B) from byte 16, then data_offset,
 * file_len; the legacy 41-field arch is 164 B, so its data_offset/file_len sit 16 B earlier */
#define OFF_ARCH 16
#define OFF_DOFF_NEW 200
#define OFF_FLEN_NEW 208
#define OFF_DOFF_OLD 184
#define OFF_FLEN_OLD 192
#define ARCH_U32(i) (OFF_ARCH + 4 * (i))   /* i-th 4-byte field of VQFArch */

struct kq4_vqf {
    const uint8_t *base;
    size_t len;
    kq4_vqf_info info;
};

static uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }
static float rdf(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

/* vqf_cand_valid (vqf.c:147-158): a (data_offset, file_len) pair consistent with the file. */
static int cand_valid(uint64_t d_off, uint64_t f_len, uint64_t file_size, uint64_t tag_len,
                      uint64_t dir_end) {
    if (d_off == 0 || f_len == 0) return 0;
    if (d_off & (VQF_ALIGN - 1)) return 0;
    if (d_off < dir_end || d_off >= file_size) return 0;
    if (f_len + tag_len != file_size) return 0;
    return f_len > d_off;
}

/* Bytes of a tensor of n elements of type qt (the converter's vq_bytes). */
static uint64_t qt_bytes(uint32_t qt, uint64_t n) {
    switch (qt) {
    case 0x01: return n * 4;                 /* F32 */
    case 0x02: return (n + 31) / 32 * 34;    /* Q8_0 */
    case 0x03: return (n + 31) / 32 * 18;    /* Q4_0 */
    case 0x05: return n * 2;                 /* F16 */
    default: return 0;
    }
}

int kq4_vqf_parse_header(const uint8_t *buf, size_t buf_len, uint64_t file_size,
                         kq4_vqf_info *info) {
    if (!buf || !info) return kq4_fail(KQ4_EINVAL, "vqf: null argument");
    if (buf_len < HDR_BYTES + ENT_BYTES || file_size < HDR_BYTES + ENT_BYTES)
        return kq4_fail(KQ4_EIO, "vqf: file too small");
    memset(info, 0, sizeof(*info));
    if (rd32(buf) != VQF_MAGIC) return kq4_fail(KQ4_EIO, "vqf: bad magic 0x%08x", rd32(buf));
    info->version = rd32(buf + 4);
    if (info->version != 2 && info->version != 3)
        return kq4_fail(KQ4_EIO, "vqf: version %u unsupported (need 2 or 3)", info->version);
    info->flags = rd32(buf + 8);
    info->n_tensors = rd32(buf + 12);
    info->dim = rd32(buf + ARCH_U32(0));
    info->n_layers = rd32(buf + ARCH_U32(1));
    info->n_heads = rd32(buf + ARCH_U32(2));
    info->n_kv_heads = rd32(buf + ARCH_U32(3));
    info->head_dim = rd32(buf + ARCH_U32(4));
    info->ffn_dim = rd32(buf + ARCH_U32(5));
    info->vocab_size = rd32(buf + ARCH_U32(6));
    info->rope_theta = rdf(buf + ARCH_U32(8));
    info->norm_eps = rdf(buf + ARCH_U32(9));
    /* vqf_header_normalize (vqf.c:160-220): geometry gate, then the one consistent layout */
    if (!(info->dim && info->n_layers && info->n_heads && info->head_dim && info->ffn_dim &&
          info->vocab_size))
        return kq4_fail(KQ4_EIO, "vqf: arch geometry invalid (dim=%u layers=%u heads=%u "
                        "head_dim=%u ffn=%u vocab=%u)", info->dim, info->n_layers,
                        info->n_heads, info->head_dim, info->ffn_dim, info->vocab_size);
    const uint64_t tag = (info->flags & KQ4_VQF_FLAG_ENC) ? 32 : 8;
    const uint64_t dir_end = HDR_BYTES + (uint64_t)info->n_tensors * ENT_BYTES;
    const uint64_t dn = rd64(buf + OFF_DOFF_NEW), fn = rd64(buf + OFF_FLEN_NEW);
    const uint64_t dl = rd64(buf + OFF_DOFF_OLD), fl = rd64(buf + OFF_FLEN_OLD);
    const int ok_new = cand_valid(dn, fn, file_size, tag, dir_end);
    const int ok_old = cand_valid(dl, fl, file_size, tag, dir_end);
    if (ok_new && !ok_old) {
        info->data_offset = dn;
        info->file_len = fn;
        info->n_experts = rd32(buf + ARCH_U32(41));
        info->moe_ffn = rd32(buf + ARCH_U32(42));
        info->top_k = rd32(buf + ARCH_U32(43));
    } else if (ok_old && !ok_new) {
        if (info->flags & (KQ4_VQF_FLAG_ENC | KQ4_VQF_FLAG_SIGNED))
            return kq4_fail(KQ4_EIO, "vqf: legacy 41-field header with ENC/SIGNED unsupported");
        info->data_offset = dl;
        info->file_len = fl;
        info->legacy_header = 1;   /* the MoE tail does not exist in this layout: zero */
    } else {
        return kq4_fail(KQ4_EIO, "vqf: header layout undetermined (new %llu/%llu valid=%d, "
                        "legacy %llu/%llu valid=%d, file %llu)", (unsigned long long)dn,
                        (unsigned long long)fn, ok_new, (unsigned long long)dl,
                        (unsigned long long)fl, ok_old, (unsigned long long)file_size);
    }
    if (buf_len < dir_end) return kq4_fail(KQ4_EINVAL, "vqf: directory not in the buffer");
    /* every entry inside the data region, its size what its type and geometry give */
    for (uint32_t i = 0; i < info->n_tensors; i++) {
        const uint8_t *e = buf + HDR_BYTES + (size_t)i * ENT_BYTES;
        const uint32_t qt = rd32(e + 32), rows = rd32(e + 36), cols = rd32(e + 40);
        const uint64_t off = rd64(e + 48), bytes = rd64(e + 56);
        if (!memchr(e, 0, 32)) return kq4_fail(KQ4_EIO, "vqf: entry %u name not terminated", i);
        if (off < info->data_offset || off > info->file_len || bytes > info->file_len - off)
            return kq4_fail(KQ4_EIO, "vqf: entry %u (%.32s) outside the data region", i, e);
        const uint64_t want = qt_bytes(qt, (uint64_t)rows * cols);
        if (want && want != bytes)
            return kq4_fail(KQ4_EIO, "vqf: entry %u (%.32s) has %llu bytes, %llu expected", i, e,
                            (unsigned long long)bytes, (unsigned long long)want);
    }
    return KQ4_OK;
}

/* FNV-1a 64 (vqf_fnv_update vqf.c:62-69). */
static uint64_t fnv(uint64_t h, const uint8_t *p, size_t n) {
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

int kq4_vqf_open(const char *path, int verify_checksum, kq4_vqf **out) {
    if (!path || !out) return kq4_fail(KQ4_EINVAL, "vqf: null argument");
    *out = NULL;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return kq4_fail(KQ4_EIO, "vqf: open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < HDR_BYTES + ENT_BYTES) {
        close(fd);
        return kq4_fail(KQ4_EIO, "vqf: %s: too small or unreadable", path);
    }
    const size_t len = (size_t)st.st_size;
    void *m = mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return kq4_fail(KQ4_EIO, "vqf: mmap %s: %s", path, strerror(errno));
    kq4_vqf *v = (kq4_vqf *)calloc(1, sizeof(*v));
    if (!v) {
        munmap(m, len);
        return kq4_fail(KQ4_ENOMEM, "vqf: out of host memory");
    }
    v->base = (const uint8_t *)m;
    v->len = len;
    int rc = kq4_vqf_parse_header(v->base, len, len, &v->info);
    if (!rc && (v->info.flags & KQ4_VQF_FLAG_ENC))
        rc = kq4_fail(KQ4_EIO, "vqf: %s is encrypted (VQF-Enc); decrypt it first", path);
    if (!rc && verify_checksum) {
        /* the trailer covers the directory and the data region (vqf.c:470-490); 0 = none */
        uint64_t want;
        memcpy(&want, v->base + len - 8, 8);
        if (want != 0) {
            uint64_t h = fnv(0xcbf29ce484222325ull, v->base + HDR_BYTES,
                             (size_t)v->info.n_tensors * ENT_BYTES);
            h = fnv(h, v->base + v->info.data_offset,
                    (size_t)(v->info.file_len - v->info.data_offset));
            if (h != want) rc = kq4_fail(KQ4_EIO, "vqf: %s: checksum mismatch", path);
        }
    }
    if (rc) {
        kq4_vqf_close(v);
        return rc;
    }
    *out = v;
    return KQ4_OK;
}

void kq4_vqf_close(kq4_vqf *v) {
    if (!v) return;
    if (v->base) munmap((void *)v->base, v->len);
    free(v);
}

const kq4_vqf_info *kq4_vqf_get_info(const kq4_vqf *v) { return v ? &v->info : NULL; }

int kq4_vqf_entry(const kq4_vqf *v, int i, char name[32], uint32_t *qtype, uint32_t *rows,
                  uint32_t *cols, const uint8_t **data, uint64_t *bytes) {
    if (!v || i < 0 || (uint32_t)i >= v->info.n_tensors)
        return kq4_fail(KQ4_EINVAL, "vqf: entry %d out of range", i);
    const uint8_t *e = v->base + HDR_BYTES + (size_t)i * ENT_BYTES;
    if (name) memcpy(name, e, 32);
    if (qtype) *qtype = rd32(e + 32);
    if (rows) *rows = rd32(e + 36);
    if (cols) *cols = rd32(e + 40);
    if (data) *data = v->base + rd64(e + 48);
    if (bytes) *bytes = rd64(e + 56);
    return KQ4_OK;
}

int kq4_vqf_find(const kq4_vqf *v, const char *name, const uint8_t **data, uint64_t *bytes) {
    if (!v || !name) return kq4_fail(KQ4_EINVAL, "vqf: null argument");
    for (uint32_t i = 0; i < v->info.n_tensors; i++) {
        const uint8_t *e = v->base + HDR_BYTES + (size_t)i * ENT_BYTES;
        if (strncmp((const char *)e, name, 32) == 0)
            return kq4_vqf_entry(v, (int)i, NULL, NULL, NULL, NULL, data, bytes);
    }
    return kq4_fail(KQ4_EINVAL, "vqf: no tensor %s", name);
}

static const char *const q4_names[8] = {"q4_q", "q4_k", "q4_v", "q4_o",
                                        "q4_gate", "q4_up", "q4_down", "q4_lm"};
static const char *const q8_names[8] = {"q8_q", "q8_k", "q8_v", "q8_o",
                                        "q8_gate", "q8_up", "q8_down", "q8_lm"};

/* Layer `layer` of projection proj: N x K from the arch, the tensor's bytes at
 * layer * N*K/32*bpb (bpb = 18 for Q4_0, 34 for Q8_0). */
static int layer_matrix(const kq4_vqf *v, const char *const *names, uint64_t bpb, int proj,
                        int layer, const uint8_t **w, int *rows, int *cols) {
    if (!v || proj < KQ4_PROJ_Q || proj > KQ4_PROJ_LM)
        return kq4_fail(KQ4_EINVAL, "vqf: projection %d", proj);
    const kq4_vqf_info *a = &v->info;
    if (layer < 0 || (proj == KQ4_PROJ_LM ? layer != 0 : (uint32_t)layer >= a->n_layers))
        return kq4_fail(KQ4_EINVAL, "vqf: layer %d of %u", layer, a->n_layers);
    const uint64_t q_out = (uint64_t)a->n_heads * a->head_dim;
    const uint64_t kv_out = (uint64_t)a->n_kv_heads * a->head_dim;
    uint64_t n = 0, k = 0;
    switch (proj) {
    case KQ4_PROJ_Q: n = q_out; k = a->dim; break;
    case KQ4_PROJ_K: case KQ4_PROJ_V: n = kv_out; k = a->dim; break;
    case KQ4_PROJ_O: n = a->dim; k = q_out; break;
    case KQ4_PROJ_GATE: case KQ4_PROJ_UP: n = a->ffn_dim; k = a->dim; break;
    case KQ4_PROJ_DOWN: n = a->dim; k = a->ffn_dim; break;
    default: n = a->vocab_size; k = a->dim; break;
    }
    if (n == 0 || n % 4 || k == 0 || k % 32 || n > 0x7fffffff || k > 0x7fffffff)
        return kq4_fail(KQ4_EIO, "vqf: %s is %llux%llu (need rows %% 4 == 0, cols %% 32 == 0)",
                        names[proj], (unsigned long long)n, (unsigned long long)k);
    const uint8_t *data;
    uint64_t bytes;
    int rc = kq4_vqf_find(v, names[proj], &data, &bytes);
    if (rc) return rc;
    /* Q4_BYTES / Q8_BYTES (N*K): layer l at l * per. n, k < 2^31, so per < 2^63; the bound is
     * checked by division, as (layer + 1) * per can wrap past 2^64 for a crafted header. */
    const uint64_t per = n * k / 32 * bpb;
    if ((uint64_t)layer >= bytes / per)
        return kq4_fail(KQ4_EIO, "vqf: %s holds %llu bytes, too few for layer %d of %llu bytes",
                        names[proj], (unsigned long long)bytes, layer, (unsigned long long)per);
    if (w) *w = data + (uint64_t)layer * per;
    if (rows) *rows = (int)n;
    if (cols) *cols = (int)k;
    return KQ4_OK;
}

int kq4_vqf_q4_matrix(const kq4_vqf *v, int proj, int layer, const uint8_t **w4x4, int *rows,
                      int *cols) {
    if (v && !(v->info.flags & KQ4_VQF_FLAG_Q4_4X4))
        return kq4_fail(KQ4_EIO, "vqf: q4 tensors not in the 4x4 tile layout (flags 0x%x)",
                        v->info.flags);
    return layer_matrix(v, q4_names, 18, proj, layer, w4x4, rows, cols);
}

int kq4_vqf_q8_matrix(const kq4_vqf *v, int proj, int layer, const uint8_t **w_tiles, int *rows,
                      int *cols, int *g) {
    int r = 0, c = 0;
    int rc = layer_matrix(v, q8_names, 34, proj, layer, w_tiles, &r, &c);
    if (rc) return rc;
    const int gg = (v->info.flags & KQ4_VQF_FLAG_Q8_8X8) ? 8 : 4;
    if (r % gg)
        return kq4_fail(KQ4_EIO, "vqf: %s has %d rows, not whole %d-row tiles", q8_names[proj], r,
                        gg);
    if (rows) *rows = r;
    if (cols) *cols = c;
    if (g) *g = gg;
    return KQ4_OK;
}

int kq4_vqf_prepare_q8_dev(const kq4_vqf *v, int proj, int layer, uint8_t *dst, void *stream) {
    const uint8_t *w;
    int rows, cols, g;
    int rc = kq4_vqf_q8_matrix(v, proj, layer, &w, &rows, &cols, &g);
    if (rc) return rc;
    return kq4_q8_weights_prepare_host(dst, w, g, rows, cols, stream);
}

int kq4_vqf_prepare_dev(const kq4_vqf *v, int proj, int layer, uint8_t *dst, void *stream) {
    const uint8_t *w;
    int rows, cols;
    int rc = kq4_vqf_q4_matrix(v, proj, layer, &w, &rows, &cols);
    if (rc) return rc;
    return kq4_weights_prepare_host(dst, w, rows, cols, stream);
}

int kq4_vqf_upload(const kq4_vqf *v, int proj, int layer, uint64_t *wkey_out) {
    const uint8_t *w;
    int rows, cols;
    int rc = kq4_vqf_q4_matrix(v, proj, layer, &w, &rows, &cols);
    if (rc) return rc;
    const uint64_t wkey = ((uint64_t)(uint32_t)layer << 32) | (uint32_t)proj;
    if (!kq4_weights_upload(wkey, w, rows, cols)) return KQ4_EHIP;   /* message already set */
    if (wkey_out) *wkey_out = wkey;
    return KQ4_OK;
}
