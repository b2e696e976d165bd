/*
 * gguf.c -- GGUF v2/v3 container parser feeding the HBM tensor cache.
 *
 * Behaviour follows the reference loader (inference/src/gguf.m:273-518):
 * little-endian header, typed metadata key/values, tensor infos, and a data
 * section that starts at the header end rounded up to `general.alignment`
 * (default 32, gguf.m:323, 511-512).  Only the MoE-relevant metadata is kept.
 * Differences: every read is bounds-checked and a truncated or malformed
 * image is rejected (the reference reads zeros past the end), and the name
 * lookup is a sorted index searched by bisection.
 */
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "orome_moe.h"
#include "orome_internal.h"

#define GGUF_MAGIC 0x46554747u /* "GGUF" little-endian */

enum {
    GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6,
    GT_BOOL = 7, GT_STR = 8, GT_ARR = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12,
};

typedef struct {
    const uint8_t *p;
    size_t n, pos;
    int bad;
} rd_t;

static int rd_need(rd_t *r, size_t k) {
    if (r->bad || k > r->n - r->pos) { r->bad = 1; return 0; }
    return 1;
}
static uint64_t rd_uint(rd_t *r, size_t k) {
    uint64_t v = 0;
    if (!rd_need(r, k)) return 0;
    memcpy(&v, r->p + r->pos, k);  /* little-endian host */
    r->pos += k;
    return v;
}
static double rd_num(rd_t *r, uint32_t t) {
    switch (t) {
        case GT_U8: case GT_BOOL: return (double)(uint8_t)rd_uint(r, 1);
        case GT_I8: return (double)(int8_t)rd_uint(r, 1);
        case GT_U16: return (double)(uint16_t)rd_uint(r, 2);
        case GT_I16: return (double)(int16_t)rd_uint(r, 2);
        case GT_U32: return (double)(uint32_t)rd_uint(r, 4);
        case GT_I32: return (double)(int32_t)rd_uint(r, 4);
        case GT_U64: return (double)rd_uint(r, 8);
        case GT_I64: return (double)(int64_t)rd_uint(r, 8);
        case GT_F32: { uint32_t b = (uint32_t)rd_uint(r, 4); float f; memcpy(&f, &b, 4); return f; }
        case GT_F64: { uint64_t b = rd_uint(r, 8); double f; memcpy(&f, &b, 8); return f; }
    }
    r->bad = 1;
    return 0;
}
/* returns a pointer into the image (not terminated) */
static const char *rd_str(rd_t *r, uint64_t *len) {
    *len = rd_uint(r, 8);
    if (!rd_need(r, *len)) return NULL;
    const char *s = (const char *)r->p + r->pos;
    r->pos += *len;
    return s;
}
static size_t scalar_size(uint32_t t) {
    switch (t) {
        case GT_U8: case GT_I8: case GT_BOOL: return 1;
        case GT_U16: case GT_I16: return 2;
        case GT_U32: case GT_I32: case GT_F32: return 4;
        case GT_U64: case GT_I64: case GT_F64: return 8;
    }
    return 0;
}
static void rd_skip(rd_t *r, uint32_t t, int depth) {
    if (depth > 4) { r->bad = 1; return; }
    if (t == GT_STR) { uint64_t l; rd_str(r, &l); return; }
    if (t == GT_ARR) {
        uint32_t et = (uint32_t)rd_uint(r, 4);
        uint64_t cnt = rd_uint(r, 8);
        size_t ss = scalar_size(et);
        if (ss) {
            if (cnt > (r->n - r->pos) / ss) { r->bad = 1; return; }
            r->pos += cnt * ss;
            return;
        }
        for (uint64_t i = 0; i < cnt && !r->bad; i++) rd_skip(r, et, depth + 1);
        return;
    }
    size_t ss = scalar_size(t);
    if (!ss) { r->bad = 1; return; }
    rd_need(r, ss);
    if (!r->bad) r->pos += ss;
}

static int key_is(const char *k, uint64_t kl, const char *want) {
    size_t wl = strlen(want);
    return kl == wl && memcmp(k, want, wl) == 0;
}

/* ggml block tables (inference/src/gguf.m:64-104) */
static size_t blk_elems(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: return 1;          /* F32 F16 BF16 */
        case 2: case 3: case 6: case 7: case 8: case 9: return 32;  /* Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q8_1 */
        case 10: case 11: case 12: case 13: case 14: case 15: return 256; /* Q2_K..Q8_K */
    }
    return 0;
}
static size_t blk_bytes(uint32_t t) {
    switch (t) {
        case 0: return 4; case 1: return 2; case 30: return 2;
        case 2: return 18; case 3: return 20; case 6: return 22; case 7: return 24;
        case 8: return 34; case 9: return 36;
        case 10: return 84; case 11: return 110; case 12: return 144; case 13: return 176;
        case 14: return 210; case 15: return 292;
    }
    return 0;
}

size_t orome_hip_gguf_tensor_size(const OromeHipGGUFTensorInfo *ti) {
    if (!ti) return 0;
    size_t be = blk_elems(ti->type), bb = blk_bytes(ti->type);
    if (!be || !bb) return 0;
    uint64_t n = 1;
    for (uint32_t d = 0; d < ti->n_dims && d < 4; d++) n *= ti->dims[d];
    return (size_t)(n / be) * bb;
}

const char *orome_hip_ggml_type_name(uint32_t t) {
    switch (t) {
        case 0: return "F32"; case 1: return "F16"; case 30: return "BF16";
        case 2: return "Q4_0"; case 3: return "Q4_1"; case 6: return "Q5_0"; case 7: return "Q5_1";
        case 8: return "Q8_0"; case 9: return "Q8_1"; case 10: return "Q2_K"; case 11: return "Q3_K";
        case 12: return "Q4_K"; case 13: return "Q5_K"; case 14: return "Q6_K"; case 15: return "Q8_K";
    }
    return "UNKNOWN";
}

int orome_hip_format_from_ggml_type(uint32_t t, OromeHipQuantFormat *out) {
    OromeHipQuantFormat f;
    switch (t) {
        case 8: f = OROME_QFMT_GGUF_Q8_0; break;
        case 12: f = OROME_QFMT_GGUF_Q4_K; break;
        case 13: f = OROME_QFMT_GGUF_Q5_K; break;
        case 14: f = OROME_QFMT_GGUF_Q6_K; break;
        case 1: f = OROME_QFMT_F16; break;
        case 30: f = OROME_QFMT_BF16; break;
        case 0: f = OROME_QFMT_F32; break;
        default:
            return orome_fail(OROME_EUNSUPPORTED, "ggml type %u (%s) has no kernel", t,
                              orome_hip_ggml_type_name(t));
    }
    if (out) *out = f;
    return OROME_OK;
}

/* name index: tensor ids sorted by name */
typedef struct {
    uint64_t n;
    uint64_t *ids;
    const OromeHipGGUFTensorInfo *tensors;
} name_index;

static const OromeHipGGUFTensorInfo *g_sort_base;
static int cmp_ids(const void *a, const void *b) {
    return strcmp(g_sort_base[*(const uint64_t *)a].name, g_sort_base[*(const uint64_t *)b].name);
}

OromeHipGGUFTensorInfo *orome_hip_gguf_find_tensor(OromeHipGGUFFile *gf, const char *name) {
    if (!gf || !name || !gf->index) return NULL;
    name_index *ix = (name_index *)gf->index;
    uint64_t lo = 0, hi = ix->n;
    while (lo < hi) {
        uint64_t mid = lo + (hi - lo) / 2;
        int c = strcmp(gf->tensors[ix->ids[mid]].name, name);
        if (c == 0) return &gf->tensors[ix->ids[mid]];
        if (c < 0) lo = mid + 1; else hi = mid;
    }
    return NULL;
}

void orome_hip_gguf_close(OromeHipGGUFFile *gf) {
    if (!gf) return;
    if (gf->tensors) {
        for (uint64_t i = 0; i < gf->num_tensors; i++) free(gf->tensors[i].name);
        free(gf->tensors);
    }
    if (gf->index) {
        free(((name_index *)gf->index)->ids);
        free(gf->index);
    }
    if (gf->owns_map && gf->mmap_base) munmap(gf->mmap_base, gf->file_size);
    if (gf->fd >= 0) close(gf->fd);
    free(gf);
}

static OromeHipGGUFFile *parse(const uint8_t *img, size_t size, OromeHipGGUFFile *gf) {
    rd_t r = {img, size, 0, 0};
    uint32_t magic = (uint32_t)rd_uint(&r, 4);
    if (r.bad || magic != GGUF_MAGIC) {
        orome_fail(OROME_EFORMAT, "gguf: bad magic 0x%08X", magic);
        goto fail;
    }
    uint32_t version = (uint32_t)rd_uint(&r, 4);
    if (version < 2 || version > 3) {
        orome_fail(OROME_EFORMAT, "gguf: unsupported version %u", version);
        goto fail;
    }
    uint64_t n_tensors = rd_uint(&r, 8), n_kv = rd_uint(&r, 8);
    if (r.bad || n_tensors > (1u << 24) || n_kv > (1u << 24)) {
        orome_fail(OROME_EFORMAT, "gguf: implausible counts (%llu tensors, %llu kv)",
                   (unsigned long long)n_tensors, (unsigned long long)n_kv);
        goto fail;
    }
    gf->alignment = 32;
    gf->rms_norm_eps = 1e-6f;
    gf->q4k_layout = OROME_Q4K_LAYOUT_REFERENCE;
    /* pass 1 over the metadata: the architecture prefix may come after the
     * keys that use it, so remember key positions and resolve afterwards */
    size_t kv_start = r.pos;
    for (int pass = 0; pass < 2; pass++) {
        r.pos = kv_start;
        char prefix[40];
        snprintf(prefix, sizeof prefix, "%s.", gf->arch[0] ? gf->arch : "llama");
        size_t pl = strlen(prefix);
        for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
            uint64_t kl;
            const char *k = rd_str(&r, &kl);
            uint32_t t = (uint32_t)rd_uint(&r, 4);
            if (r.bad) break;
            if (pass == 0) {
                if (key_is(k, kl, "general.architecture") && t == GT_STR) {
                    uint64_t vl;
                    const char *v = rd_str(&r, &vl);
                    if (v) {
                        size_t c = vl < sizeof gf->arch - 1 ? vl : sizeof gf->arch - 1;
                        memcpy(gf->arch, v, c);
                        gf->arch[c] = 0;
                    }
                    continue;
                }
                if (key_is(k, kl, "general.alignment") && t != GT_STR && t != GT_ARR) {
                    gf->alignment = (uint32_t)rd_num(&r, t);
                    continue;
                }
                if (key_is(k, kl, OROME_Q4K_LAYOUT_KEY) && t == GT_STR) {
                    uint64_t vl;
                    const char *v = rd_str(&r, &vl);
                    if (v && key_is(v, vl, "ggml")) gf->q4k_layout = OROME_Q4K_LAYOUT_GGML;
                    else if (v && key_is(v, vl, "reference")) gf->q4k_layout = OROME_Q4K_LAYOUT_REFERENCE;
                    else {
                        orome_fail(OROME_EFORMAT, "gguf: unknown %s value", OROME_Q4K_LAYOUT_KEY);
                        goto fail;
                    }
                    continue;
                }
                rd_skip(&r, t, 0);
                continue;
            }
            if (kl > pl && memcmp(k, prefix, pl) == 0 && t != GT_STR && t != GT_ARR) {
                const char *f = k + pl;
                uint64_t fl = kl - pl;
                double v = rd_num(&r, t);
                if (key_is(f, fl, "block_count")) gf->num_layers = (int)v;
                else if (key_is(f, fl, "embedding_length")) gf->hidden_dim = (int)v;
                else if (key_is(f, fl, "expert_count")) gf->num_experts = (int)v;
                else if (key_is(f, fl, "expert_used_count")) gf->num_experts_per_tok = (int)v;
                else if (key_is(f, fl, "expert_feed_forward_length")) gf->moe_intermediate = (int)v;
                else if (key_is(f, fl, "feed_forward_length") && !gf->moe_intermediate)
                    gf->moe_intermediate = (int)v;
                else if (key_is(f, fl, "attention.layer_norm_rms_epsilon")) gf->rms_norm_eps = (float)v;
                continue;
            }
            rd_skip(&r, t, 0);
        }
        if (r.bad) {
            orome_fail(OROME_EFORMAT, "gguf: truncated metadata");
            goto fail;
        }
    }
    if (gf->alignment == 0 || (gf->alignment & (gf->alignment - 1))) {
        orome_fail(OROME_EFORMAT, "gguf: alignment %u is not a power of two", gf->alignment);
        goto fail;
    }
    gf->num_tensors = n_tensors;
    gf->tensors = calloc(n_tensors ? n_tensors : 1, sizeof(OromeHipGGUFTensorInfo));
    if (!gf->tensors) { orome_fail(OROME_ENOMEM, "gguf: out of host memory"); goto fail; }
    for (uint64_t i = 0; i < n_tensors; i++) {
        OromeHipGGUFTensorInfo *ti = &gf->tensors[i];
        uint64_t nl;
        const char *nm = rd_str(&r, &nl);
        ti->n_dims = (uint32_t)rd_uint(&r, 4);
        if (r.bad || !nm || ti->n_dims > 4) {
            orome_fail(OROME_EFORMAT, "gguf: bad tensor info %llu", (unsigned long long)i);
            goto fail;
        }
        ti->name = malloc(nl + 1);
        memcpy(ti->name, nm, nl);
        ti->name[nl] = 0;
        for (uint32_t d = 0; d < ti->n_dims; d++) ti->dims[d] = rd_uint(&r, 8);
        for (uint32_t d = ti->n_dims; d < 4; d++) ti->dims[d] = 1;
        ti->type = (uint32_t)rd_uint(&r, 4);
        ti->offset = rd_uint(&r, 8);
        if (r.bad) { orome_fail(OROME_EFORMAT, "gguf: truncated tensor infos"); goto fail; }
    }
    size_t a = gf->alignment;
    gf->data_offset = (r.pos + a - 1) & ~(a - 1);
    for (uint64_t i = 0; i < n_tensors; i++) {
        OromeHipGGUFTensorInfo *ti = &gf->tensors[i];
        size_t sz = orome_hip_gguf_tensor_size(ti);
        if (gf->data_offset + ti->offset + sz > size) {
            orome_fail(OROME_EFORMAT, "gguf: tensor %s extends past the end of the image", ti->name);
            goto fail;
        }
    }
    name_index *ix = calloc(1, sizeof *ix);
    ix->n = n_tensors;
    ix->ids = malloc(sizeof(uint64_t) * (n_tensors ? n_tensors : 1));
    for (uint64_t i = 0; i < n_tensors; i++) ix->ids[i] = i;
    g_sort_base = gf->tensors;
    qsort(ix->ids, n_tensors, sizeof(uint64_t), cmp_ids);
    gf->index = ix;

    int moe = 0;
    for (uint64_t i = 0; i < n_tensors; i++)
        if (strstr(gf->tensors[i].name, "_exps")) { moe = 1; break; }
    gf->ffn_type = (moe || gf->num_experts > 0) ? OROME_FFN_MOE : OROME_FFN_DENSE;
    if (!gf->moe_intermediate && moe) {
        /* gguf.m:476-488: the gate_exps dimension that is neither H nor E */
        OromeHipGGUFTensorInfo *g = orome_hip_gguf_find_tensor(gf, "blk.0.ffn_gate_exps.weight");
        if (g && g->n_dims >= 2) gf->moe_intermediate = (int)g->dims[1];
    }
    return gf;
fail:
    orome_hip_gguf_close(gf);
    return NULL;
}

OromeHipGGUFFile *orome_hip_gguf_open_memory(const void *data, size_t size) {
    if (!data) { orome_fail(OROME_EINVAL, "gguf: NULL image"); return NULL; }
    OromeHipGGUFFile *gf = calloc(1, sizeof *gf);
    gf->fd = -1;
    gf->mmap_base = (void *)data;
    gf->file_size = size;
    gf->owns_map = false;
    return parse((const uint8_t *)data, size, gf);
}

OromeHipGGUFFile *orome_hip_gguf_open(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { orome_fail(OROME_ENOTFOUND, "gguf: cannot open %s", path); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        orome_fail(OROME_EFORMAT, "gguf: %s is too small", path);
        return NULL;
    }
    void *m = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
        close(fd);
        orome_fail(OROME_EHIP, "gguf: mmap of %s failed", path);
        return NULL;
    }
    OromeHipGGUFFile *gf = calloc(1, sizeof *gf);
    gf->fd = fd;
    gf->mmap_base = m;
    gf->file_size = (size_t)st.st_size;
    gf->owns_map = true;
    return parse((const uint8_t *)m, (size_t)st.st_size, gf);
}

int orome_hip_model_config_from_gguf(const OromeHipGGUFFile *gf, OromeHipModelConfig *cfg) {
    if (!gf || !cfg) return orome_fail(OROME_EINVAL, "orome_hip_model_config_from_gguf: NULL argument");
    memset(cfg, 0, sizeof *cfg);
    snprintf(cfg->name, sizeof cfg->name, "%s", gf->arch);
    cfg->hidden_dim = gf->hidden_dim;
    cfg->num_layers = gf->num_layers;
    cfg->rms_norm_eps = gf->rms_norm_eps;
    cfg->ffn_type = gf->ffn_type;
    cfg->num_experts = gf->num_experts;
    cfg->num_experts_per_tok = gf->num_experts_per_tok;
    cfg->moe_intermediate = gf->moe_intermediate;
    /* inference/src/main.m:576-588: S from the shared gate's second dim */
    OromeHipGGUFTensorInfo *sg = orome_hip_gguf_find_tensor((OromeHipGGUFFile *)gf, "blk.0.ffn_gate_shexp.weight");
    cfg->shared_intermediate = (sg && sg->n_dims >= 2) ? (int)sg->dims[1] : 0;
    if (cfg->hidden_dim <= 0 || cfg->num_layers <= 0)
        return orome_fail(OROME_EFORMAT, "gguf: missing block_count/embedding_length");
    return OROME_OK;
}
