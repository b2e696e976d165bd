/*
 * synth.c -- seeded synthetic Qwen3.5-MoE GGUF images (see orome_synth.h).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "orome_internal.h"
#include "orome_moe.h"
#include "orome_synth.h"

/* ---------------------------------------------------------------- rng */
typedef struct { uint64_t s[4]; } xo_t;

static uint64_t splitmix(uint64_t *x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static void xo_seed(xo_t *r, uint64_t seed, uint64_t stream) {
    uint64_t x = seed ^ (stream * 0xD1B54A32D192ED03ull + 0x8CB92BA72F3D8DD7ull);
    for (int i = 0; i < 4; i++) r->s[i] = splitmix(&x);
}
static inline uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }
static inline uint64_t xo_next(xo_t *r) {
    uint64_t *s = r->s;
    uint64_t out = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t; s[3] = rotl(s[3], 45);
    return out;
}
static double xo_unit(xo_t *r) { return ((double)(xo_next(r) >> 11) + 0.5) * 0x1.0p-53; }
static double xo_normal(xo_t *r) {
    double u1 = xo_unit(r), u2 = xo_unit(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}
static void xo_bytes(xo_t *r, uint8_t *dst, size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8) { uint64_t v = xo_next(r); memcpy(dst + i, &v, 8); }
    if (i < n) { uint64_t v = xo_next(r); memcpy(dst + i, &v, n - i); }
}

/* float -> fp16 bits, round to nearest even */
static uint16_t to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax < 0x38800000u) {
        if (ax == 0) return (uint16_t)sign;
        int be = (int)(ax >> 23);
        uint32_t m = ax & 0x7FFFFFu;
        if (be == 0) be = 1; else m |= 0x800000u;
        int sh = 126 - be;
        if (sh > 24) return (uint16_t)sign;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), hf = 1u << (sh - 1);
        if (rem > hf || (rem == hf && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u, q = m >> 13, rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    int he = (int)(ax >> 23) - 112;
    if (q == 0x800u) { q = 0x400u; he++; }
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (q & 0x3FFu));
}
static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* one row-block range of a quantized tensor: `n` weights */
/* Scale bytes 8..11 of a Q4_K block from the reference packing (8 = scales
 * 4|5, 9 = scales 6|7, 10 = mins 4|5, 11 = mins 6|7) to ggml's (8 + j =
 * scale 4+j | min 4+j << 4); the values the block decodes to are unchanged. */
static void q4k_to_ggml(uint8_t *blk) {
    uint8_t *b = blk + 12;
    const uint8_t r8 = b[0], r9 = b[1], r10 = b[2], r11 = b[3];
    b[0] = (uint8_t)((r8 & 0xF) | ((r10 & 0xF) << 4));
    b[1] = (uint8_t)((r8 >> 4) | (r10 & 0xF0));
    b[2] = (uint8_t)((r9 & 0xF) | ((r11 & 0xF) << 4));
    b[3] = (uint8_t)((r9 >> 4) | (r11 & 0xF0));
}

static void fill_quant(xo_t *r, uint32_t type, uint8_t *dst, size_t nweights, int centered, int ggml) {
    if (type == 12) {  /* Q4_K */
        for (size_t b = 0; b < nweights / 256; b++) {
            uint8_t *p = dst + b * 144;
            float d = (float)(fabs(xo_normal(r)) * 2e-3);
            put16(p, to_f16(d));
            put16(p + 2, to_f16((float)(fabs(xo_normal(r)) * 1e-3)));
            xo_bytes(r, p + 4, 140);
            if (centered) {
                /* mins = scales under the reference packing: bytes 4..7 copy
                 * 0..3 and bytes 10..11 copy 8..9 */
                uint16_t dq = to_f16(d);
                float dd;
                { uint32_t e = (dq >> 10) & 31, m = dq & 1023;
                  dd = e ? ldexpf((float)(m | 1024), (int)e - 25) : ldexpf((float)m, -24); }
                put16(p + 2, to_f16(7.5f * dd));
                memcpy(p + 8, p + 4, 4);
                memcpy(p + 14, p + 12, 2);
            }
            if (ggml) q4k_to_ggml(p);
        }
    } else if (type == 13) {  /* Q5_K: Q4_K's header, qh[32] and ql[128] uniform */
        for (size_t b = 0; b < nweights / 256; b++) {
            uint8_t *p = dst + b * 176;
            put16(p, to_f16((float)(fabs(xo_normal(r)) * 1e-3)));
            put16(p + 2, to_f16((float)(fabs(xo_normal(r)) * 1e-3)));
            xo_bytes(r, p + 4, 172);
        }
    } else if (type == 14) {  /* Q6_K */
        for (size_t b = 0; b < nweights / 256; b++) {
            uint8_t *p = dst + b * 210;
            xo_bytes(r, p, 192);
            for (int i = 0; i < 16; i++) p[192 + i] = (uint8_t)(int8_t)((int)(xo_next(r) % 128u) - 64);
            put16(p + 208, to_f16((float)(fabs(xo_normal(r)) * 2e-3)));
        }
    } else if (type == 8) {  /* Q8_0 */
        for (size_t b = 0; b < nweights / 32; b++) {
            uint8_t *p = dst + b * 34;
            put16(p, to_f16((float)(fabs(xo_normal(r)) * 4e-3)));
            for (int i = 0; i < 32; i++) p[2 + i] = (uint8_t)(int8_t)((int)(xo_next(r) % 255u) - 127);
        }
    }
}

static size_t type_bytes(uint32_t type, size_t n) {
    switch (type) {
        case 0: return n * 4;
        case 12: return n / 256 * 144;
        case 13: return n / 256 * 176;
        case 14: return n / 256 * 210;
        case 8: return n / 32 * 34;
    }
    return 0;
}

/* ------------------------------------------------------------- layout */
enum { K_NORM, K_ROUTER, K_SHGATEVEC, K_BIAS, K_GATE, K_UP, K_DOWN, K_SHG, K_SHU, K_SHD, K_COUNT };

typedef struct {
    char name[96];
    uint32_t n_dims;
    uint64_t dims[3];
    uint32_t type;
    int kind, layer;
    uint64_t offset;  /* in the data section */
    size_t bytes;
} tdesc;

#define ALIGN 32u

static int spec_ok(const orome_synth_spec *s) {
    if (!s || s->num_layers <= 0 || s->hidden_dim <= 0 || s->hidden_dim % 256 ||
        s->num_experts <= 0 || s->moe_intermediate <= 0 || s->moe_intermediate % 256 ||
        s->shared_intermediate < 0 || s->shared_intermediate % 256)
        return 0;
    uint32_t ok[] = {12, 13, 14, 8};
    uint32_t ts[] = {s->gate_type, s->up_type, s->down_type, s->shared_gate_type, s->shared_down_type};
    for (int i = 0; i < 5; i++) {
        if (i >= 3 && !s->shared_intermediate) continue;
        int f = 0;
        for (int j = 0; j < 4; j++) f |= ts[i] == ok[j];
        if (!f) return 0;
    }
    return 1;
}

static int build_descs(const orome_synth_spec *s, tdesc **out) {
    int per = K_COUNT, n = 0;
    tdesc *d = calloc((size_t)s->num_layers * per, sizeof(tdesc));
    uint64_t H = (uint64_t)s->hidden_dim, E = (uint64_t)s->num_experts,
             M = (uint64_t)s->moe_intermediate, S = (uint64_t)s->shared_intermediate;
    uint64_t off = 0;
    for (int l = 0; l < s->num_layers; l++) {
        for (int k = 0; k < per; k++) {
            tdesc t;
            memset(&t, 0, sizeof t);
            t.kind = k;
            t.layer = l;
            uint32_t down = s->down_type;
            if (s->q6k_down_every > 0 && l % s->q6k_down_every == s->q6k_down_every - 1) down = 14;
            switch (k) {
                case K_NORM: snprintf(t.name, sizeof t.name, "blk.%d.ffn_norm.weight", l);
                    t.n_dims = 1; t.dims[0] = H; t.type = 0; break;
                case K_ROUTER: snprintf(t.name, sizeof t.name, "blk.%d.ffn_gate_inp.weight", l);
                    t.n_dims = 2; t.dims[0] = H; t.dims[1] = E; t.type = 0; break;
                case K_SHGATEVEC: if (!S) continue;
                    snprintf(t.name, sizeof t.name, "blk.%d.ffn_gate_inp_shexp.weight", l);
                    t.n_dims = 1; t.dims[0] = H; t.type = 0; break;
                case K_BIAS: if (!s->zipf_bias) continue;
                    snprintf(t.name, sizeof t.name, "blk.%d.exp_probs_b.bias", l);
                    t.n_dims = 1; t.dims[0] = E; t.type = 0; break;
                case K_GATE: snprintf(t.name, sizeof t.name, "blk.%d.ffn_gate_exps.weight", l);
                    t.n_dims = 3; t.dims[0] = H; t.dims[1] = M; t.dims[2] = E; t.type = s->gate_type; break;
                case K_UP: snprintf(t.name, sizeof t.name, "blk.%d.ffn_up_exps.weight", l);
                    t.n_dims = 3; t.dims[0] = H; t.dims[1] = M; t.dims[2] = E; t.type = s->up_type; break;
                case K_DOWN: snprintf(t.name, sizeof t.name, "blk.%d.ffn_down_exps.weight", l);
                    t.n_dims = 3; t.dims[0] = M; t.dims[1] = H; t.dims[2] = E; t.type = down; break;
                case K_SHG: if (!S) continue;
                    snprintf(t.name, sizeof t.name, "blk.%d.ffn_gate_shexp.weight", l);
                    t.n_dims = 2; t.dims[0] = H; t.dims[1] = S; t.type = s->shared_gate_type; break;
                case K_SHU: if (!S) continue;
                    snprintf(t.name, sizeof t.name, "blk.%d.ffn_up_shexp.weight", l);
                    t.n_dims = 2; t.dims[0] = H; t.dims[1] = S; t.type = s->shared_gate_type; break;
                case K_SHD: if (!S) continue;
                    snprintf(t.name, sizeof t.name, "blk.%d.ffn_down_shexp.weight", l);
                    t.n_dims = 2; t.dims[0] = S; t.dims[1] = H; t.type = s->shared_down_type; break;
            }
            uint64_t nel = 1;
            for (uint32_t i = 0; i < t.n_dims; i++) nel *= t.dims[i];
            t.bytes = type_bytes(t.type, nel);
            t.offset = off;
            off = (off + t.bytes + ALIGN - 1) / ALIGN * ALIGN;
            d[n++] = t;
        }
    }
    *out = d;
    return n;
}

static size_t str_bytes(const char *s) { return 8 + strlen(s); }

typedef struct { const char *key; int is_str; uint32_t u; float f; int is_f; const char *s; } kv_t;

static int make_kvs(const orome_synth_spec *s, kv_t *kv, char keys[][64]) {
    int n = 0;
    kv[n++] = (kv_t){"general.architecture", 1, 0, 0, 0, "qwen35moe"};
    kv[n++] = (kv_t){"general.alignment", 0, ALIGN, 0, 0, NULL};
    const char *f[] = {"block_count", "embedding_length", "expert_count", "expert_used_count",
                       "expert_feed_forward_length", "expert_shared_feed_forward_length"};
    uint32_t v[] = {(uint32_t)s->num_layers, (uint32_t)s->hidden_dim, (uint32_t)s->num_experts,
                    (uint32_t)s->num_experts_per_tok, (uint32_t)s->moe_intermediate,
                    (uint32_t)s->shared_intermediate};
    for (int i = 0; i < 6; i++) {
        snprintf(keys[i], 64, "qwen35moe.%s", f[i]);
        kv[n++] = (kv_t){keys[i], 0, v[i], 0, 0, NULL};
    }
    snprintf(keys[6], 64, "qwen35moe.attention.layer_norm_rms_epsilon");
    kv[n++] = (kv_t){keys[6], 0, 0, s->rms_norm_eps, 1, NULL};
    if (s->q4k_ggml_layout) kv[n++] = (kv_t){OROME_Q4K_LAYOUT_KEY, 1, 0, 0, 0, "ggml"};
    return n;
}

static size_t header_bytes(const orome_synth_spec *s, const tdesc *d, int nt) {
    kv_t kv[16];
    char keys[8][64];
    int nk = make_kvs(s, kv, keys);
    size_t b = 4 + 4 + 8 + 8;
    for (int i = 0; i < nk; i++) b += str_bytes(kv[i].key) + 4 + (kv[i].is_str ? str_bytes(kv[i].s) : 4);
    for (int i = 0; i < nt; i++) b += str_bytes(d[i].name) + 4 + 8 * d[i].n_dims + 4 + 8;
    return (b + ALIGN - 1) / ALIGN * ALIGN;
}

size_t orome_synth_gguf_size(const orome_synth_spec *s) {
    if (!spec_ok(s)) return 0;
    tdesc *d;
    int nt = build_descs(s, &d);
    size_t data = nt ? (size_t)(d[nt - 1].offset + d[nt - 1].bytes) : 0;
    size_t total = header_bytes(s, d, nt) + data;
    free(d);
    return total;
}

static uint8_t *w_u32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); return p + 4; }
static uint8_t *w_u64(uint8_t *p, uint64_t v) { memcpy(p, &v, 8); return p + 8; }
static uint8_t *w_str(uint8_t *p, const char *s) {
    uint64_t l = strlen(s);
    p = w_u64(p, l);
    memcpy(p, s, l);
    return p + l;
}

static uint64_t stream_id(int layer, int kind, uint64_t unit) {
    return (((uint64_t)layer * 16 + (uint64_t)kind) << 32) | unit;
}

int orome_synth_gguf_write(const orome_synth_spec *s, void *dst, size_t size) {
    if (!spec_ok(s) || !dst) return orome_fail(OROME_EINVAL, "synth: invalid spec");
    tdesc *d;
    int nt = build_descs(s, &d);
    size_t hb = header_bytes(s, d, nt);
    size_t need = hb + (nt ? (size_t)(d[nt - 1].offset + d[nt - 1].bytes) : 0);
    if (size < need) { free(d); return orome_fail(OROME_EINVAL, "synth: buffer too small"); }
    uint8_t *base = (uint8_t *)dst, *p = base;
    kv_t kv[16];
    char keys[8][64];
    int nk = make_kvs(s, kv, keys);
    p = w_u32(p, 0x46554747u);
    p = w_u32(p, 3);
    p = w_u64(p, (uint64_t)nt);
    p = w_u64(p, (uint64_t)nk);
    for (int i = 0; i < nk; i++) {
        p = w_str(p, kv[i].key);
        if (kv[i].is_str) { p = w_u32(p, 8); p = w_str(p, kv[i].s); }
        else if (kv[i].is_f) { p = w_u32(p, 6); memcpy(p, &kv[i].f, 4); p += 4; }
        else { p = w_u32(p, 4); p = w_u32(p, kv[i].u); }
    }
    for (int i = 0; i < nt; i++) {
        p = w_str(p, d[i].name);
        p = w_u32(p, d[i].n_dims);
        for (uint32_t j = 0; j < d[i].n_dims; j++) p = w_u64(p, d[i].dims[j]);
        p = w_u32(p, d[i].type);
        p = w_u64(p, d[i].offset);
    }
    memset(p, 0, (size_t)(base + hb - p));
    uint8_t *data = base + hb;

    /* work units: expert tensors split per expert, others whole */
    size_t nunits = 0;
    for (int i = 0; i < nt; i++) nunits += (d[i].n_dims == 3) ? d[i].dims[2] : 1;
    int *ut = malloc(sizeof(int) * nunits);
    uint64_t *ue = malloc(sizeof(uint64_t) * nunits);
    size_t u = 0;
    for (int i = 0; i < nt; i++) {
        uint64_t ne = (d[i].n_dims == 3) ? d[i].dims[2] : 1;
        for (uint64_t e = 0; e < ne; e++) { ut[u] = i; ue[u] = e; u++; }
    }
    const double zs = s->zipf_s > 0 ? s->zipf_s : 1.1;
    #pragma omp parallel for schedule(dynamic, 4)
    for (long long iu = 0; iu < (long long)nunits; iu++) {
        const tdesc *t = &d[ut[iu]];
        uint64_t e = ue[iu];
        xo_t r;
        xo_seed(&r, s->seed, stream_id(t->layer, t->kind, e));
        uint8_t *out = data + t->offset;
        if (t->type != 0) {
            size_t per = t->bytes / ((t->n_dims == 3) ? t->dims[2] : 1);
            size_t nw = (size_t)t->dims[0] * t->dims[1];
            fill_quant(&r, t->type, out + e * per, nw, s->centered, s->q4k_ggml_layout);
            continue;
        }
        float *f = (float *)out;
        size_t n = t->bytes / 4;
        if (t->kind == K_NORM) {
            for (size_t i = 0; i < n; i++) f[i] = 1.0f;
        } else if (t->kind == K_BIAS) {
            /* Zipf popularity over ranks 1..E mapped through a seeded permutation */
            int E = (int)n;
            int *perm = malloc(sizeof(int) * E);
            for (int i = 0; i < E; i++) perm[i] = i;
            for (int i = E - 1; i > 0; i--) {
                int j = (int)(xo_next(&r) % (uint64_t)(i + 1));
                int tmp = perm[i]; perm[i] = perm[j]; perm[j] = tmp;
            }
            double z = 0;
            for (int rk = 1; rk <= E; rk++) z += pow((double)rk, -zs);
            for (int ex = 0; ex < E; ex++) f[ex] = (float)log(pow((double)(perm[ex] + 1), -zs) / z);
            free(perm);
        } else {
            for (size_t i = 0; i < n; i++) f[i] = (float)(xo_normal(&r) * 0.02);
        }
    }
    free(ut);
    free(ue);
    free(d);
    return OROME_OK;
}

int orome_synth_normal(uint64_t seed, uint64_t stream, float std, float *out, size_t n) {
    if (!out && n) return orome_fail(OROME_EINVAL, "synth: NULL output");
    xo_t r;
    xo_seed(&r, seed, 0xFFFF000000000000ull ^ stream);
    for (size_t i = 0; i < n; i++) out[i] = (float)(xo_normal(&r) * std);
    return OROME_OK;
}
