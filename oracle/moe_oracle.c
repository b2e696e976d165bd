/*
 * moe_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Scalar C restatement of the Orome MoE feed-forward path, used as the parity
 * checker for the HIP kernels and as the timed CPU baseline.  Nothing in the
 * product library links, loads or calls this file; only tests/, the smoke
 * check and bench.py's cpu_baseline leg do.
 *
 * Build: oracle/Makefile  (gcc -O2 -ffp-contract=off -fopenmp).
 * -ffp-contract=off keeps every a*b+c as two roundings except where fmaf() is
 * written out explicitly (router and RMSNorm sums, whose order is a defined
 * part of the contract shared with the GPU).
 *
 * Every function cites the reference source it restates
 * (paths relative to the reference repository root).
 *
 * Pinning (what checks each function beyond re-typing it):
 *   orc_fp16_to_f32        exhaustive over all 65536 codes vs numpy float16
 *   orc_f32_to_f16         exhaustive round trip + all midpoints vs numpy RNE
 *   orc_unpack_q4k_pair    exhaustive over every byte value of each field,
 *                          vs an independent bit-formula table; KAT
 *                          tests/test_q4k.m:36-66 (reference layout)
 *   orc_decode_row Q4_K    KAT test_q4k.m; closed form d*sc*q - dmin*m on
 *                          one-hot fields; exactness (Finding: products exact)
 *   orc_decode_row Q6_K    closed forms on one-hot ql/qh fields; the ggml
 *                          q6_K layout equivalence on random blocks
 *   orc_decode_row Q8_0    KAT tests/test_q8_0.m:27-70
 *   orc_router_logits      KAT tests/test_f32.m:17-30 and a float64 dot
 *                          product bound (textbook)
 *   orc_topk_route         brute force: sort by (-logit, index); invariants
 *   orc_dispatch           numpy stable argsort; permutation invariants
 *   orc_moe_forward        closed forms (constant nibbles, one-hot x,
 *                          SiLU(0)=0, sigmoid(0)=0.5) and a float64 numpy
 *                          restatement on small shapes
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* QuantFormat values, same order as the reference enum
 * (inference/include/orome.h:227-235). */
enum { Q4_K = 0, Q5_K = 1, Q6_K = 2, Q8_0 = 3, F16 = 4, BF16 = 5, F32 = 6 };

/* ---------------------------------------------------------------- A1 --- */
/* inference/src/format.m:17-32 */
ORC_API float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (ex == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        return ldexpf((float)mant, -24) * (sign ? -1.0f : 1.0f);
    }
    if (ex == 31) return mant ? NAN : (sign ? -INFINITY : INFINITY);
    uint32_t f = (sign << 31) | ((ex + 112) << 23) | (mant << 13);
    float out;
    memcpy(&out, &f, 4);
    return out;
}

/* float -> IEEE half, round to nearest even.  This is the conversion the
 * reference kernels apply when they stage activations in threadgroup memory
 * as `half(x)` (inference/src/shaders.metal:2190-2193, 2252-2255, 2612-2613).
 * Written from the IEEE-754 definition: keep 11 significant bits, round the
 * dropped bits to nearest, ties to even, saturate to inf above 65519.99. */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax < 0x38800000u) {  /* |f| < 2^-14: half subnormal or zero, unit 2^-24 */
        if (ax == 0) return (uint16_t)sign;
        int be = (int)(ax >> 23);
        uint32_t m = ax & 0x7FFFFFu;
        if (be == 0) be = 1; else m |= 0x800000u;
        int shift = 126 - be;  /* value / 2^-24 = m * 2^(be-126) */
        if (shift > 24) return (uint16_t)sign;
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), hf = 1u << (shift - 1);
        if (rem > hf || (rem == hf && (q & 1u))) q++;
        return (uint16_t)(sign | q);  /* a carry into 0x400 is the right normal encoding */
    }
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t q = m >> 13;  /* 11 significant bits */
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    int he = (int)(ax >> 23) - 112;
    if (q == 0x800u) { q = 0x400u; he++; }
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (q & 0x3FFu));
}

ORC_API float orc_round_half(float f) { return orc_fp16_to_f32(orc_f32_to_f16(f)); }

/* F32 -> BF16 truncation applied to RMSNorm weights at load
 * (inference/src/format.m:436-450) followed by the bf16 -> f32 widen
 * (inference/src/format.m:34-39). */
ORC_API float orc_bf16_trunc(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    b &= 0xFFFF0000u;
    float o;
    memcpy(&o, &b, 4);
    return o;
}

/* ---------------------------------------------------------------- A2 --- */
/* inference/src/format.m:41-64 (GPU twin inference/src/shaders.metal:1413-1436).
 * Reference layout, NOT ggml's: for pair g>=2 the low nibbles of scales come
 * from byte 8+(g-2) and of mins from byte 10+(g-2). */
ORC_API void orc_unpack_q4k_pair(const uint8_t *s, uint32_t g, float *sc_lo, float *sc_hi,
                                 float *mn_lo, float *mn_hi) {
    if (g < 2) {
        uint32_t b = g * 2;
        *sc_lo = (float)(s[b] & 63);
        *sc_hi = (float)(s[b + 1] & 63);
        *mn_lo = (float)(s[b + 4] & 63);
        *mn_hi = (float)(s[b + 5] & 63);
        return;
    }
    uint32_t b = (g - 2) * 2;
    uint8_t scp = s[8 + (g - 2)];
    uint8_t mnp = s[10 + (g - 2)];
    *sc_lo = (float)((scp & 0xF) | ((s[b] >> 6) << 4));
    *sc_hi = (float)((scp >> 4) | ((s[b + 1] >> 6) << 4));
    *mn_lo = (float)((mnp & 0xF) | ((s[b + 4] >> 6) << 4));
    *mn_hi = (float)((mnp >> 4) | ((s[b + 5] >> 6) << 4));
}

/* orc_unpack_q4k_pair over n 12-byte scale regions: out[16 r + 2 g + h] =
 * scale of sub-block 2 g + h, out[16 r + 8 + 2 g + h] = its min (lets a test
 * sweep every byte value of a field in one call). */
ORC_API void orc_unpack_q4k_batch(const uint8_t *s12, size_t n, float *out) {
    for (size_t r = 0; r < n; r++)
        for (uint32_t g = 0; g < 4; g++)
            orc_unpack_q4k_pair(s12 + 12 * r, g, out + 16 * r + 2 * g, out + 16 * r + 2 * g + 1,
                                out + 16 * r + 8 + 2 * g, out + 16 * r + 8 + 2 * g + 1);
}

/* ------------------------------------------------------------- A3-A5 --- */
/* inference/src/format.m:66-79 */
static void dec_q8_0(const uint8_t *row, uint32_t n, float *out) {
    for (uint32_t blk = 0; blk < n / 32; blk++) {
        const uint8_t *b = row + blk * 34;
        float d = orc_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        const int8_t *q = (const int8_t *)(b + 2);
        for (uint32_t j = 0; j < 32; j++) out[blk * 32 + j] = d * (float)q[j];
    }
}

/* inference/src/format.m:81-108 */
static void dec_q4_k(const uint8_t *row, uint32_t n, float *out) {
    for (uint32_t sb = 0; sb < n / 256; sb++) {
        const uint8_t *p = row + sb * 144;
        float d = orc_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        float dmin = orc_fp16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
        const uint8_t *qs = p + 16;
        for (uint32_t g = 0; g < 4; g++) {
            float sl, sh, ml, mh;
            orc_unpack_q4k_pair(p + 4, g, &sl, &sh, &ml, &mh);
            float a_lo = d * sl, a_hi = d * sh, b_lo = dmin * ml, b_hi = dmin * mh;
            for (uint32_t l = 0; l < 32; l++) {
                uint8_t byte = qs[g * 32 + l];
                out[sb * 256 + g * 64 + l] = a_lo * (float)(byte & 0xF) - b_lo;
                out[sb * 256 + g * 64 + 32 + l] = a_hi * (float)(byte >> 4) - b_hi;
            }
        }
    }
}

/* inference/src/format.m:110-142 */
static void dec_q5_k(const uint8_t *row, uint32_t n, float *out) {
    for (uint32_t sb = 0; sb < n / 256; sb++) {
        const uint8_t *p = row + sb * 176;
        float d = orc_fp16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        float dmin = orc_fp16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
        const uint8_t *qh = p + 16, *ql = p + 48;
        for (uint32_t g = 0; g < 4; g++) {
            float sl, sh, ml, mh;
            orc_unpack_q4k_pair(p + 4, g, &sl, &sh, &ml, &mh);
            float a_lo = d * sl, a_hi = d * sh, b_lo = dmin * ml, b_hi = dmin * mh;
            for (uint32_t l = 0; l < 32; l++) {
                uint8_t byte = ql[g * 32 + l];
                uint32_t lo = (byte & 0xF) | ((qh[l] >> (2 * g)) & 1u) << 4;
                uint32_t hi = (byte >> 4) | ((qh[l] >> (2 * g + 1)) & 1u) << 4;
                out[sb * 256 + g * 64 + l] = a_lo * (float)lo - b_lo;
                out[sb * 256 + g * 64 + 32 + l] = a_hi * (float)hi - b_hi;
            }
        }
    }
}

/* inference/src/format.m:144-174 */
static void dec_q6_k(const uint8_t *row, uint32_t n, float *out) {
    for (uint32_t sb = 0; sb < n / 256; sb++) {
        const uint8_t *p = row + sb * 210;
        float d = orc_fp16_to_f32((uint16_t)(p[208] | (p[209] << 8)));
        for (uint32_t h = 0; h < 2; h++) {
            const uint8_t *ql = p + h * 64, *qh = p + 128 + h * 32;
            const int8_t *sc = (const int8_t *)(p + 192) + h * 8;
            float *o = out + sb * 256 + h * 128;
            for (uint32_t l = 0; l < 32; l++) {
                uint32_t is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[l] = d * (float)sc[is] * (float)q1;
                o[l + 32] = d * (float)sc[is + 2] * (float)q2;
                o[l + 64] = d * (float)sc[is + 4] * (float)q3;
                o[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* bytes of one row of `n` weights; gguf.m:64-104 block tables */
ORC_API size_t orc_row_bytes(int fmt, uint32_t n) {
    switch (fmt) {
        case Q4_K: return (size_t)(n / 256) * 144;
        case Q5_K: return (size_t)(n / 256) * 176;
        case Q6_K: return (size_t)(n / 256) * 210;
        case Q8_0: return (size_t)(n / 32) * 34;
        case F16: case BF16: return (size_t)n * 2;
        case F32: return (size_t)n * 4;
    }
    return 0;
}

/* inference/src/format.m:176-218 (format_decode_row_f32), one row.
 * Returns 0 on success, -1 for a shape the format cannot hold. */
ORC_API int orc_decode_row(int fmt, const uint8_t *row, uint32_t n, float *out) {
    switch (fmt) {
        case Q4_K: if (n % 256) return -1; dec_q4_k(row, n, out); return 0;
        case Q5_K: if (n % 256) return -1; dec_q5_k(row, n, out); return 0;
        case Q6_K: if (n % 256) return -1; dec_q6_k(row, n, out); return 0;
        case Q8_0: if (n % 32) return -1; dec_q8_0(row, n, out); return 0;
        case F32: memcpy(out, row, (size_t)n * 4); return 0;
        case F16:
            for (uint32_t j = 0; j < n; j++)
                out[j] = orc_fp16_to_f32((uint16_t)(row[2 * j] | (row[2 * j + 1] << 8)));
            return 0;
        case BF16:
            for (uint32_t j = 0; j < n; j++) {
                uint32_t b = (uint32_t)(row[2 * j] | (row[2 * j + 1] << 8)) << 16;
                memcpy(&out[j], &b, 4);
            }
            return 0;
    }
    return -1;
}

ORC_API int orc_decode_rows(int fmt, const uint8_t *data, uint32_t rows, uint32_t n, float *out) {
    size_t rb = orc_row_bytes(fmt, n);
    for (uint32_t r = 0; r < rows; r++)
        if (orc_decode_row(fmt, data + r * rb, n, out + (size_t)r * n)) return -1;
    return 0;
}

/* ---------------------------------------------------------------- A6 --- */
/* Canonical fp32 dot product shared bit-for-bit with the GPU kernels.
 * Restates matvec_f32_pair (inference/src/shaders.metal:1368-1392): lane-
 * strided partial sums followed by a cross-lane tree.  The reference leaves
 * the order to Metal's simd_sum; this build fixes it so that router logits,
 * and therefore expert indices, are bit-exact between CPU and GPU:
 *   64 lanes; lane L owns elements j = 256*i + 4*L + c (c = 0..3), summed
 *   in increasing (i, c) with a fused multiply-add into a zero start;
 *   then for off = 32,16,8,4,2,1: p[L] = p[L] + p[L+off].
 * Requires n % 256 == 0. */
ORC_API float orc_canon_dot(const float *a, const float *b, uint32_t n) {
    float p[64];
    for (int L = 0; L < 64; L++) {
        float acc = 0.0f;
        for (uint32_t i = 0; i < n / 256; i++)
            for (int c = 0; c < 4; c++) {
                uint32_t j = 256 * i + 4 * L + c;
                acc = fmaf(a[j], b[j], acc);
            }
        p[L] = acc;
    }
    for (int off = 1; off < 64; off <<= 1)
        for (int L = 0; L < 64; L += 2 * off) p[L] = p[L] + p[L + off];
    return p[0];
}

/* logits[t*(E+1) + e] = W_r[e] . x[t] for e < E; logits[t*(E+1) + E] = w_sg . x[t]
 * (inference/src/shaders.metal:1368-1392, dispatched at inference/src/engine.m:658-679).
 * A NULL w_sg writes 0 into the shared-gate slot. */
ORC_API void orc_router_logits(const float *W, const float *wsg, const float *x, int T, int E,
                               int H, float *logits) {
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        for (int e = 0; e < E; e++)
            logits[(size_t)t * (E + 1) + e] = orc_canon_dot(W + (size_t)e * H, x + (size_t)t * H, H);
        logits[(size_t)t * (E + 1) + E] = wsg ? orc_canon_dot(wsg, x + (size_t)t * H, H) : 0.0f;
    }
}

/* ---------------------------------------------------------------- A7 --- */
/* inference/src/shaders.metal:1141-1234 (softmax_topk_route):
 *  - K rounds of argmax over the raw logits (plus the optional per-expert bias
 *    of the skewed-routing config); slot order = descending logit;
 *  - exact ties go to the lower expert index.  That is the rule the task's
 *    contract states; the reference's own kernel resolves an exact tie by the
 *    position in its shuffle-down tree (1166-1200: lane L keeps its value
 *    against L + offset on a tie, so a tie between experts 1 and 2 selects 2,
 *    one between 8 and 16 selects 16).  Distinct values select identically;
 *  - w_k = exp(l_k - l_0) / sum_k exp(l_j - l_0), summed k = 0..K-1 and
 *    multiplied by the reciprocal of the sum (1212-1226);
 *  - the shared-gate logit is passed through (1232).
 * -0.0 and +0.0 compare equal (IEEE), so they tie by index.  Logits must not
 * be NaN. */
ORC_API void orc_topk_route(const float *logits, const float *bias, int T, int E, int K,
                            int32_t *idx, float *w, float *sg_logit) {
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t)t * (E + 1);
        unsigned char taken[4096];
        memset(taken, 0, (size_t)E);
        float vals[64];
        for (int k = 0; k < K; k++) {
            int best = -1;
            float bv = 0.0f;
            for (int e = 0; e < E; e++) {
                if (taken[e]) continue;
                float v = bias ? l[e] + bias[e] : l[e];
                if (best < 0 || v > bv) { best = e; bv = v; }
            }
            taken[best] = 1;
            idx[t * K + k] = best;
            vals[k] = bv;
        }
        float mx = vals[0], sum = 0.0f, tw[64];
        for (int k = 0; k < K; k++) { tw[k] = expf(vals[k] - mx); sum += tw[k]; }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int k = 0; k < K; k++) w[t * K + k] = tw[k] * inv;
        if (sg_logit) sg_logit[t] = l[E];
    }
}

/* ---------------------------------------------------------------- A8 --- */
/* Token -> expert dispatch (no counterpart in the reference, which routes one
 * token at a time).  Contract: stable counting sort of the pairs p = t*K + k,
 * taken in increasing p, by expert idx[p].  offsets[e]..offsets[e+1] is the
 * run of expert e in `pairs`; offsets has E+1 entries. */
ORC_API void orc_dispatch(const int32_t *idx, int T, int K, int E, uint32_t *offsets,
                          uint32_t *pairs) {
    uint32_t *cnt = calloc((size_t)E + 1, sizeof(uint32_t));
    for (int p = 0; p < T * K; p++) cnt[idx[p]]++;
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + cnt[e];
    memcpy(cnt, offsets, (size_t)E * sizeof(uint32_t));
    for (int p = 0; p < T * K; p++) pairs[cnt[idx[p]]++] = (uint32_t)p;
    free(cnt);
}

/* ---------------------------------------------------------------- A14 -- */
/* RMSNorm before the MoE block, x = (h * rsqrt(mean(h^2) + eps)) * w_bf16
 * (inference/src/shaders.metal:128-149, weights truncated to bf16 at load,
 * inference/src/format.m:436-450).  The sum of squares uses the canonical
 * order of orc_canon_dot; the reciprocal square root is computed as
 * 1/sqrtf (both correctly rounded). */
ORC_API void orc_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x) {
    for (int t = 0; t < T; t++) {
        const float *ht = h + (size_t)t * H;
        float ss = orc_canon_dot(ht, ht, H);
        float scale = 1.0f / sqrtf(ss / (float)H + eps);
        for (int j = 0; j < H; j++) x[(size_t)t * H + j] = (ht[j] * scale) * orc_bf16_trunc(w ? w[j] : 1.0f);
    }
}

/* ----------------------------------------------------------- A9-A13 --- */
typedef struct {
    int E, H, M, S;
    const float *router;       /* [E][H] fp32 (ffn_gate_inp) */
    const float *shared_gate_vec; /* [H] fp32 (ffn_gate_inp_shexp) or NULL */
    const float *bias;         /* [E] or NULL (skewed-routing config) */
    const uint8_t *gate; size_t gate_stride; int gate_fmt;  /* [E][M rows of H] */
    const uint8_t *up;   size_t up_stride;   int up_fmt;
    const uint8_t *down; size_t down_stride; int down_fmt;  /* [E][H rows of M] */
    const uint8_t *sh_gate; int sh_gate_fmt;  /* [S rows of H] or NULL: no shared expert */
    const uint8_t *sh_up;   int sh_up_fmt;
    const uint8_t *sh_down; int sh_down_fmt;  /* [H rows of S] */
} orc_layer;

static float silu(float g) { return g / (1.0f + expf(-g)); }

/* act[r] = silu(Wg[r].hx) * (Wu[r].hx), hx = half(x): restates
 * batch_expert_gate_up_swiglu_q4k_dyn (inference/src/shaders.metal:2232-2310)
 * and shared_gate_up_swiglu_q{4k,8_0} (2316-2445) with a sequential fp32 sum. */
static void gate_up(const float *Wg, const float *Wu, int rows, int n, const float *hx,
                    float *act) {
    for (int r = 0; r < rows; r++) {
        const float *g = Wg + (size_t)r * n, *u = Wu + (size_t)r * n;
        float sg = 0.0f, su = 0.0f;
        for (int j = 0; j < n; j++) { sg += g[j] * hx[j]; su += u[j] * hx[j]; }
        act[r] = silu(sg) * su;
    }
}

/* y[r] = Wd[r].half(act): batch_expert_down_q4k_dyn (shaders.metal:2590-2668),
 * dequant_matvec_q4k/q6k/q8_0 for the shared expert (1438, 1888, 1627). */
static void down(const float *Wd, int rows, int n, const float *hact, float *y) {
    for (int r = 0; r < rows; r++) {
        const float *w = Wd + (size_t)r * n;
        float s = 0.0f;
        for (int j = 0; j < n; j++) s += w[j] * hact[j];
        y[r] = s;
    }
}

/* Full MoE block for T tokens (inference/src/engine.m:158-340 stage order):
 * routing, top-k, routed experts, shared expert, combine
 *   h_out[t] = (h_in[t] + sum_k w_k y_k) + sigmoid(s_t) * y_shared
 * (moe_combine_copy_sq_k8, inference/src/shaders.metal:1079-1135).
 * h_in may be NULL (zero residual).  Optional debug outputs (any may be NULL):
 * logits [T][E+1], idx/w [T][K], y_routed [T][K][H], y_shared [T][H].
 * Experts are decoded once each and applied to all tokens routed to them,
 * which computes exactly the per-token arithmetic above. */
ORC_API int orc_moe_forward(const orc_layer *L, const float *x, const float *h_in, float *h_out,
                            int T, int K, float *dbg_logits, int32_t *dbg_idx, float *dbg_w,
                            float *dbg_y, float *dbg_ysh) {
    const int E = L->E, H = L->H, M = L->M, S = L->S;
    if (H % 256 || M % 256 || (L->sh_gate && S % 256) || K < 1 || K > 64 || E > 4096) return -1;
    float *logits = malloc(sizeof(float) * (size_t)T * (E + 1));
    int32_t *idx = malloc(sizeof(int32_t) * (size_t)T * K);
    float *w = malloc(sizeof(float) * (size_t)T * K);
    float *sgl = malloc(sizeof(float) * (size_t)T);
    float *hx = malloc(sizeof(float) * (size_t)T * H);
    float *y = calloc((size_t)T * K * H, sizeof(float));
    float *ysh = calloc((size_t)T * H, sizeof(float));
    uint32_t *off = malloc(sizeof(uint32_t) * (E + 1));
    uint32_t *pairs = malloc(sizeof(uint32_t) * (size_t)T * K);
    float *Wg = malloc(sizeof(float) * (size_t)M * H);
    float *Wu = malloc(sizeof(float) * (size_t)M * H);
    float *Wd = malloc(sizeof(float) * (size_t)H * M);

    orc_router_logits(L->router, L->shared_gate_vec, x, T, E, H, logits);
    orc_topk_route(logits, L->bias, T, E, K, idx, w, sgl);
    orc_dispatch(idx, T, K, E, off, pairs);
    for (size_t i = 0; i < (size_t)T * H; i++) hx[i] = orc_round_half(x[i]);

    size_t gb = orc_row_bytes(L->gate_fmt, H), ub = orc_row_bytes(L->up_fmt, H),
           db = orc_row_bytes(L->down_fmt, M);
    for (int e = 0; e < E; e++) {
        uint32_t n = off[e + 1] - off[e];
        if (!n) continue;
        const uint8_t *ge = L->gate + (size_t)e * L->gate_stride;
        const uint8_t *ue = L->up + (size_t)e * L->up_stride;
        const uint8_t *de = L->down + (size_t)e * L->down_stride;
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < M; r++) {
            orc_decode_row(L->gate_fmt, ge + r * gb, H, Wg + (size_t)r * H);
            orc_decode_row(L->up_fmt, ue + r * ub, H, Wu + (size_t)r * H);
        }
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < H; r++) orc_decode_row(L->down_fmt, de + r * db, M, Wd + (size_t)r * M);
        #pragma omp parallel for schedule(dynamic, 1)
        for (uint32_t q = 0; q < n; q++) {
            uint32_t p = pairs[off[e] + q];
            int t = (int)(p / K);
            float *act = malloc(sizeof(float) * M);
            gate_up(Wg, Wu, M, H, hx + (size_t)t * H, act);
            for (int r = 0; r < M; r++) act[r] = orc_round_half(act[r]);
            down(Wd, H, M, act, y + (size_t)p * H);
            free(act);
        }
    }
    if (L->sh_gate) {
        size_t sgb = orc_row_bytes(L->sh_gate_fmt, H), sub = orc_row_bytes(L->sh_up_fmt, H),
               sdb = orc_row_bytes(L->sh_down_fmt, S);
        float *Sg = malloc(sizeof(float) * (size_t)S * H), *Su = malloc(sizeof(float) * (size_t)S * H),
              *Sd = malloc(sizeof(float) * (size_t)H * S);
        for (int r = 0; r < S; r++) {
            orc_decode_row(L->sh_gate_fmt, L->sh_gate + r * sgb, H, Sg + (size_t)r * H);
            orc_decode_row(L->sh_up_fmt, L->sh_up + r * sub, H, Su + (size_t)r * H);
        }
        for (int r = 0; r < H; r++) orc_decode_row(L->sh_down_fmt, L->sh_down + r * sdb, S, Sd + (size_t)r * S);
        #pragma omp parallel for schedule(dynamic, 1)
        for (int t = 0; t < T; t++) {
            float *act = malloc(sizeof(float) * S);
            gate_up(Sg, Su, S, H, hx + (size_t)t * H, act);
            for (int r = 0; r < S; r++) act[r] = orc_round_half(act[r]);
            down(Sd, H, S, act, ysh + (size_t)t * H);
            free(act);
        }
        free(Sg); free(Su); free(Sd);
    }
    for (int t = 0; t < T; t++) {
        float g = L->sh_gate ? 1.0f / (1.0f + expf(-sgl[t])) : 0.0f;
        for (int r = 0; r < H; r++) {
            float moe = 0.0f;
            for (int k = 0; k < K; k++) moe += w[t * K + k] * y[((size_t)t * K + k) * H + r];
            float base = h_in ? h_in[(size_t)t * H + r] : 0.0f;
            h_out[(size_t)t * H + r] = (base + moe) + g * ysh[(size_t)t * H + r];
        }
    }
    if (dbg_logits) memcpy(dbg_logits, logits, sizeof(float) * (size_t)T * (E + 1));
    if (dbg_idx) memcpy(dbg_idx, idx, sizeof(int32_t) * (size_t)T * K);
    if (dbg_w) memcpy(dbg_w, w, sizeof(float) * (size_t)T * K);
    if (dbg_y) memcpy(dbg_y, y, sizeof(float) * (size_t)T * K * H);
    if (dbg_ysh) memcpy(dbg_ysh, ysh, sizeof(float) * (size_t)T * H);
    free(logits); free(idx); free(w); free(sgl); free(hx); free(y); free(ysh); free(off);
    free(pairs); free(Wg); free(Wu); free(Wd);
    return 0;
}

ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

ORC_API void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
