/*
 * moe_misc.hip -- scalar dequant kernels, fp16 staging and the prefill combine.
 */
#include "dev_common.h"
#include "kernels.h"

/* Row dequant to fp32 (and optionally fp16 RNE), one thread per 32-weight
 * chunk.  Arithmetic restates format_decode_row_f32
 * (inference/src/format.m:66-174): Q4_K and Q5_K (d*sc)*q - dmin*m, Q6_K (d*sc)*q,
 * Q8_0 d*q; every product is exact in fp32, so fused or not the result is
 * the same. */
__global__ void k_dequant(int fmt, const uint8_t *src, uint32_t rows, uint32_t n, float *o32,
                          _Float16 *o16) {
    const uint32_t nch = n / 32;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)rows * nch) return;
    const uint32_t r = (uint32_t)(gid / nch), c = (uint32_t)(gid % nch);
    float v[32];
    int pos[32];
    if (fmt == 0) { /* Q4_K: chunk = (super-block, group g, half of the 32 bytes) */
        const uint8_t *sb = src + (size_t)r * (n / 256) * 144 + (c >> 3) * 144;
        u4 hdr = ld_u4(sb);
        const int g = (c & 7) >> 1, lh = (c & 1) * 16;
        Q4Affine af = q4k_affine(hdr, g);
        for (int i = 0; i < 16; i++) {
            uint32_t byte = sb[16 + g * 32 + lh + i];
            int k = (c >> 3) * 256 + g * 64 + lh + i;
            v[i] = af.a_lo * (float)(byte & 0xF) - af.b_lo;
            pos[i] = k;
            v[16 + i] = af.a_hi * (float)(byte >> 4) - af.b_hi;
            pos[16 + i] = k + 32;
        }
    } else if (fmt == 1) { /* Q5_K: the Q4_K chunks plus bit 2g / 2g+1 of qh[l] */
        const uint8_t *sb = src + (size_t)r * (n / 256) * 176 + (c >> 3) * 176;
        u4 hdr = ld_u4(sb);
        const int g = (c & 7) >> 1, lh = (c & 1) * 16;
        Q4Affine af = q4k_affine(hdr, g);
        for (int i = 0; i < 16; i++) {
            const uint32_t byte = sb[48 + g * 32 + lh + i], qh = sb[16 + lh + i];
            const int k = (c >> 3) * 256 + g * 64 + lh + i;
            v[i] = af.a_lo * (float)((byte & 0xF) | ((qh >> (2 * g)) & 1u) << 4) - af.b_lo;
            pos[i] = k;
            v[16 + i] = af.a_hi * (float)((byte >> 4) | ((qh >> (2 * g + 1)) & 1u) << 4) - af.b_hi;
            pos[16 + i] = k + 32;
        }
    } else if (fmt == 2) { /* Q6_K: chunk = (super-block, half, 8 positions) */
        const uint8_t *sb = src + (size_t)r * (n / 256) * 210 + (c >> 3) * 210;
        const int h = (c >> 2) & 1, l0 = 8 * (c & 3);
        const uint8_t *ql = sb + h * 64, *qh = sb + 128 + h * 32;
        const int8_t *sc = (const int8_t *)(sb + 192) + h * 8;
        float d = f16_bits_to_f32((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
        for (int i = 0; i < 8; i++) {
            int l = l0 + i, is = l / 16, base = (c >> 3) * 256 + h * 128;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            v[i] = d * (float)sc[is] * (float)q1; pos[i] = base + l;
            v[8 + i] = d * (float)sc[is + 2] * (float)q2; pos[8 + i] = base + l + 32;
            v[16 + i] = d * (float)sc[is + 4] * (float)q3; pos[16 + i] = base + l + 64;
            v[24 + i] = d * (float)sc[is + 6] * (float)q4; pos[24 + i] = base + l + 96;
        }
    } else { /* Q8_0: chunk = block */
        const uint8_t *b = src + (size_t)r * (n / 32) * 34 + c * 34;
        float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        for (int i = 0; i < 32; i++) {
            v[i] = d * (float)(int8_t)b[2 + i];
            pos[i] = c * 32 + i;
        }
    }
    for (int i = 0; i < 32; i++) {
        if (o32) o32[(size_t)r * n + pos[i]] = v[i];
        if (o16) o16[(size_t)r * n + pos[i]] = (_Float16)v[i];
    }
}

int launch_dequant(int fmt, const uint8_t *src, uint32_t rows, uint32_t n, float *o32,
                   _Float16 *o16, hipStream_t s) {
    if (fmt < 0 || fmt > 3) return -2;
    if ((fmt == 3 && n % 32) || (fmt != 3 && n % 256)) return -1;
    size_t work = (size_t)rows * (n / 32);
    if (!work) return 0;
    KLAUNCH(k_dequant, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, s, fmt, src,
                       rows, n, o32, o16);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* x fp32 -> fp16 RNE (the reference's half(x) staging), each 4-group stored
 * (0,2,1,3) for the grouped GEMMs; n is a multiple of 4 */
__global__ void k_to_f16(const float *x, size_t n, _Float16 *o) {
    size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= n) {
        f4 v = *(const f4 *)(x + i);
        h4 h = {(_Float16)v.x, (_Float16)v.z, (_Float16)v.y, (_Float16)v.w}; /* (0,2,1,3) */
        *(h4 *)(o + i) = h;
    } else {
        for (; i < n; i++) o[i] = (_Float16)x[i];
    }
}

int launch_to_f16(const float *x, int T, int H, _Float16 *x16, hipStream_t s) {
    size_t n = (size_t)T * H;
    KLAUNCH(k_to_f16, dim3((unsigned)((n / 4 + 255) / 256 + 1)), dim3(256), 0, s, x, n, x16);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Prefill combine (moe_combine_copy_sq_k8, shaders.metal:1079-1135):
 *   h_out = (h_in + sum_k w_k y[pos(t,k)]) + sigmoid(s_t) * y_shared[t]
 * y holds expert outputs in expert-sorted pair order. 4 columns per thread. */
/* one 4-column group of a token's combine (the order k_combine and
 * k_combine_norm share); v/wk hold the K expert rows and weights, base the
 * h_in columns (0 without h_in), sv the shared expert's columns */
template <int KM>
DEV f4 combine4(const f4 (&v)[KM], const float (&wk)[KM], int K, f4 base, f4 sv, float g, int has_sh) {
    f4 moe = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (k < K) {
            moe.x += wk[k] * v[k].x; moe.y += wk[k] * v[k].y; moe.z += wk[k] * v[k].z; moe.w += wk[k] * v[k].w;
        }
    f4 o = {base.x + moe.x, base.y + moe.y, base.z + moe.z, base.w + moe.w};
    if (has_sh) {
        o.x = o.x + g * sv.x; o.y = o.y + g * sv.y; o.z = o.z + g * sv.z; o.w = o.w + g * sv.w;
    }
    return o;
}

/* A token's pair positions and weights (uniform loads, index clamped to
 * K - 1 past K: every load is unconditional, so none is waited for alone). */
template <int KM>
DEV void combine_pairs(const uint32_t *pos, const float *w, int t, int K, uint32_t (&pk)[KM], float (&wk)[KM]) {
#pragma unroll
    for (int k = 0; k < KM; k++) {
        const int kc = min(k, K - 1);
        pk[k] = pos[t * K + kc];
        wk[k] = w[t * K + kc];
    }
    /* hold the weights here, beside the positions the row addresses wait for
     * anyway (left alone, the scheduler reloads them after the rows arrive) */
#pragma unroll
    for (int k = 0; k < KM; k++) asm volatile("" : : "s"(wk[k]));
}

/* Canonical sum of squares of the 256 columns a wave holds as one f4 per
 * lane (columns 4 L .. 4 L + 3 at lane L): fma over the four from zero, then
 * the canonical wave sum.  Part b of a row is this over columns 256 b ..
 * 256 b + 255, the Sigma h^2 partial of moe_combine_copy_sq_k8
 * (inference/src/shaders.metal:1079-1135) in this library's fixed order. */
DEV float sumsq_part(f4 o) {
    float acc = 0.0f;
    acc = __builtin_fmaf(o.x, o.x, acc);
    acc = __builtin_fmaf(o.y, o.y, acc);
    acc = __builtin_fmaf(o.z, o.z, acc);
    acc = __builtin_fmaf(o.w, o.w, acc);
    return wave_sum_canon(acc);
}

/* res: copy of h_out (or NULL); ssq: [T][H/256] parts (or NULL; the
 * launcher passes it only when every wave holds whole 256-column blocks) */
template <int KM>
__global__ void k_combine(const float *y, const float *ysh, const uint32_t *pos, const float *w,
                          const float *sgl, int has_sh, const float *h_in, float *h_out, float *res, float *ssq,
                          int T, int H, int K) {
    const int t = blockIdx.y;
    const int c = min((int)(blockIdx.x * blockDim.x + threadIdx.x) * 4, H - 4);
    const bool live = (int)(blockIdx.x * blockDim.x + threadIdx.x) * 4 < H;
    uint32_t pk[KM];
    float wk[KM];
    combine_pairs<KM>(pos, w, t, K, pk, wk);
    const float sgt = sgl[t];
    /* all rows in flight together */
    f4 v[KM];
#pragma unroll
    for (int k = 0; k < KM; k++) v[k] = *(const f4 *)(y + (size_t)pk[k] * H + c);
    const f4 hb = *(const f4 *)((h_in ? h_in : y) + (size_t)t * H + c);
    const f4 sv = *(const f4 *)((has_sh ? ysh : y) + (size_t)t * H + c);
    const float g = has_sh ? sigmoid_f(sgt) : 0.0f;
    const f4 o = combine4<KM>(v, wk, K, h_in ? hb : f4{0, 0, 0, 0}, sv, g, has_sh);
    if (live) {
        *(f4 *)(h_out + (size_t)t * H + c) = o;
        if (res) *(f4 *)(res + (size_t)t * H + c) = o;
    }
    if (ssq) { /* whole waves of 256 live columns (H % 1024 == 0) */
        const float part = sumsq_part(o);
        if ((threadIdx.x & 63) == 0) ssq[(size_t)t * (H / 256) + c / 256] = part;
    }
}

/* Sigma h^2 parts of rows already written (sumsq_part per 256 columns): one
 * wave per (block b, token t). */
__global__ __launch_bounds__(64) void k_sumsq_parts(const float *h, int H, float *ssq) {
    const int b = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const f4 o = *(const f4 *)(h + (size_t)t * H + 256 * b + 4 * lane);
    const float part = sumsq_part(o);
    if (lane == 0) ssq[(size_t)t * (H / 256) + b] = part;
}

int launch_sumsq_parts(const float *h, int T, int H, float *ssq, hipStream_t s) {
    if (H % 256) return -2;
    KLAUNCH(k_sumsq_parts, dim3((unsigned)(H / 256), (unsigned)T), dim3(64), 0, s, h, H, ssq);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Prefill combine with the next layer's RMSNorm (k_rmsnorm's arithmetic)
 * fused in: one block of NI / 2 waves per token; wave w combines columns
 * 256 i + 4 L .. +3 (lane L) for i = w, w + NI / 2 with all of its loads
 * issued together, stores h_out and keeps the values in LDS; wave 0 then
 * forms the sum of squares in the canonical order (per lane over i, then
 * the canonical wave sum), so xnorm is bit-identical to k_rmsnorm run on
 * h_out, and every wave writes its columns of xnorm. */
template <int CN_W, int KM>
__global__ __launch_bounds__(64 * CN_W) void k_combine_norm(const float *y, const float *ysh, const uint32_t *pos,
                                                             const float *w, const float *sgl, int has_sh,
                                                             const float *h_in, float *h_out, float *res, float *ssq,
                                                             int T, int H, int K, const float *nw, float eps,
                                                             float *xnorm, _Float16 *x16) {
    __shared__ f4 ro[CANON_NI][64];
    __shared__ float sc;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, t = blockIdx.x;
    const int NI = H / 256;
    uint32_t pk[KM];
    float wk[KM];
    combine_pairs<KM>(pos, w, t, K, pk, wk);
    const float sgt = sgl[t];
    constexpr int PW = 2; /* steps per wave: NI = 2 CN_W */
    f4 v[PW][KM], hb[PW], sv[PW], wq[PW];
#pragma unroll
    for (int q = 0; q < PW; q++) {
        const int i = min(wv + CN_W * q, NI - 1), c = 256 * i + 4 * lane;
#pragma unroll
        for (int k = 0; k < KM; k++) v[q][k] = *(const f4 *)(y + (size_t)pk[k] * H + c);
        hb[q] = *(const f4 *)((h_in ? h_in : y) + (size_t)t * H + c);
        sv[q] = *(const f4 *)((has_sh ? ysh : y) + (size_t)t * H + c);
        wq[q] = *(const f4 *)((nw ? nw : y) + c);
    }
    const float g = has_sh ? sigmoid_f(sgt) : 0.0f;
#pragma unroll
    for (int q = 0; q < PW; q++) {
        const int i = wv + CN_W * q, c = 256 * i + 4 * lane;
        if (i < NI) {
            const f4 o = combine4<KM>(v[q], wk, K, h_in ? hb[q] : f4{0, 0, 0, 0}, sv[q], g, has_sh);
            *(f4 *)(h_out + (size_t)t * H + c) = o;
            if (res) *(f4 *)(res + (size_t)t * H + c) = o;
            ro[i][lane] = o;
            if (ssq) {
                const float part = sumsq_part(o);
                if (lane == 0) ssq[(size_t)t * NI + i] = part;
            }
        }
    }
    __syncthreads();
    if (wv == 0) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < CANON_NI; i++)
            if (i < NI) {
                const f4 o = ro[i][lane];
                acc = __builtin_fmaf(o.x, o.x, acc);
                acc = __builtin_fmaf(o.y, o.y, acc);
                acc = __builtin_fmaf(o.z, o.z, acc);
                acc = __builtin_fmaf(o.w, o.w, acc);
            }
        const float ss = wave_sum_canon(acc);
        if (lane == 0) sc = 1.0f / sqrtf(ss / (float)H + eps);
    }
    __syncthreads();
    const float scale = sc;
#pragma unroll
    for (int q = 0; q < PW; q++) {
        const int i = wv + CN_W * q, j = 256 * i + 4 * lane;
        if (i < NI) {
            const f4 o = ro[i][lane];
            const f4 wn = nw ? wq[q] : f4{1, 1, 1, 1};
            f4 r;
            r.x = (o.x * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wn.x) & 0xFFFF0000u);
            r.y = (o.y * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wn.y) & 0xFFFF0000u);
            r.z = (o.z * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wn.z) & 0xFFFF0000u);
            r.w = (o.w * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wn.w) & 0xFFFF0000u);
            *(f4 *)(xnorm + (size_t)t * H + j) = r;
            if (x16) /* the GEMMs' fp16 copy, (0,2,1,3) within the 4-group */
                *(h4 *)(x16 + (size_t)t * H + j) = h4{(_Float16)r.x, (_Float16)r.z, (_Float16)r.y, (_Float16)r.w};
        }
    }
}

int launch_combine_norm(const float *y, const float *ysh, const uint32_t *pos, const float *w, const float *sgl,
                        int has_shared, const float *h_in, float *h_out, float *res, float *ssq, int T, int H, int K,
                        const float *nw, float eps, float *xnorm, _Float16 *x16, hipStream_t s) {
    const int NI = H / 256;
    if (H % 512 || NI > 2 * 8 || NI > CANON_NI || K < 1 || K > OROME_MAXK) return -2;
#define CN_LAUNCH(CW)                                                                                            \
    do {                                                                                                         \
        if (K <= 8)                                                                                              \
            KLAUNCH((k_combine_norm<CW, 8>), dim3((unsigned)T), dim3(64 * CW), 0, s, y, ysh, pos, w,   \
                               sgl, has_shared, h_in, h_out, res, ssq, T, H, K, nw, eps, xnorm, x16);               \
        else                                                                                                     \
            KLAUNCH((k_combine_norm<CW, OROME_MAXK>), dim3((unsigned)T), dim3(64 * CW), 0, s, y, ysh, \
                               pos, w, sgl, has_shared, h_in, h_out, res, ssq, T, H, K, nw, eps, xnorm, x16);         \
    } while (0)
    switch (NI / 2) {
        case 1: CN_LAUNCH(1); break;
        case 2: CN_LAUNCH(2); break;
        case 3: CN_LAUNCH(3); break;
        case 4: CN_LAUNCH(4); break;
        case 5: CN_LAUNCH(5); break;
        case 6: CN_LAUNCH(6); break;
        case 7: CN_LAUNCH(7); break;
        default: CN_LAUNCH(8); break;
    }
#undef CN_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_combine(const float *y, const float *ysh, const uint32_t *pos, const float *w,
                   const float *sgl, int has_shared, const float *h_in, float *h_out, float *res, float *ssq,
                   int T, int H, int K, hipStream_t s) {
    if (H % 4 || K < 1 || K > OROME_MAXK) return -2;
    dim3 grid((H / 4 + 255) / 256, T);
    /* the parts come out of the combine when its waves hold whole 256-column
     * blocks; otherwise from a pass over h_out */
    float *fused = H % 1024 == 0 ? ssq : nullptr;
    if (K <= 8)
        KLAUNCH(k_combine<8>, grid, dim3(256), 0, s, y, ysh, pos, w, sgl, has_shared, h_in, h_out, res,
                           fused, T, H, K);
    else
        KLAUNCH(k_combine<OROME_MAXK>, grid, dim3(256), 0, s, y, ysh, pos, w, sgl, has_shared, h_in, h_out,
                           res, fused, T, H, K);
    if (hipGetLastError() != hipSuccess) return -3;
    if (ssq && !fused) return launch_sumsq_parts(h_out, T, H, ssq, s);
    return 0;
}

/* Bounded busy-wait on the GPU (one lane): holds the stream for `ticks` of the
 * 100 MHz real-time counter so the host can queue work behind it.  The loop
 * always ends (tick deadline or iteration cap). */
__global__ void k_delay(uint64_t ticks) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < (1u << 26); it++) {
        if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(127);
    }
}

int launch_delay(uint32_t usec, hipStream_t s) {
    KLAUNCH(k_delay, dim3(1), dim3(64), 0, s, (uint64_t)usec * 100u);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Q4_K scale bytes 8..11 (block bytes 12..15) from the ggml packing
 * (byte 8 + j = scale 4+j low nibble | min 4+j high nibble) to the
 * reference's (byte 8 = scales 4|5, 9 = scales 6|7, 10 = mins 4|5,
 * 11 = mins 6|7, inference/src/format.m:41-64); one thread per 144-byte
 * block. */
__global__ void k_q4k_ggml_to_ref(uint8_t *blocks, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t *w = (uint32_t *)(blocks + i * 144 + 12);
    const uint32_t g = *w;
    const uint32_t g8 = g & 0xFFu, g9 = (g >> 8) & 0xFFu, g10 = (g >> 16) & 0xFFu, g11 = g >> 24;
    const uint32_t r8 = (g8 & 0xFu) | ((g9 & 0xFu) << 4), r9 = (g10 & 0xFu) | ((g11 & 0xFu) << 4);
    const uint32_t r10 = (g8 >> 4) | (g9 & 0xF0u), r11 = (g10 >> 4) | (g11 & 0xF0u);
    *w = r8 | (r9 << 8) | (r10 << 16) | (r11 << 24);
}

int launch_q4k_ggml_to_ref(uint8_t *blocks, size_t n, hipStream_t s) {
    if (((uintptr_t)blocks & 3) || !n) return -1;
    KLAUNCH(k_q4k_ggml_to_ref, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, blocks, n);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Fill of `words` 32-bit words with `v` (a kernel, not a memset node, so
 * that callers may capture it in a graph). */
__global__ void k_fill_u32(uint32_t *p, uint32_t v, size_t words) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

int launch_fill_u32(void *p, uint32_t v, size_t words, hipStream_t s) {
    const unsigned blocks = (unsigned)((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024);
    if (!blocks) return 0;
    KLAUNCH(k_fill_u32, dim3(blocks), dim3(256), 0, s, (uint32_t *)p, v, words);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_zero(void *p, size_t bytes, hipStream_t s) {
    if (bytes % 4) return -1;
    return launch_fill_u32(p, 0u, bytes / 4, s);
}
