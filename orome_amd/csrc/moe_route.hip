/*
 * moe_route.hip -- router logits, top-k selection and token->expert dispatch.
 *
 * Router logits restate matvec_f32_pair (inference/src/shaders.metal:1368-1392)
 * with a fixed reduction order shared bit-for-bit with the C oracle:
 *   lane L of a wave64 owns elements j = 256*i + 4*L + c, summed in (i, c)
 *   order with fused multiply-adds from zero, then a balanced tree over
 *   contiguous lanes (xor butterfly 1,2,...,32 as seen by lane 0), done with
 *   DPP within rows of 16 and readlanes across rows.  Identical logits make
 *   the selected experts identical.
 * Selection restates softmax_topk_route (shaders.metal:1141-1234): K rounds
 * of argmax, ties to the lower expert index, softmax over the K winners.
 * It runs as a wave64 max over 64-bit keys (order-preserving float bits,
 * then the complemented index), so one reduction settles value and tie.
 * Dispatch is a stable counting sort of pairs p = t*K + k by expert.
 */
#include "dev_common.h"
#include "kernels.h"

#include "route_dev.h"

/* canonical dot of one wave over H (H % 256 == 0, H <= 4096), for up to
 * TMAX tokens; all loads of a row are issued before the multiply-adds */
#define CANON_NI 16
template <int TMAX>
DEV void canon_dots(const float *wrow, const float *x, int T, int H, int lane, float *acc) {
    const int NI = H / 256;
    f4 wv[CANON_NI];
#pragma unroll
    for (int i = 0; i < CANON_NI; i++)
        if (i < NI) wv[i] = *(const f4 *)(wrow + 256 * i + 4 * lane);
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        acc[t] = 0.0f;
        if (t < T) {
            f4 xv[CANON_NI];
#pragma unroll
            for (int i = 0; i < CANON_NI; i++)
                if (i < NI) xv[i] = *(const f4 *)(x + (size_t)t * H + 256 * i + 4 * lane);
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < CANON_NI; i++)
                if (i < NI) {
                    a = __builtin_fmaf(wv[i].x, xv[i].x, a);
                    a = __builtin_fmaf(wv[i].y, xv[i].y, a);
                    a = __builtin_fmaf(wv[i].z, xv[i].z, a);
                    a = __builtin_fmaf(wv[i].w, xv[i].w, a);
                }
            acc[t] = wave_sum_canon(a);
        }
    }
}

/* Small-batch router logits (T <= 16): every wave computes one router row
 * (or the shared-gate row) for all tokens. */
__global__ __launch_bounds__(256) void k_route_small(RouteArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int E = a.E, H = a.H, T = a.T;
    if (row > E) return;
    const float *wr = row < E ? a.W + (size_t)row * H : a.wsg;
    float acc[16];
    if (wr) {
        canon_dots<16>(wr, a.x, T, H, lane, acc);
    } else {
#pragma unroll
        for (int t = 0; t < 16; t++) acc[t] = 0.0f;
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < 16; t++)
            if (t < T) a.logits[(size_t)t * (E + 1) + row] = acc[t];
    }
}

template <int EPL>
__global__ __launch_bounds__(256) void k_topk_dispatch_small(RouteArgs a) {
    topk_dispatch_block<EPL, false>(a);
}

/* Large-batch router logits: a block computes 16 rows x 8 tokens; each wave
 * 4 rows x 8 tokens with the canonical per-logit order. */
__global__ __launch_bounds__(256) void k_route_logits(RouteArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int E = a.E, H = a.H, T = a.T;
    const int r0 = blockIdx.x * 16 + wv * 4, t0 = blockIdx.y * 8;
    float acc[4][8];
    const float *wr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int row = r0 + r;
        wr[r] = row < E ? a.W + (size_t)row * H : (row == E ? a.wsg : nullptr);
#pragma unroll
        for (int t = 0; t < 8; t++) acc[r][t] = 0.0f;
    }
    const int nt = min(8, T - t0);
    for (int i = 0; i < H / 256; i++) {
        f4 xv[8];
#pragma unroll
        for (int t = 0; t < 8; t++)
            xv[t] = t < nt ? *(const f4 *)(a.x + (size_t)(t0 + t) * H + 256 * i + 4 * lane) : f4{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (!wr[r]) continue;
            f4 w = *(const f4 *)(wr[r] + 256 * i + 4 * lane);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                acc[r][t] = __builtin_fmaf(w.x, xv[t].x, acc[r][t]);
                acc[r][t] = __builtin_fmaf(w.y, xv[t].y, acc[r][t]);
                acc[r][t] = __builtin_fmaf(w.z, xv[t].z, acc[r][t]);
                acc[r][t] = __builtin_fmaf(w.w, xv[t].w, acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int row = r0 + r;
        if (row > E) continue;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            float s = wave_sum_canon(acc[r][t]);
            if (lane == 0 && t < nt) a.logits[(size_t)(t0 + t) * (E + 1) + row] = s;
        }
    }
}

/* Large-batch selection: one wave per token. */
template <int EPL>
__global__ __launch_bounds__(256) void k_topk(RouteArgs a) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    wave_topk<EPL>(a.logits + (size_t)t * (a.E + 1), a.bias, a.E, a.K, lane, a.idx + t * a.K,
                   a.w + t * a.K, a.sgl + t, nullptr);
}

/* Block-wide exclusive scan of three counters per expert (one thread per
 * expert, E <= DSP_THREADS), Hillis-Steele over LDS. */
#define DSP_THREADS 1024
DEV void block_scan3(uint32_t *a, uint32_t *b, uint32_t *c, int n) {
    const int tid = threadIdx.x;
    for (int off = 1; off < n; off <<= 1) {
        uint32_t va = 0, vb = 0, vc = 0;
        if (tid < n && tid >= off) { va = a[tid - off]; vb = b[tid - off]; vc = c[tid - off]; }
        __syncthreads();
        if (tid < n && tid >= off) { a[tid] += va; b[tid] += vb; c[tid] += vc; }
        __syncthreads();
    }
}

/* Dispatch for any T (one block of 1024 threads):
 *  1. LDS histogram of the T*K expert ids; block scans give the offsets, the
 *     active-expert ranks and the GEMM tile offsets.
 *  2. Stable scatter in chunks of 1024 tokens: each expert keeps a 1024-bit
 *     membership mask of the chunk's tokens, so a pair's rank inside its
 *     expert is the popcount of the mask below its token, plus the count
 *     carried from earlier chunks.
 *  3. Active-expert list and GEMM tile list (expert, first row, rows), tiles
 *     of tile_m rows; the shared expert (id E) covers tokens 0..T-1. */
__global__ __launch_bounds__(DSP_THREADS) void k_dispatch(RouteArgs a, uint32_t *tiles, int tile_m,
                                                          int has_shared) {
    extern __shared__ uint32_t lds[];
    const int E = a.E, K = a.K, T = a.T, tid = threadIdx.x;
    uint32_t *hist = lds;                   /* E */
    uint32_t *offs = hist + E;              /* E (inclusive scan of hist) */
    uint32_t *arank = offs + E;             /* E (inclusive scan of active) */
    uint32_t *toff = arank + E;             /* E (inclusive scan of tile counts) */
    uint32_t *cursor = toff + E;            /* E */
    uint32_t *mask = cursor + E;            /* E * 32 */
    uint32_t *wpre = mask + (size_t)E * 32; /* E * 32 */
    for (int e = tid; e < E; e += DSP_THREADS) { hist[e] = 0; cursor[e] = 0; }
    __syncthreads();
    for (int p = tid; p < T * K; p += DSP_THREADS) atomicAdd(&hist[a.idx[p]], 1u);
    __syncthreads();
    if (tid < E) {
        offs[tid] = hist[tid];
        arank[tid] = hist[tid] != 0;
        toff[tid] = (hist[tid] + tile_m - 1) / tile_m;
    }
    __syncthreads();
    block_scan3(offs, arank, toff, E);
    /* inclusive -> exclusive views: ex(x)[e] = x[e] - own */
    if (tid < E) {
        const uint32_t c = hist[tid];
        const uint32_t o = offs[tid] - c;
        a.offsets[tid] = o;
        if (c) {
            const uint32_t r = arank[tid] - 1;
            ACT_E(a.list, r) = (uint32_t)tid;
            ACT_OFF(a.list, E, r) = o;
            const uint32_t nt = (c + tile_m - 1) / tile_m, t0 = toff[tid] - nt;
            for (uint32_t j = 0; j < nt; j++) {
                tiles[1 + 3 * (t0 + j)] = (uint32_t)tid;
                tiles[2 + 3 * (t0 + j)] = o + j * tile_m;
                tiles[3 + 3 * (t0 + j)] = min((uint32_t)tile_m, c - j * tile_m);
            }
        }
    }
    if (tid == 0) {
        const uint32_t n_act = arank[E - 1], nt = toff[E - 1];
        a.offsets[E] = offs[E - 1];
        ACT_N(a.list) = n_act;
        ACT_OFF(a.list, E, n_act) = offs[E - 1];
        const uint32_t nsh = has_shared ? (uint32_t)((T + tile_m - 1) / tile_m) : 0;
        tiles[0] = nt + nsh;
    }
    if (has_shared) {
        const uint32_t nt = toff[E - 1];
        for (int j = tid; j * tile_m < T; j += DSP_THREADS) {
            tiles[1 + 3 * (nt + j)] = (uint32_t)E;
            tiles[2 + 3 * (nt + j)] = (uint32_t)(j * tile_m);
            tiles[3 + 3 * (nt + j)] = (uint32_t)min(tile_m, T - j * tile_m);
        }
    }
    for (int base = 0; base < T; base += 1024) {
        for (int i = tid; i < E * 32; i += DSP_THREADS) mask[i] = 0;
        __syncthreads();
        const int t = base + tid;
        const bool live = t < T;
        int ek[OROME_MAXK];
#pragma unroll
        for (int k = 0; k < OROME_MAXK; k++)
            if (k < K) ek[k] = live ? a.idx[t * K + k] : 0;
        if (live)
#pragma unroll
            for (int k = 0; k < OROME_MAXK; k++)
                if (k < K) atomicOr(&mask[ek[k] * 32 + (tid >> 5)], 1u << (tid & 31));
        __syncthreads();
        for (int i = tid; i < E * 32; i += DSP_THREADS) {
            /* prefix popcount over the 32 words of one expert: word w of
             * expert e sums words 0..w-1 (32 lanes of a wave share e) */
            const int e = i >> 5, w = i & 31;
            uint32_t s = 0;
            for (int v = 0; v < w; v++) s += __popc(mask[e * 32 + v]);
            wpre[i] = s;
        }
        __syncthreads();
        if (live)
#pragma unroll
            for (int k = 0; k < OROME_MAXK; k++)
                if (k < K) {
                    const int e = ek[k];
                    const uint32_t wd = mask[e * 32 + (tid >> 5)];
                    const uint32_t rank = cursor[e] + wpre[e * 32 + (tid >> 5)] + __popc(wd & ((1u << (tid & 31)) - 1u));
                    const uint32_t pos = offs[e] - hist[e] + rank;
                    const uint32_t p = (uint32_t)(t * K + k);
                    a.pairs[pos] = p;
                    a.pos[p] = pos;
                }
        __syncthreads();
        for (int e = tid; e < E; e += DSP_THREADS)
            cursor[e] += wpre[e * 32 + 31] + __popc(mask[e * 32 + 31]);
        __syncthreads();
    }
}

/* RMSNorm (inference/src/shaders.metal:128-149) with the canonical sum of
 * squares: x = (h * (1 / sqrt(ss/H + eps))) * bf16(w); one wave per token. */
__global__ __launch_bounds__(64) void k_rmsnorm(const float *h, const float *w, int H, float eps,
                                                float *x) {
    const int lane = threadIdx.x, t = blockIdx.x;
    const float *ht = h + (size_t)t * H;
    const int NI = H / 256;
    f4 v[CANON_NI];
#pragma unroll
    for (int i = 0; i < CANON_NI; i++)
        if (i < NI) v[i] = *(const f4 *)(ht + 256 * i + 4 * lane);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CANON_NI; i++)
        if (i < NI) {
            acc = __builtin_fmaf(v[i].x, v[i].x, acc);
            acc = __builtin_fmaf(v[i].y, v[i].y, acc);
            acc = __builtin_fmaf(v[i].z, v[i].z, acc);
            acc = __builtin_fmaf(v[i].w, v[i].w, acc);
        }
    float ss = wave_sum_canon(acc);
    /* sqrtf and / lower to correctly rounded sequences (__fsqrt_rn does not) */
    float scale = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
    for (int i = 0; i < CANON_NI; i++)
        if (i < NI) {
            const int j = 256 * i + 4 * lane;
            f4 wv = w ? *(const f4 *)(w + j) : f4{1, 1, 1, 1};
            f4 o;
            o.x = (v[i].x * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wv.x) & 0xFFFF0000u);
            o.y = (v[i].y * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wv.y) & 0xFFFF0000u);
            o.z = (v[i].z * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wv.z) & 0xFFFF0000u);
            o.w = (v[i].w * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wv.w) & 0xFFFF0000u);
            *(f4 *)(x + (size_t)t * H + j) = o;
        }
}

/* ------------------------------------------------------------ launch */
static int epl_for(int E) {
    if (E <= 64) return 1;
    if (E <= 128) return 2;
    if (E <= 256) return 4;
    if (E <= 512) return 8;
    if (E <= 1024) return 16;
    return 0;
}

#define EPL_SWITCH(E, KERNEL, ...)                                        \
    switch (epl_for(E)) {                                                 \
        case 1: hipLaunchKernelGGL(KERNEL<1>, __VA_ARGS__); break;        \
        case 2: hipLaunchKernelGGL(KERNEL<2>, __VA_ARGS__); break;        \
        case 4: hipLaunchKernelGGL(KERNEL<4>, __VA_ARGS__); break;        \
        case 8: hipLaunchKernelGGL(KERNEL<8>, __VA_ARGS__); break;        \
        case 16: hipLaunchKernelGGL(KERNEL<16>, __VA_ARGS__); break;      \
        default: return -2;                                               \
    }

int launch_route_small(const RouteArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T > 16 || a.T * a.K > 256 || a.H % 256 || a.H > 4096) return -2;
    hipLaunchKernelGGL(k_route_small, dim3((a.E + 1 + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk_dispatch_small(const RouteArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T * a.K > 256) return -2;
    EPL_SWITCH(a.E, k_topk_dispatch_small, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_route_logits(const RouteArgs &a, hipStream_t s) {
    if (a.H % 256) return -2;
    dim3 grid((a.E + 1 + 15) / 16, (a.T + 7) / 8);
    hipLaunchKernelGGL(k_route_logits, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk(const RouteArgs &a, hipStream_t s) {
    dim3 grid((a.T + 3) / 4);
    EPL_SWITCH(a.E, k_topk, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_dispatch(const RouteArgs &a, uint32_t *tiles, int tile_m, int has_shared, hipStream_t s) {
    size_t lds = sizeof(uint32_t) * ((size_t)a.E * 5 + (size_t)a.E * 64);
    if (lds > 160 * 1024 || a.E > DSP_THREADS) return -2;
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DSP_THREADS), lds, s, a, tiles, tile_m, has_shared);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x, hipStream_t s) {
    if (H % 256 || H > 256 * CANON_NI) return -2;
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(64), 0, s, h, w, H, eps, x);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
