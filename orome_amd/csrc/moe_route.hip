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

/* -------------------------------------------------------- key helpers */
DEV uint64_t route_key(float v, int e) {
    if (v == 0.0f) v = 0.0f; /* -0 and +0 tie by index, as in IEEE compare */
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}
DEV float key_value(uint64_t k) {
    uint32_t ord = (uint32_t)(k >> 32);
    uint32_t b = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    return __builtin_bit_cast(float, b);
}
DEV int key_expert(uint64_t k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

template <int CTRL>
DEV uint64_t dpp64(uint64_t v) {
    return ((uint64_t)dppu<CTRL>((uint32_t)(v >> 32)) << 32) | dppu<CTRL>((uint32_t)v);
}
DEV uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
DEV uint64_t readlane64(uint64_t v, int l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), l) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
}
/* wave64 maximum of a 64-bit key (DPP within rows, then the four row maxima) */
DEV uint64_t wave_max64(uint64_t m) {
    m = max64(m, dpp64<DPP_XOR1>(m));
    m = max64(m, dpp64<DPP_XOR2>(m));
    m = max64(m, dpp64<DPP_HALF_MIRROR>(m));
    m = max64(m, dpp64<DPP_MIRROR>(m));
    return max64(max64(readlane64(m, 0), readlane64(m, 16)), max64(readlane64(m, 32), readlane64(m, 48)));
}

/* One token's top-K on one wave.  Lane 0 writes idx/w/sgl; e_out (LDS, may be
 * NULL) receives the K expert ids. */
template <int EPL>
DEV void wave_topk(const float *l, const float *bias, int E, int K, int lane, int32_t *idx_out,
                   float *w_out, float *sgl_out, int *e_out) {
    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        int e = lane + 64 * j;
        key[j] = 0;
        if (e < E) {
            float v = l[e];
            if (bias) v = v + bias[e];
            key[j] = route_key(v, e);
        }
    }
    float vals[OROME_MAXK];
    int ids[OROME_MAXK];
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++) {
        if (k < K) {
            uint64_t m = key[0];
#pragma unroll
            for (int j = 1; j < EPL; j++) m = key[j] > m ? key[j] : m;
            m = wave_max64(m);
#pragma unroll
            for (int j = 0; j < EPL; j++)
                if (key[j] == m) key[j] = 0;
            vals[k] = key_value(m);
            ids[k] = key_expert(m);
        }
    }
    if (lane == 0) {
        float mx = vals[0], sum = 0.0f, tw[OROME_MAXK];
#pragma unroll
        for (int k = 0; k < OROME_MAXK; k++)
            if (k < K) {
                tw[k] = expf(vals[k] - mx);
                sum += tw[k];
            }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
        for (int k = 0; k < OROME_MAXK; k++)
            if (k < K) {
                idx_out[k] = ids[k];
                w_out[k] = tw[k] * inv;
                if (e_out) e_out[k] = ids[k];
            }
        *sgl_out = l[E];
    }
}

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

/* Small-batch selection and dispatch (T*K <= 256), one block: a wave per
 * token for the top-k, then the stable counting sort of the T*K pairs by
 * ranking each pair against all others. */
template <int EPL>
__global__ __launch_bounds__(256) void k_topk_dispatch_small(RouteArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int E = a.E, T = a.T, K = a.K;
    __shared__ int s_e[256];
    __shared__ int s_head[256];
    for (int t = wv; t < T; t += 4)
        wave_topk<EPL>(a.logits + (size_t)t * (E + 1), a.bias, E, K, lane, a.idx + t * K, a.w + t * K,
                       a.sgl + t, s_e + t * K);
    __syncthreads();
    const int NP = T * K, p = threadIdx.x;
    int e = 0, less = 0, before = 0;
    if (p < NP) {
        e = s_e[p];
        for (int q = 0; q < NP; q++) {
            int eq = s_e[q];
            less += eq < e;
            before += (q < p) & (eq == e);
        }
        uint32_t pos = (uint32_t)(less + before);
        a.pairs[pos] = (uint32_t)p;
        a.pos[p] = pos;
        s_head[p] = before == 0;
    }
    __syncthreads();
    if (p < NP && s_head[p]) {
        int rank = 0;
        for (int q = 0; q < NP; q++) rank += s_head[q] & (s_e[q] < e);
        ACT_E(a.list, rank) = (uint32_t)e;
        ACT_OFF(a.list, E, rank) = (uint32_t)less;
    }
    if (threadIdx.x == 0) {
        int n = 0;
        for (int q = 0; q < NP; q++) n += s_head[q];
        ACT_N(a.list) = (uint32_t)n;
        ACT_OFF(a.list, E, n) = (uint32_t)NP;
    }
    for (int ee = threadIdx.x; ee <= E; ee += 256) {
        int c = 0;
        for (int q = 0; q < NP; q++) c += s_e[q] < ee;
        a.offsets[ee] = (uint32_t)c;
    }
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

/* Dispatch for any T (one block of 1024 threads):
 *  1. LDS histogram of the T*K expert ids; exclusive scan -> offsets.
 *  2. Stable scatter in chunks of 1024 tokens: each expert keeps a 1024-bit
 *     membership mask of the chunk's tokens, so a pair's rank inside its
 *     expert is the popcount of the mask below its token, plus the count
 *     carried from earlier chunks.
 *  3. Active-expert list and GEMM tile list (expert, first row, rows), tiles
 *     of GEMM_TILE_M rows; the shared expert (id E) covers tokens 0..T-1. */
#define DSP_THREADS 1024
__global__ __launch_bounds__(DSP_THREADS) void k_dispatch(RouteArgs a, uint32_t *tiles, int tile_m,
                                                          int has_shared) {
    extern __shared__ uint32_t lds[];
    const int E = a.E, K = a.K, T = a.T, tid = threadIdx.x;
    uint32_t *hist = lds;                  /* E */
    uint32_t *offs = hist + E;             /* E+1 */
    uint32_t *cursor = offs + E + 1;       /* E */
    uint32_t *mask = cursor + E;           /* E * 32 */
    uint32_t *wpre = mask + (size_t)E * 32; /* E * 32 */
    for (int e = tid; e < E; e += DSP_THREADS) { hist[e] = 0; cursor[e] = 0; }
    __syncthreads();
    for (int p = tid; p < T * K; p += DSP_THREADS) atomicAdd(&hist[a.idx[p]], 1u);
    __syncthreads();
    if (tid == 0) {
        uint32_t s = 0;
        for (int e = 0; e < E; e++) {
            offs[e] = s;
            s += hist[e];
        }
        offs[E] = s;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += DSP_THREADS) a.offsets[e] = offs[e];
    for (int base = 0; base < T; base += 1024) {
        for (int i = tid; i < E * 32; i += DSP_THREADS) mask[i] = 0;
        __syncthreads();
        const int t = base + tid;
        const bool live = t < T;
        if (live)
            for (int k = 0; k < K; k++) {
                int e = a.idx[t * K + k];
                atomicOr(&mask[e * 32 + (tid >> 5)], 1u << (tid & 31));
            }
        __syncthreads();
        for (int e = tid; e < E; e += DSP_THREADS) {
            uint32_t s = 0;
            for (int w = 0; w < 32; w++) {
                wpre[e * 32 + w] = s;
                s += __popc(mask[e * 32 + w]);
            }
        }
        __syncthreads();
        if (live)
            for (int k = 0; k < K; k++) {
                int e = a.idx[t * K + k];
                uint32_t wd = mask[e * 32 + (tid >> 5)];
                uint32_t rank = cursor[e] + wpre[e * 32 + (tid >> 5)] + __popc(wd & ((1u << (tid & 31)) - 1u));
                uint32_t pos = offs[e] + rank;
                uint32_t p = (uint32_t)(t * K + k);
                a.pairs[pos] = p;
                a.pos[p] = pos;
            }
        __syncthreads();
        for (int e = tid; e < E; e += DSP_THREADS)
            cursor[e] += wpre[e * 32 + 31] + __popc(mask[e * 32 + 31]);
        __syncthreads();
    }
    if (tid == 0) {
        uint32_t n = 0, nt = 0;
        for (int e = 0; e < E; e++) {
            uint32_t c = hist[e];
            if (!c) continue;
            ACT_E(a.list, n) = (uint32_t)e;
            ACT_OFF(a.list, E, n) = offs[e];
            n++;
            for (uint32_t r = 0; r < c; r += (uint32_t)tile_m) {
                tiles[1 + 3 * nt] = (uint32_t)e;
                tiles[2 + 3 * nt] = offs[e] + r;
                tiles[3 + 3 * nt] = min((uint32_t)tile_m, c - r);
                nt++;
            }
        }
        ACT_N(a.list) = n;
        ACT_OFF(a.list, E, n) = offs[E];
        if (has_shared)
            for (int r = 0; r < T; r += tile_m) {
                tiles[1 + 3 * nt] = (uint32_t)E;
                tiles[2 + 3 * nt] = (uint32_t)r;
                tiles[3 + 3 * nt] = (uint32_t)min(tile_m, T - r);
                nt++;
            }
        tiles[0] = nt;
    }
}

/* RMSNorm (inference/src/shaders.metal:128-149) with the canonical sum of
 * squares: x = (h * (1 / sqrt(ss/H + eps))) * bf16(w); one wave per token. */
__global__ __launch_bounds__(64) void k_rmsnorm(const float *h, const float *w, int H, float eps,
                                                float *x) {
    const int lane = threadIdx.x, t = blockIdx.x;
    const float *ht = h + (size_t)t * H;
    float acc = 0.0f;
    for (int i = 0; i < H / 256; i++) {
        f4 v = *(const f4 *)(ht + 256 * i + 4 * lane);
        acc = __builtin_fmaf(v.x, v.x, acc);
        acc = __builtin_fmaf(v.y, v.y, acc);
        acc = __builtin_fmaf(v.z, v.z, acc);
        acc = __builtin_fmaf(v.w, v.w, acc);
    }
    float ss = wave_sum_canon(acc);
    /* sqrtf and / lower to correctly rounded sequences (__fsqrt_rn does not) */
    float scale = 1.0f / sqrtf(ss / (float)H + eps);
    for (int j = lane; j < H; j += 64) {
        float wj = w ? __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w[j]) & 0xFFFF0000u) : 1.0f;
        x[(size_t)t * H + j] = __fmul_rn(__fmul_rn(ht[j], scale), wj);
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
    size_t lds = sizeof(uint32_t) * ((size_t)a.E * 3 + 1 + (size_t)a.E * 64);
    if (lds > 160 * 1024) return -2;
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DSP_THREADS), lds, s, a, tiles, tile_m, has_shared);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x, hipStream_t s) {
    if (H % 256) return -2;
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(64), 0, s, h, w, H, eps, x);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
