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

/* canonical dot of one wave over H (H % 256 == 0, H <= 256 CANON_NI), for
 * up to TMAX tokens; all loads of a row are issued before the multiply-adds */
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

/* As canon_dots, with x = RMSNorm(h) computed in place (RMSNorm of
 * inference/src/shaders.metal:128-149, the same arithmetic and canonical sum
 * of squares as k_rmsnorm, so x is bit-identical to that kernel's output);
 * write_x stores x for the later kernels. */
template <int TMAX>
DEV void canon_dots_norm(const float *wrow, const RouteArgs &a, int lane, bool write_x, float *acc) {
    const int NI = a.H / 256, H = a.H, T = a.T;
    f4 wv[CANON_NI], nw[CANON_NI];
#pragma unroll
    for (int i = 0; i < CANON_NI; i++)
        if (i < NI) {
            wv[i] = wrow ? *(const f4 *)(wrow + 256 * i + 4 * lane) : f4{0, 0, 0, 0};
            const f4 w = a.norm_w ? *(const f4 *)(a.norm_w + 256 * i + 4 * lane) : f4{1, 1, 1, 1};
            nw[i] = f4{__builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.x) & 0xFFFF0000u),
                       __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.y) & 0xFFFF0000u),
                       __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.z) & 0xFFFF0000u),
                       __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.w) & 0xFFFF0000u)};
        }
#pragma unroll
    for (int t = 0; t < TMAX; t++) {
        acc[t] = 0.0f;
        if (t < T) {
            f4 hv[CANON_NI];
#pragma unroll
            for (int i = 0; i < CANON_NI; i++)
                if (i < NI) hv[i] = *(const f4 *)(a.norm_h + (size_t)t * H + 256 * i + 4 * lane);
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < CANON_NI; i++)
                if (i < NI) {
                    ss = __builtin_fmaf(hv[i].x, hv[i].x, ss);
                    ss = __builtin_fmaf(hv[i].y, hv[i].y, ss);
                    ss = __builtin_fmaf(hv[i].z, hv[i].z, ss);
                    ss = __builtin_fmaf(hv[i].w, hv[i].w, ss);
                }
            ss = wave_sum_canon(ss);
            const float scale = 1.0f / sqrtf(ss / (float)H + a.norm_eps);
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < CANON_NI; i++)
                if (i < NI) {
                    const f4 x = {(hv[i].x * scale) * nw[i].x, (hv[i].y * scale) * nw[i].y,
                                  (hv[i].z * scale) * nw[i].z, (hv[i].w * scale) * nw[i].w};
                    if (write_x) *(f4 *)(a.xnorm + (size_t)t * H + 256 * i + 4 * lane) = x;
                    d = __builtin_fmaf(wv[i].x, x.x, d);
                    d = __builtin_fmaf(wv[i].y, x.y, d);
                    d = __builtin_fmaf(wv[i].z, x.z, d);
                    d = __builtin_fmaf(wv[i].w, x.w, d);
                }
            acc[t] = wave_sum_canon(d);
        }
    }
}

/* Small-batch router logits (T <= 16): every wave computes one router row
 * (or the shared-gate row) for all tokens; with NORM, x is RMSNorm(norm_h)
 * and the row-0 wave also writes it out. */
template <bool NORM>
__global__ __launch_bounds__(256) void k_route_small(RouteArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    const int E = a.E, H = a.H, T = a.T;
    if (row > E) return;
    const float *wr = row < E ? a.W + (size_t)row * H : a.wsg;
    float acc[16];
    if (NORM) {
        canon_dots_norm<16>(wr, a, lane, row == 0, acc);
    } else if (wr) {
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

/* Large-batch router logits: a block computes 32 rows (expert rows, then the
 * shared-gate row E) x 8 tokens, so the 2 MB router matrix is what gets
 * re-read (from L2) rather than the activations; each wave 8 rows x 8
 * tokens, lane L
 * accumulating k = 256 i + 4 L + c in (i, c) order with fma from zero. */
__global__ __launch_bounds__(256) void k_route_logits(RouteArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int E = a.E, H = a.H, T = a.T;
    const int r0 = blockIdx.x * 32 + wv * 8, t0 = blockIdx.y * 8;
    const float *wr[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int row = r0 + r;
        wr[r] = row < E ? a.W + (size_t)row * H : (row == E ? a.wsg : nullptr);
    }
    const int nt = min(8, T - t0);
    float acc[64]; /* output o = 8 r + t */
#pragma unroll
    for (int o = 0; o < 64; o++) acc[o] = 0.0f;
    for (int i = 0; i < H / 256; i++) {
        f4 xv[8];
#pragma unroll
        for (int t = 0; t < 8; t++)
            xv[t] = t < nt ? *(const f4 *)(a.x + (size_t)(t0 + t) * H + 256 * i + 4 * lane) : f4{0, 0, 0, 0};
        /* the first row group's blocks also stage x as fp16 for the grouped
         * GEMMs (round to nearest even, each 4-group stored (0,2,1,3)): wave
         * wv writes tokens wv and wv + 4 */
        if (a.x16 && blockIdx.x == 0) {
#pragma unroll
            for (int t = 0; t < 8; t++)
                if ((t & 3) == wv && t < nt)
                    *(h4 *)(a.x16 + (size_t)(t0 + t) * H + 256 * i + 4 * lane) =
                        h4{(_Float16)xv[t].x, (_Float16)xv[t].z, (_Float16)xv[t].y, (_Float16)xv[t].w};
        }
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const f4 w = wr[r] ? *(const f4 *)(wr[r] + 256 * i + 4 * lane) : f4{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                float &c = acc[8 * r + t];
                c = __builtin_fmaf(w.x, xv[t].x, c);
                c = __builtin_fmaf(w.y, xv[t].y, c);
                c = __builtin_fmaf(w.z, xv[t].z, c);
                c = __builtin_fmaf(w.w, xv[t].w, c);
            }
        }
    }
    /* Butterfly reduce-scatter over the 64 lanes: at stage s lanes L and
     * L ^ 2^s add the partial sums of the half of their outputs that L keeps
     * (bit s of L picks the half).  Each add joins the subtree sums of lanes
     * [L0, L0 + 2^s) and [L0 + 2^s, L0 + 2^(s+1)), so every output is summed
     * in the canonical contiguous balanced tree; lane L ends with output
     * bitreverse6(L). */
#pragma unroll
    for (int st = 0; st < 6; st++) {
        const int half = 32 >> st;
        const bool hi = (lane >> st) & 1;
#pragma unroll
        for (int o = 0; o < half; o++) {
            const float send = hi ? acc[o] : acc[o + half];
            const float keep = hi ? acc[o + half] : acc[o];
            acc[o] = keep + __shfl_xor(send, 1 << st, 64);
        }
    }
    const int o = (int)(__builtin_bitreverse32((uint32_t)lane) >> 26);
    const int row = r0 + (o >> 3), tok = t0 + (o & 7);
    if (row <= E && tok < T) a.logits[(size_t)tok * (E + 1) + row] = acc[0];
}

/* Large-batch selection: one wave per token. */
template <int EPL>
__global__ __launch_bounds__(256) void k_topk(RouteArgs a) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    wave_topk<EPL>(a.logits + (size_t)t * (a.E + 1), a.bias, a.E, a.K, lane, a.idx + t * a.K,
                   a.w + t * a.K, a.sgl + t, nullptr);
}

/* Dispatch for any T, in three launches over blocks of DSP_TOK tokens.  A
 * pair p = t*K + k goes to position offsets[e] + (number of earlier tokens
 * that picked e): a stable counting sort by expert (tokens pick distinct
 * experts, so token order is pair order inside an expert).
 *  1. count:   per block, an LDS token-membership mask per expert
 *              (DSP_TOK bits) and its popcount -> cnt[block][e].
 *  2. scan:    one block: per expert an exclusive scan of cnt over blocks
 *              (in place) and the total; block scans of the totals give the
 *              offsets, active-expert ranks and GEMM tile offsets; then the
 *              active list and two GEMM tile lists (expert, first row, rows):
 *              experts with <= GEMM_TILE_SMALL rows get one small tile, the
 *              others tiles of GEMM_TILE_BIG rows; the shared expert (id E)
 *              covers tokens 0..T-1 in small tiles when the average expert
 *              has <= GEMM_TILE_SMALL rows, else in big ones.
 *  3. scatter: per block, the same masks; a pair's rank is its expert's
 *              offset + the block's base + the popcount of the mask below
 *              its token. */
#define DSP_TOK 256
#define DSP_WORDS (DSP_TOK / 32)
#define DSP_THREADS 1024

DEV void dispatch_masks(const RouteArgs &a, uint32_t *mask, int ek[OROME_MAXK]) {
    const int E = a.E, K = a.K, tid = threadIdx.x, t = blockIdx.x * DSP_TOK + tid;
    for (int i = tid; i < E * DSP_WORDS; i += DSP_TOK) mask[i] = 0;
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++)
        if (k < K) ek[k] = t < a.T ? a.idx[t * K + k] : -1;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++)
        if (k < K && ek[k] >= 0) atomicOr(&mask[ek[k] * DSP_WORDS + (tid >> 5)], 1u << (tid & 31));
    __syncthreads();
}

__global__ __launch_bounds__(DSP_TOK) void k_dispatch_count(RouteArgs a, uint32_t *cnt) {
    extern __shared__ uint32_t mask[]; /* E * DSP_WORDS */
    int ek[OROME_MAXK];
    dispatch_masks(a, mask, ek);
    for (int e = threadIdx.x; e < a.E; e += DSP_TOK) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < DSP_WORDS; w++) c += __popc(mask[e * DSP_WORDS + w]);
        cnt[(size_t)blockIdx.x * a.E + e] = c;
    }
}

/* Block-wide inclusive scan of four counters per expert (one thread per
 * expert, E <= DSP_THREADS), Hillis-Steele over LDS. */
DEV void block_scan4(uint32_t *a, uint32_t *b, uint32_t *c, uint32_t *d, int n) {
    const int tid = threadIdx.x;
    for (int off = 1; off < n; off <<= 1) {
        uint32_t va = 0, vb = 0, vc = 0, vd = 0;
        if (tid < n && tid >= off) { va = a[tid - off]; vb = b[tid - off]; vc = c[tid - off]; vd = d[tid - off]; }
        __syncthreads();
        if (tid < n && tid >= off) { a[tid] += va; b[tid] += vb; c[tid] += vc; d[tid] += vd; }
        __syncthreads();
    }
}

/* Tiles of one expert: rows <= GEMM_TILE_SMALL -> one small tile, else
 * ceil(rows / GEMM_TILE_BIG) big tiles. */
DEV uint32_t n_small_tiles(uint32_t c) { return c != 0 && c <= GEMM_TILE_SMALL; }
DEV uint32_t n_big_tiles(uint32_t c) { return c > GEMM_TILE_SMALL ? (c + GEMM_TILE_BIG - 1) / GEMM_TILE_BIG : 0; }
DEV void put_tiles(uint32_t *list, uint32_t t0, uint32_t e, uint32_t first, uint32_t c, uint32_t tm) {
    for (uint32_t j = 0; j * tm < c; j++) {
        list[1 + 3 * (t0 + j)] = e;
        list[2 + 3 * (t0 + j)] = first + j * tm;
        list[3 + 3 * (t0 + j)] = min(tm, c - j * tm);
    }
}

/* Given per-expert counts (hist, copied into offs), and offs/arank/ts/tbg
 * filled with the counts, active flags and tile counts: scans them and
 * writes offsets, the active list and the two GEMM tile lists (E <=
 * blockDim.x; every thread of the block calls it). */
DEV void dispatch_lists(const RouteArgs &a, const uint32_t *hist, uint32_t *offs, uint32_t *arank, uint32_t *ts,
                        uint32_t *tbg, uint32_t *tiles_s, uint32_t *tiles_b, int has_shared) {
    const int E = a.E, T = a.T, tid = threadIdx.x;
    block_scan4(offs, arank, ts, tbg, E);
    /* inclusive -> exclusive views: ex(x)[e] = x[e] - own */
    if (tid < E) {
        const uint32_t c = hist[tid];
        const uint32_t o = offs[tid] - c;
        a.offsets[tid] = o;
        if (c) {
            const uint32_t r = arank[tid] - 1;
            ACT_E(a.list, r) = (uint32_t)tid;
            ACT_OFF(a.list, E, r) = o;
            if (c <= GEMM_TILE_SMALL) put_tiles(tiles_s, ts[tid] - 1, (uint32_t)tid, o, c, GEMM_TILE_SMALL);
            else put_tiles(tiles_b, tbg[tid] - n_big_tiles(c), (uint32_t)tid, o, c, GEMM_TILE_BIG);
        }
    }
    if (tid == 0) {
        const uint32_t n_act = arank[E - 1], ns = ts[E - 1], nb = tbg[E - 1], Tu = (uint32_t)T;
        a.offsets[E] = offs[E - 1];
        ACT_N(a.list) = n_act;
        ACT_OFF(a.list, E, n_act) = offs[E - 1];
        /* the shared expert (id E) over tokens 0..T-1, in the list that holds
         * most of the routed work (a lone list of shared tiles would run as
         * a tail after the other launch) */
        const bool sm = (size_t)T * a.K <= (size_t)GEMM_TILE_SMALL * E;
        const uint32_t tm = sm ? GEMM_TILE_SMALL : GEMM_TILE_BIG, nsh = has_shared ? (Tu + tm - 1) / tm : 0;
        if (has_shared) put_tiles(sm ? tiles_s : tiles_b, sm ? ns : nb, (uint32_t)E, 0, Tu, tm);
        tiles_s[0] = ns + (sm ? nsh : 0);
        tiles_b[0] = nb + (sm ? 0 : nsh);
    }
}

__global__ __launch_bounds__(DSP_THREADS) void k_dispatch_scan(RouteArgs a, uint32_t *cnt, int G,
                                                               uint32_t *tiles_s, uint32_t *tiles_b,
                                                               int has_shared) {
    __shared__ uint32_t hist[DSP_THREADS], offs[DSP_THREADS], arank[DSP_THREADS], ts[DSP_THREADS],
        tbg[DSP_THREADS];
    const int E = a.E, T = a.T, tid = threadIdx.x;
    if (tid < E) {
        uint32_t run = 0;
        for (int g = 0; g < G; g++) {
            const uint32_t c = cnt[(size_t)g * E + tid];
            cnt[(size_t)g * E + tid] = run;
            run += c;
        }
        hist[tid] = run;
        offs[tid] = run;
        arank[tid] = run != 0;
        ts[tid] = n_small_tiles(run);
        tbg[tid] = n_big_tiles(run);
    }
    __syncthreads();
    dispatch_lists(a, hist, offs, arank, ts, tbg, tiles_s, tiles_b, has_shared);
}

__global__ __launch_bounds__(DSP_TOK) void k_dispatch_scatter(RouteArgs a, const uint32_t *base) {
    extern __shared__ uint32_t mask[]; /* E * DSP_WORDS, then E * DSP_WORDS word prefixes */
    uint32_t *wpre = mask + a.E * DSP_WORDS;
    int ek[OROME_MAXK];
    dispatch_masks(a, mask, ek);
    const int E = a.E, K = a.K, tid = threadIdx.x, t = blockIdx.x * DSP_TOK + tid;
    for (int e = tid; e < E; e += DSP_TOK) {
        uint32_t run = a.offsets[e] + base[(size_t)blockIdx.x * E + e];
#pragma unroll
        for (int w = 0; w < DSP_WORDS; w++) {
            wpre[e * DSP_WORDS + w] = run;
            run += __popc(mask[e * DSP_WORDS + w]);
        }
    }
    __syncthreads();
    const uint32_t below = (1u << (tid & 31)) - 1u;
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++)
        if (k < K && ek[k] >= 0) {
            const int i = ek[k] * DSP_WORDS + (tid >> 5);
            const uint32_t pos = wpre[i] + __popc(mask[i] & below);
            const uint32_t p = (uint32_t)(t * K + k);
            a.pairs[pos] = p;
            a.pos[p] = pos;
        }
}

/* The same dispatch in one block for T <= DSP_THREADS tokens (one launch
 * instead of three; the positions are identical): thread t sets its pairs'
 * bits in the membership masks of its DSP_TOK-token sub-chunk; an expert's
 * count is the popcount of its masks; offsets and lists follow as in
 * k_dispatch_scan; a pair's position is its expert's offset + the counts of
 * earlier sub-chunks + the popcount of its sub-chunk's mask below its token.
 * LDS: masks and word prefixes for DSP1_SUB sub-chunks of up to 256 experts. */
#define DSP1_SUB (DSP_THREADS / DSP_TOK)
__global__ __launch_bounds__(DSP_THREADS) void k_dispatch_one(RouteArgs a, uint32_t *tiles_s, uint32_t *tiles_b,
                                                              int has_shared) {
    __shared__ uint32_t hist[DSP_THREADS], offs[DSP_THREADS], arank[DSP_THREADS], ts[DSP_THREADS],
        tbg[DSP_THREADS];
    __shared__ uint32_t mask[DSP1_SUB * 256 * DSP_WORDS], wpre[DSP1_SUB * 256 * DSP_WORDS];
    const int E = a.E, K = a.K, T = a.T, tid = threadIdx.x;
    const int sub = tid / DSP_TOK, tl = tid % DSP_TOK;
    for (int i = tid; i < DSP1_SUB * E * DSP_WORDS; i += DSP_THREADS) mask[i] = 0;
    __syncthreads();
    int ek[OROME_MAXK];
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++)
        if (k < K) {
            ek[k] = tid < T ? a.idx[tid * K + k] : -1;
            if (ek[k] >= 0) atomicOr(&mask[(sub * E + ek[k]) * DSP_WORDS + (tl >> 5)], 1u << (tl & 31));
        }
    __syncthreads();
    if (tid < E) { /* word prefixes from 0, and the expert's count */
        uint32_t run = 0;
        for (int sc = 0; sc < DSP1_SUB; sc++)
#pragma unroll
            for (int w = 0; w < DSP_WORDS; w++) {
                const int i = (sc * E + tid) * DSP_WORDS + w;
                wpre[i] = run;
                run += __popc(mask[i]);
            }
        hist[tid] = run;
        offs[tid] = run;
        arank[tid] = run != 0;
        ts[tid] = n_small_tiles(run);
        tbg[tid] = n_big_tiles(run);
    }
    __syncthreads();
    dispatch_lists(a, hist, offs, arank, ts, tbg, tiles_s, tiles_b, has_shared);
    __syncthreads();
    const uint32_t below = (1u << (tl & 31)) - 1u;
#pragma unroll
    for (int k = 0; k < OROME_MAXK; k++)
        if (k < K && ek[k] >= 0) {
            const int e = ek[k], i = (sub * E + e) * DSP_WORDS + (tl >> 5);
            const uint32_t pos = offs[e] - hist[e] + wpre[i] + __popc(mask[i] & below);
            const uint32_t p = (uint32_t)(tid * K + k);
            a.pairs[pos] = p;
            a.pos[p] = pos;
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
    if (a.norm_h) hipLaunchKernelGGL(k_route_small<true>, dim3((a.E + 1 + 3) / 4), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_route_small<false>, dim3((a.E + 1 + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk_dispatch_small(const RouteArgs &a, hipStream_t s) {
    if (a.T < 1 || a.T * a.K > 256) return -2;
    EPL_SWITCH(a.E, k_topk_dispatch_small, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_route_logits(const RouteArgs &a, hipStream_t s) {
    if (a.H % 256) return -2;
    dim3 grid((a.E + 1 + 31) / 32, (a.T + 7) / 8);
    hipLaunchKernelGGL(k_route_logits, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk(const RouteArgs &a, hipStream_t s) {
    dim3 grid((a.T + 3) / 4);
    EPL_SWITCH(a.E, k_topk, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int dispatch_blocks(int T) { return (T + DSP_TOK - 1) / DSP_TOK; }

int launch_dispatch(const RouteArgs &a, uint32_t *tiles_s, uint32_t *tiles_b, int has_shared, uint32_t *cnt,
                    hipStream_t s) {
    const size_t lds = sizeof(uint32_t) * (size_t)a.E * DSP_WORDS * 2;
    if (lds > 64 * 1024 || a.E > DSP_THREADS || a.K > OROME_MAXK) return -2;
#ifndef DISPATCH_ONE
#define DISPATCH_ONE 1
#endif
    if (DISPATCH_ONE && a.E <= 256 && a.T <= DSP_THREADS) {
        hipLaunchKernelGGL(k_dispatch_one, dim3(1), dim3(DSP_THREADS), 0, s, a, tiles_s, tiles_b, has_shared);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const int G = dispatch_blocks(a.T);
    hipLaunchKernelGGL(k_dispatch_count, dim3(G), dim3(DSP_TOK), lds / 2, s, a, cnt);
    hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(DSP_THREADS), 0, s, a, cnt, G, tiles_s, tiles_b, has_shared);
    hipLaunchKernelGGL(k_dispatch_scatter, dim3(G), dim3(DSP_TOK), lds, s, a, (const uint32_t *)cnt);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x, hipStream_t s) {
    if (H % 256 || H > 256 * CANON_NI) return -2;
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(64), 0, s, h, w, H, eps, x);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
