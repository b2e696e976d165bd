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
 * of argmax, exact ties to the lower expert index (the contract's rule; the
 * reference's tree settles exact ties by tree position), softmax over the K
 * winners.
 * A round is a wave64 max over order-preserving 32-bit images of the values;
 * the lowest lane holding the maximum settles ties.
 * Dispatch is a stable counting sort of pairs p = t*K + k by expert.
 */
#include "dev_common.h"
#include "kernels.h"

#include "route_dev.h"

/* Small-batch router logits (T <= 16): every wave computes one router row
 * (or the shared-gate row) for all tokens; with NORM, x is RMSNorm(norm_h)
 * and the row-0 wave also writes it out. */
/* RS waves per row: wave h of a row takes tokens h TMAX .. h TMAX + TMAX - 1
 * (5..8 tokens: two waves of 4, 9..16: four, instead of one wave with
 * dependent 4-token chunks). */
/* FOLD (> 0: the EPL of the selection): the block that finishes last also
 * runs the top-k and the dispatch for every token (topk_dispatch_block),
 * which saves a launch.  The logits cross blocks through a release/acquire
 * pair on a.counter (agent scope), stored and loaded as agent-scope atomics;
 * the last block returns the counter to zero for the next launch. */
template <bool NORM, int TMAX, int NIM, int RS, int FOLD>
__global__ __launch_bounds__(FOLD ? 512 : 256) void k_route_small(RouteArgs a) {
    /* the arguments in one round of scalar loads at entry (left alone, the
     * router rows' address came two dependent rounds after the first) */
    asm volatile("" ::"s"(a.W), "s"(a.wsg), "s"(a.bias), "s"(a.x), "s"(a.T), "s"(a.E), "s"(a.H), "s"(a.K),
                 "s"(a.logits), "s"(a.x16), "s"(a.norm_h), "s"(a.norm_w), "s"(a.norm_eps), "s"(a.xnorm),
                 "s"(gridDim.x));
    constexpr int W = FOLD ? 8 : 4; /* waves: the folding block selects with 8 */
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * (W / RS) + wv / RS, tb = (wv % RS) * TMAX;
    const int E = a.E, H = a.H, T = a.T;
    if (TMAX == 1 && !FOLD && H <= 2048) {
        /* one token: the block stages x once in LDS for its four rows */
        __shared__ f4 xl[512];
        const float *src = NORM ? a.norm_h : a.x;
        const int q = threadIdx.x;
        const f4 xp[2] = {*(const f4 *)(src + 4 * min(q, H / 4 - 1)), *(const f4 *)(src + 4 * min(q + 256, H / 4 - 1))};
        const bool live = row <= E;
        const float *wr = !live ? nullptr : row < E ? a.W + (size_t)row * H : a.wsg;
        float acc[TMAX];
        canon_dots<TMAX, NIM, NORM>(wr, a, lane, (NORM || a.x16) && row == 0, acc, 0, xl, xp);
        if (live && lane == 0) a.logits[row] = acc[0];
        return;
    }
    if (row <= E && tb < T) {
        const float *wr = row < E ? a.W + (size_t)row * H : a.wsg;
        float acc[TMAX];
        canon_dots<TMAX, NIM, NORM>(wr, a, lane, (NORM || a.x16) && row == 0, acc, tb);
        if (lane == 0) {
#pragma unroll
            for (int t = 0; t < TMAX; t++)
                if (tb + t < T) {
                    float *o = a.logits + (size_t)(tb + t) * (E + 1) + row;
                    if (FOLD) st_coh(o, acc[t]);
                    else *o = acc[t];
                }
        }
    }
    if constexpr (FOLD > 0) {
        /* Ordering (HIP's scoped memory model): the workgroup barrier orders
         * every wave's logit stores before thread 0's counter increment,
         * which is an agent-scope release.  In the block that reads the
         * final count, thread 0 fences acquire at agent scope after that
         * read, before the barrier that broadcasts it, so the logits of all
         * blocks (through the counter's release sequence) happen-before every
         * wave's loads, whichever XCD wrote them.  The other blocks only
         * release. */
        __shared__ int last;
        __syncthreads();
        if (threadIdx.x == 0) {
            last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
            if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
        if (!last) return;
        topk_dispatch_block<FOLD, true>(a);
        /* back to zero for the next launch (the kernel boundary orders it
         * before that launch's increments) */
        if (threadIdx.x == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
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

/* ------------------------------------------------ two-pass large-batch router
 * The selection needs the canonical logits only where they decide it.  Pass 1
 * computes every logit approximately on the matrix cores; pass 2 brackets
 * each canonical logit C(t,e) by the approximation A(t,e) +- eps(t,e),
 * recomputes in the canonical order exactly the experts whose upper bound
 * reaches the K-th largest lower bound (the only ones that can be among the K
 * winners), and selects among those with the unchanged rounds.  The winners,
 * their order, the weights and the shared-gate logit are therefore those of
 * the canonical router bit for bit; a non-candidate's logit stays the
 * approximation, within eps of the canonical value.
 *
 * The bound.  A = 2^-s_e * sum_i fp16(x_i) fp16(2^s_e w_i) with the products
 * exact in fp32 and the sum accumulated in fp32 (any order).  Per element,
 * |fp16(v) - v| <= 2^-11 |v| + 2^-14 (the second term also covers inputs the
 * hardware would treat as zero); 2^s_e puts the row's largest |w| in
 * [2^14, 2^15), so w's absolute term is below 2^-28 max|w_e|.  Summing, with
 * sum |w_i x_i| <= |w||x| and sum |w_i| <= sqrt(H) |w|, and the accumulation
 * error of both sums (gamma_H with u = 2^-23 for the matrix cores, u = 2^-24
 * for the canonical fma chain) gives
 *   |A - C| <= |w| (c1' |x| + 2^-14 sqrt(H)),
 *   c1' = 2^-10 + 2^-21 + 2^-28 sqrt(H) + 2 gamma_H(2^-23).
 * route_eps_coeffs returns 9/8 of these coefficients.  wnorm[e] >= |w_e| is
 * rounded up at pack time and |x| is rounded up in pass 2; a non-finite
 * approximation or bound makes the expert a candidate. */

/* W16/wscale/wnorm for one router matrix: a block per row.  W16 rows hold
 * each 4-group of k in the order (0,2,1,3), the order of the fp16 copy of x
 * that the grouped GEMMs read, so the approximation pass can take either
 * that copy or x itself (permuted as it converts) as its other operand. */
__global__ __launch_bounds__(256) void k_pack_router(const float *W, int H, _Float16 *W16, float *wscale,
                                                      float *wnorm) {
    const int e = blockIdx.x;
    const float *row = W + (size_t)e * H;
    __shared__ float smax[4];
    __shared__ double ssq[4];
    float m = 0.0f;
    double q = 0.0;
    bool bad = false;
    for (int i = threadIdx.x; i < H; i += 256) {
        const float v = row[i];
        bad |= !__builtin_isfinite(v);
        m = fmaxf(m, fabsf(v));
        q += (double)v * (double)v;
    }
    for (int o = 32; o; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o, 64));
        q += __shfl_xor(q, o, 64);
    }
    const int anybad = __syncthreads_or(bad);
    if ((threadIdx.x & 63) == 0) { smax[threadIdx.x >> 6] = m; ssq[threadIdx.x >> 6] = q; }
    __syncthreads();
    m = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    q = (ssq[0] + ssq[1]) + (ssq[2] + ssq[3]);
    int sh = 0; /* 2^sh * m in [2^14, 2^15) */
    bool unbounded = anybad;
    if (m > 0.0f && !anybad) {
        int ex;
        (void)frexpf(m, &ex); /* m = f * 2^ex, f in [0.5, 1) */
        sh = 15 - ex;
        if (sh > 126 || sh < -126) { /* outside the bound's assumptions: always a candidate */
            sh = sh > 126 ? 126 : -126;
            unbounded = true;
        }
    }
    const float sc = ldexpf(1.0f, sh);
    for (int i = threadIdx.x; i < H; i += 256)
        W16[(size_t)e * H + ((i & ~3) | ((i & 1) << 1) | ((i >> 1) & 1))] = (_Float16)(row[i] * sc);
    if (threadIdx.x == 0) {
        wscale[e] = ldexpf(1.0f, -sh);
        /* sqrt in double, then one float step up: an upper bound of |w| */
        const float n = (float)sqrt(q);
        wnorm[e] = unbounded ? __builtin_inff() : nextafterf(n, __builtin_inff()) * (1.0f + 0x1p-20f);
    }
}


/* Pass 1: approximate logits on the matrix cores (v_mfma_f32_16x16x32_f16,
 * tokens as A rows, experts as B columns), split over k.  Block (tile, q)
 * sums k in [q H/8, (q+1) H/8) for 16*TTS tokens and every expert into
 * part[q][t][e], unscaled (the top-k adds the 8 slices and applies wscale).
 * The slices go to linear ids with the same id % 8, so each slice's blocks
 * run on one XCD: that XCD reads its eighth of x and of W16 from HBM once,
 * and a block moves 16*TTS rows of x plus E rows of W16 of one slice to its
 * CU (at T = 512, 36 MB over all blocks, against 64 MB for 16 x 32 tiles
 * over all of k).  The block's x slice is converted once into LDS as fp16
 * A fragments (round to nearest even, each 4-group stored (0,2,1,3), the
 * order of W16's rows), and into x16 for the grouped GEMMs; in a prefill
 * stack, where the previous layer's combine + RMSNorm has written x16, the
 * pass reads it instead (XH) and stages nothing.  Wave w takes the expert
 * groups w, w + NW, ... (16*TES experts each), issues a group's W16 loads
 * for the slice, then runs its MFMAs. */
template <int TTS, int TES, int NW, bool XH, int KS_MAX>
__global__ __launch_bounds__(64 * NW) void k_route_approx(RouteArgs a) {
    /* the arguments in one round of scalar loads at entry (left alone, the
     * packed router's address came in a second round) */
    asm volatile("" ::"s"(a.W16), "s"(a.x), "s"(a.x16), "s"(a.x16in), "s"(a.part), "s"(a.dcnt), "s"(a.tmask),
                 "s"(a.T), "s"(a.E), "s"(a.H), "s"(gridDim.x));
    /* KS_MAX: the largest slice (H / 8) the launch allows */
    __shared__ __attribute__((aligned(16))) _Float16 xs[16 * TTS][KS_MAX + 16];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int E = a.E, H = a.H, T = a.T, KS = H / 8, nst = KS / 32;
    const int q = blockIdx.x & 7, t0 = (blockIdx.x >> 3) * (16 * TTS), k0 = q * KS;
    const int r = lane & 15, kq = (lane >> 4) * 8;
    const int ngr = (E + 16 * TES - 1) / (16 * TES);
    /* 8 steps (256 k) of a group's W16 loads at a time, all issued before
     * the chunk's MFMAs (the whole slice at H = 2048); steps past the slice
     * are clamped and unused */
    h8 B[8][TES];
    auto load_b = [&](int g, int c0) {
#pragma unroll
        for (int st = 0; st < 8; st++)
#pragma unroll
            for (int es = 0; es < TES; es++)
                B[st][es] = *(const h8 *)(a.W16 + (size_t)min(g * 16 * TES + es * 16 + r, E - 1) * H + k0 + kq +
                                          32 * min(c0 + st, nst - 1));
    };
    if (a.dcnt && blockIdx.x == 0)
        for (int i = threadIdx.x; i < (T + 255) / 256 * E; i += 64 * NW) a.dcnt[i] = 0u;
    if (a.tmask) { /* the token marks, 16 bytes a thread over all blocks */
        const size_t n16 = (size_t)E * TMASK_LD(T) / 16;
        for (size_t i = (size_t)blockIdx.x * 64 * NW + threadIdx.x; i < n16; i += (size_t)gridDim.x * 64 * NW)
            *(u4 *)(a.tmask + 16 * i) = u4{0u, 0u, 0u, 0u};
    }
    /* stage the slice, 8 k values (two 4-groups) per item: the x loads go
     * out first, then the first chunk's W16 loads, so the conversion waits
     * only for x (loads complete in order) */
    constexpr int NIT = (16 * TTS * (KS_MAX / 8) + 64 * NW - 1) / (64 * NW);
    const int ipr = KS / 8, items = 16 * TTS * ipr;
    f4 xl[NIT][2];
    h8 xh[NIT];
#pragma unroll
    for (int j = 0; j < NIT; j++) {
        const int it = min((int)threadIdx.x + 64 * NW * j, items - 1), rr = it / ipr, c = (it % ipr) * 8;
        const int t = min(t0 + rr, T - 1);
        if (XH) {
            xh[j] = *(const h8 *)(a.x16in + (size_t)t * H + k0 + c);
        } else {
            xl[j][0] = *(const f4 *)(a.x + (size_t)t * H + k0 + c);
            xl[j][1] = *(const f4 *)(a.x + (size_t)t * H + k0 + c + 4);
        }
    }
    if (wv < ngr) load_b(wv, 0);
#pragma unroll
    for (int j = 0; j < NIT; j++) {
        const int it = (int)threadIdx.x + 64 * NW * j, rr = it / ipr, c = (it % ipr) * 8;
        if (it < items) {
            const f4 lo = xl[j][0], hi = xl[j][1];
            const h8 v = XH ? xh[j]
                            : h8{(_Float16)lo.x, (_Float16)lo.z, (_Float16)lo.y, (_Float16)lo.w,
                                 (_Float16)hi.x, (_Float16)hi.z, (_Float16)hi.y, (_Float16)hi.w};
            if (!XH && a.x16 && t0 + rr < T) *(h8 *)(a.x16 + (size_t)(t0 + rr) * H + k0 + c) = v;
            *(h8 *)&xs[rr][c] = v;
        }
    }
    __syncthreads();
    for (int g = wv; g < ngr; g += NW) {
        const int e0 = g * 16 * TES;
        f4 acc[TTS][TES];
#pragma unroll
        for (int ts = 0; ts < TTS; ts++)
#pragma unroll
            for (int es = 0; es < TES; es++) acc[ts][es] = f4{0, 0, 0, 0};
        for (int c0 = 0; c0 < nst; c0 += 8) {
            if (c0 || g != wv) load_b(g, c0);
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const int step = c0 + st;
                if (step < nst) {
#pragma unroll
                    for (int ts = 0; ts < TTS; ts++) {
                        const h8 A = *(const h8 *)&xs[ts * 16 + r][32 * step + kq];
#pragma unroll
                        for (int es = 0; es < TES; es++)
                            acc[ts][es] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[st][es], acc[ts][es], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int ts = 0; ts < TTS; ts++)
#pragma unroll
            for (int es = 0; es < TES; es++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int t = t0 + ts * 16 + 4 * (lane >> 4) + v, e = e0 + es * 16 + (lane & 15);
                    if (t < T && e < E) a.part[((size_t)q * T + t) * E + e] = acc[ts][es][v];
                }
    }
}

/* Pass 2: WPT waves per token (the lane layout of wave_topk).  Every wave of
 * a token adds up the approximation's partial sums, computes the bounds, the K-th largest lower bound and the candidate
 * list; the candidates (the shared-gate row first) are recomputed NB = 32/NI
 * rows at a time, batch i by wave i % WPT, with all loads of a batch in
 * flight together; the exact values meet in LDS and the token's first wave
 * selects.  NI >= H / 256. */
template <int EPL, int NI, int WPT>
__global__ __launch_bounds__(256) void k_topk_exact(RouteArgs a) {
    constexpr int NB = 32 / NI, TPB = 4 / WPT;
    __shared__ float exv[TPB][64 * EPL + 1];
    __shared__ int clist[4][64 * EPL + 1];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw = wv % WPT, tb = wv / WPT;
    const int t = blockIdx.x * TPB + tb;
    const bool live = t < a.T;
    const int E = a.E, H = a.H, K = a.K, ni = H / 256;
    float *lrow = a.logits + (size_t)min(t, a.T - 1) * (E + 1);
    const float *xrow = a.x + (size_t)min(t, a.T - 1) * H;
    /* every load unconditional (indices clamped, values masked where used):
     * a load under a branch makes the compiler wait for it */
    f4 xv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) xv[i] = *(const f4 *)(xrow + 256 * min(i, ni - 1) + 4 * lane);
#pragma unroll
    for (int i = 0; i < NI; i++)
        if (i >= ni) xv[i] = f4{0, 0, 0, 0};
    float v[EPL], bv[EPL], rn[EPL];
    const float *bias = a.bias ? a.bias : a.wnorm;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = min(lane * EPL + j, E - 1);
        rn[j] = a.wnorm[e];
        bv[j] = bias[e];
    }
    { /* the approximate logit: the pass's partial sums, slices ascending, then the row scale */
        const int tt = min(t, a.T - 1);
        float pq[8][EPL];
        if (EPL == 4 && E % 4 == 0) { /* one 16-byte load per slice (lanes past E clamped) */
            const int e4 = min(lane * 4, E - 4);
#pragma unroll
            for (int qq = 0; qq < 8; qq++) {
                const f4 v4 = *(const f4 *)(a.part + ((size_t)qq * a.T + tt) * E + e4);
                pq[qq][0] = v4.x; pq[qq][EPL > 1 ? 1 : 0] = v4.y; pq[qq][EPL > 2 ? 2 : 0] = v4.z; pq[qq][EPL > 3 ? 3 : 0] = v4.w;
            }
        } else {
#pragma unroll
            for (int qq = 0; qq < 8; qq++)
#pragma unroll
                for (int j = 0; j < EPL; j++) pq[qq][j] = a.part[((size_t)qq * a.T + tt) * E + min(lane * EPL + j, E - 1)];
        }
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            float sum = pq[0][j];
#pragma unroll
            for (int qq = 1; qq < 8; qq++) sum += pq[qq][j];
            v[j] = sum * a.wscale[min(lane * EPL + j, E - 1)];
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        ss = __builtin_fmaf(xv[i].x, xv[i].x, ss);
        ss = __builtin_fmaf(xv[i].y, xv[i].y, ss);
        ss = __builtin_fmaf(xv[i].z, xv[i].z, ss);
        ss = __builtin_fmaf(xv[i].w, xv[i].w, ss);
    }
    /* |x| rounded up: the fp32 sum of squares is within H 2^-24 of itself */
    const float xn = sqrtf(wave_sum_fast(ss)) * (1.0f + 0x1p-10f);
    /* lower bounds (as keys) and upper bounds of the selection values */
    uint32_t lo[EPL];
    float hi[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const float eps = rn[j] * __builtin_fmaf(a.eps_c1, xn, a.eps_c2);
        float l = v[j] - eps, h = v[j] + eps;
        if (a.bias) { l += bv[j]; h += bv[j]; }
        const bool known = __builtin_isfinite(v[j]) && __builtin_isfinite(eps);
        if (!known || !(l == l)) l = -__builtin_inff();
        if (!known || !(h == h)) h = __builtin_inff();
        lo[j] = lane * EPL + j < E ? route_ord(l) : 0u;
        hi[j] = h;
    }
    /* the K-th largest lower bound */
#pragma unroll
    for (int pass = 0; pass < EPL; pass++)
#pragma unroll
        for (int j = pass & 1; j + 1 < EPL; j += 2)
            if (lo[j + 1] > lo[j]) { const uint32_t tk = lo[j]; lo[j] = lo[j + 1]; lo[j + 1] = tk; }
    uint32_t m = 0u;
#pragma unroll 1
    for (int k = 0; k < K; k++) {
        m = wave_max_u32(lo[0]);
        const int wl = (int)__builtin_ctzll(__ballot(lo[0] == m));
        if (lane == wl) {
#pragma unroll
            for (int j = 0; j + 1 < EPL; j++) lo[j] = lo[j + 1];
            lo[EPL - 1] = 0u;
        }
    }
    const float L = ord_value(m);
    bool cand[EPL];
    /* the candidate list (the shared-gate row E first), in this wave's own
     * LDS slot: position = rows before it in (j, lane) order */
    int nc = a.wsg ? 1 : 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        cand[j] = lane * EPL + j < E && !(hi[j] < L);
        const uint64_t mk = __ballot(cand[j]);
        const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        if (cand[j]) clist[wv][nc + below] = lane * EPL + j;
        nc += (int)__builtin_popcountll(mk);
    }
    if (a.wsg && lane == 0) clist[wv][0] = E;
    __builtin_amdgcn_wave_barrier();
    /* canonical recomputation, NB rows a batch, batch i by wave i % WPT */
    for (int base = tw * NB; live && base < nc; base += WPT * NB) {
        int ids[NB];
#pragma unroll
        for (int b = 0; b < NB; b++)
            ids[b] = base + b < nc ? __builtin_amdgcn_readfirstlane(clist[wv][base + b]) : -1;
        f4 w[NB][NI];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float *row = ids[b] == E ? a.wsg : a.W + (size_t)max(ids[b], 0) * H;
#pragma unroll
            for (int i = 0; i < NI; i++) w[b][i] = *(const f4 *)(row + 256 * min(i, ni - 1) + 4 * lane);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (ids[b] < 0) break;
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < NI; i++)
                if (i < ni) {
                    d = __builtin_fmaf(w[b][i].x, xv[i].x, d);
                    d = __builtin_fmaf(w[b][i].y, xv[i].y, d);
                    d = __builtin_fmaf(w[b][i].z, xv[i].z, d);
                    d = __builtin_fmaf(w[b][i].w, xv[i].w, d);
                }
            d = wave_sum_canon(d);
            if (lane == 0) exv[tb][ids[b]] = d;
        }
    }
    if (WPT > 1) __syncthreads();
    if (!live || tw != 0) return;
    const float sg = a.wsg ? exv[tb][E] : 0.0f;
    uint32_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        if (cand[j]) v[j] = exv[tb][lane * EPL + j];
        key[j] = cand[j] ? route_ord(a.bias ? v[j] + bv[j] : v[j]) : 0u;
        if (lane * EPL + j < E) lrow[lane * EPL + j] = v[j];
    }
    if (lane == 0) lrow[E] = sg;
    const TopkLane r = wave_topk_keys<EPL>(key, sg, K, lane, a.idx + t * K, a.w + t * K, a.sgl + t, nullptr);
    /* the three-launch dispatch's per-block expert counts (order-free) */
    if (a.dcnt && lane < K) atomicAdd(a.dcnt + (size_t)(t / 256) * E + r.id, 1u);
    if (a.tmask && lane < K) a.tmask[(size_t)r.id * TMASK_LD(a.T) + t] = 1;
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

template <int KM>
DEV void dispatch_masks(const RouteArgs &a, uint32_t *mask, int (&ek)[KM]) {
    const int E = a.E, K = a.K, tid = threadIdx.x, t = blockIdx.x * DSP_TOK + tid;
    /* the token's ids loaded together (indices clamped; a load under a
     * branch is waited for alone); -1 marks no pair */
#pragma unroll
    for (int k = 0; k < KM; k++) ek[k] = a.idx[min(t, a.T - 1) * K + min(k, K - 1)];
    for (int i = tid; i < E * DSP_WORDS; i += DSP_TOK) mask[i] = 0;
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (k >= K || t >= a.T) ek[k] = -1;
    lds_barrier();
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (ek[k] >= 0) atomicOr(&mask[ek[k] * DSP_WORDS + (tid >> 5)], 1u << (tid & 31));
    lds_barrier();
}

template <int KM>
__global__ __launch_bounds__(DSP_TOK) void k_dispatch_count(RouteArgs a, uint32_t *cnt) {
    extern __shared__ uint32_t mask[]; /* E * DSP_WORDS */
    int ek[KM];
    dispatch_masks<KM>(a, mask, ek);
    for (int e = threadIdx.x; e < a.E; e += DSP_TOK) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < DSP_WORDS; w++) c += __popc(mask[e * DSP_WORDS + w]);
        cnt[(size_t)blockIdx.x * a.E + e] = c;
    }
}

/* Tiles of one expert: rows <= GEMM_TILE_SMALL -> one small tile, else
 * ceil(rows / GEMM_TILE_BIG) big tiles.  While the batch is small (T K <=
 * GEMM_TILE_SMALL E, tile_small_only) every expert is cut into small tiles:
 * the few big experts of a skewed routing would otherwise leave most CUs
 * idle in a big-tile launch of their own, and the shared expert is in the
 * small list then anyway (the host launches only that list). */
DEV bool tile_small_only(const RouteArgs &a) { return (size_t)a.T * a.K <= (size_t)GEMM_TILE_SMALL * a.E; }
DEV uint32_t n_small_tiles(uint32_t c, bool so) {
    return so ? (c + GEMM_TILE_SMALL - 1) / GEMM_TILE_SMALL : c != 0 && c <= GEMM_TILE_SMALL;
}
DEV uint32_t n_big_tiles(uint32_t c, bool so) {
    return !so && c > GEMM_TILE_SMALL ? (c + GEMM_TILE_BIG - 1) / GEMM_TILE_BIG : 0;
}
DEV void put_tiles(uint32_t *list, uint32_t t0, uint32_t e, uint32_t first, uint32_t c, uint32_t tm) {
    for (uint32_t j = 0; j * tm < c; j++) {
        list[1 + 3 * (t0 + j)] = e;
        list[2 + 3 * (t0 + j)] = first + j * tm;
        list[3 + 3 * (t0 + j)] = min(tm, c - j * tm);
    }
}

/* Given the count c of expert tid (threads tid < E <= blockDim.x; others
 * pass anything): scans counts, active flags and tile counts (two 16-bit
 * fields per word: T K <= 32768, E <= 1024) and writes offsets, the active
 * list and the two GEMM tile lists, and the expert's exclusive offset to
 * xo[tid] (LDS, when given).  Every thread of the block calls it; wsum:
 * LDS, 32 words. */
DEV void dispatch_lists(const RouteArgs &a, uint32_t c, uint32_t *xo, uint32_t *wsum, uint32_t *tiles_s,
                        uint32_t *tiles_b, int has_shared, bool glob = true) {
    /* glob false: the exclusive offsets into xo only (the blocks of a
     * dispatch that one other block writes the lists for) */
    const int E = a.E, T = a.T, tid = threadIdx.x;
    const bool so = tile_small_only(a), mine = tid < E;
    if (!mine) c = 0;
    const uint32_t ns_own = n_small_tiles(c, so), nb_own = n_big_tiles(c, so);
    uint32_t x = c | ((uint32_t)(c != 0) << 16), y = ns_own | (nb_own << 16), tx, ty;
    scan2_block(x, y, wsum, tx, ty);
    if (mine) {
        const uint32_t o = (x & 0xFFFFu) - c;
        if (xo) xo[tid] = o;
    }
    if (!glob) return;
    if (mine) {
        const uint32_t o = (x & 0xFFFFu) - c;
        a.offsets[tid] = o;
        if (c) {
            const uint32_t r = (x >> 16) - 1;
            ACT_E(a.list, r) = (uint32_t)tid;
            ACT_OFF(a.list, E, r) = o;
            if (c <= GEMM_TILE_SMALL || so)
                put_tiles(tiles_s, (y & 0xFFFFu) - ns_own, (uint32_t)tid, o, c, GEMM_TILE_SMALL);
            else put_tiles(tiles_b, (y >> 16) - nb_own, (uint32_t)tid, o, c, GEMM_TILE_BIG);
        }
    }
    if (tid == 0) {
        const uint32_t n_act = tx >> 16, ns = ty & 0xFFFFu, nb = ty >> 16, Tu = (uint32_t)T, total = tx & 0xFFFFu;
        a.offsets[E] = total;
        ACT_N(a.list) = n_act;
        ACT_OFF(a.list, E, n_act) = total;
        /* the shared expert (id E) over tokens 0..T-1, in the list that holds
         * most of the routed work (a lone list of shared tiles would run as
         * a tail after the other launch) */
        const uint32_t tm = so ? GEMM_TILE_SMALL : GEMM_TILE_BIG, nsh = has_shared ? (Tu + tm - 1) / tm : 0;
        if (has_shared) put_tiles(so ? tiles_s : tiles_b, so ? ns : nb, (uint32_t)E, 0, Tu, tm);
        tiles_s[0] = ns + (so ? nsh : 0);
        tiles_b[0] = nb + (so ? 0 : nsh);
    }
}

__global__ __launch_bounds__(DSP_THREADS) void k_dispatch_scan(RouteArgs a, uint32_t *cnt, int G,
                                                               uint32_t *tiles_s, uint32_t *tiles_b,
                                                               int has_shared) {
    __shared__ uint32_t wsum[32];
    const int E = a.E, tid = threadIdx.x;
    uint32_t run = 0;
    if (tid < E) {
        /* counts 16 blocks at a time, all loaded before the prefixes are
         * stored (a load behind a store waits for it) */
        for (int g0 = 0; g0 < G; g0 += 16) {
            uint32_t c[16];
#pragma unroll
            for (int j = 0; j < 16; j++) c[j] = cnt[(size_t)min(g0 + j, G - 1) * E + tid];
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (g0 + j < G) {
                    cnt[(size_t)(g0 + j) * E + tid] = run;
                    run += c[j];
                }
        }
    }
    dispatch_lists(a, run, nullptr, wsum, tiles_s, tiles_b, has_shared);
}

template <int KM>
__global__ __launch_bounds__(DSP_TOK) void k_dispatch_scatter(RouteArgs a, const uint32_t *base) {
    extern __shared__ uint32_t mask[]; /* E * DSP_WORDS, then E * DSP_WORDS word prefixes */
    uint32_t *wpre = mask + a.E * DSP_WORDS;
    int ek[KM];
    dispatch_masks<KM>(a, mask, ek);
    const int E = a.E, K = a.K, tid = threadIdx.x, t = blockIdx.x * DSP_TOK + tid;
    for (int e = tid; e < E; e += DSP_TOK) {
        uint32_t run = a.offsets[e] + base[(size_t)blockIdx.x * E + e];
#pragma unroll
        for (int w = 0; w < DSP_WORDS; w++) {
            wpre[e * DSP_WORDS + w] = run;
            run += __popc(mask[e * DSP_WORDS + w]);
        }
    }
    lds_barrier();
    const uint32_t below = (1u << (tid & 31)) - 1u;
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (ek[k] >= 0) {
            const int i = ek[k] * DSP_WORDS + (tid >> 5);
            const uint32_t pos = wpre[i] + __popc(mask[i] & below);
            const uint32_t p = (uint32_t)(t * K + k);
            a.pairs[pos] = p;
            a.pos[p] = pos;
        }
}

/* Scan and scatter in one launch, for counts the exact top-k made (E <=
 * DSP_TOK): every block forms every expert's total and its own prefix over
 * the earlier blocks from the counts (G E words), scans the totals, and
 * block 0 writes the offsets and lists; then each scatters its tokens as
 * k_dispatch_scatter does.  The counts are left as they are (the
 * approximation pass of the next forward clears them). */
template <int KM>
__global__ __launch_bounds__(DSP_TOK) void k_dispatch_scan_scatter(RouteArgs a, const uint32_t *cnt, int G,
                                                                   uint32_t *tiles_s, uint32_t *tiles_b,
                                                                   int has_shared) {
    asm volatile("" ::"s"(a.idx), "s"(a.E), "s"(a.K), "s"(a.T), "s"(a.offsets), "s"(a.pairs), "s"(a.pos),
                 "s"(cnt), "s"(G), "s"(gridDim.x));
    extern __shared__ uint32_t mask[]; /* E * DSP_WORDS, then E * DSP_WORDS word prefixes */
    __shared__ uint32_t xo[DSP_TOK], wsum[32];
    uint32_t *wpre = mask + a.E * DSP_WORDS;
    const int E = a.E, K = a.K, tid = threadIdx.x, t = blockIdx.x * DSP_TOK + tid, gb = blockIdx.x;
    uint32_t tot = 0, pre = 0;
    if (tid < E) {
        /* 8 blocks' counts at a time, all loaded before any is used */
        for (int g0 = 0; g0 < G; g0 += 8) {
            uint32_t c[8];
#pragma unroll
            for (int j = 0; j < 8; j++) c[j] = cnt[(size_t)min(g0 + j, G - 1) * E + tid];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (g0 + j < G) {
                    tot += c[j];
                    if (g0 + j < gb) pre += c[j];
                }
        }
    }
    int ek[KM];
    dispatch_masks<KM>(a, mask, ek);
    dispatch_lists(a, tot, xo, wsum, tiles_s, tiles_b, has_shared, gb == 0);
    if (tid < E) {
        uint32_t run = xo[tid] + pre;
#pragma unroll
        for (int w = 0; w < DSP_WORDS; w++) {
            wpre[tid * DSP_WORDS + w] = run;
            run += __popc(mask[tid * DSP_WORDS + w]);
        }
    }
    lds_barrier();
    const uint32_t below = (1u << (tid & 31)) - 1u;
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (ek[k] >= 0) {
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
template <int KM>
__global__ __launch_bounds__(DSP_THREADS) void k_dispatch_one(RouteArgs a, uint32_t *tiles_s, uint32_t *tiles_b,
                                                              int has_shared) {
    __shared__ uint32_t xo[256], wsum[32];
    __shared__ uint32_t mask[DSP1_SUB * 256 * DSP_WORDS], wpre[DSP1_SUB * 256 * DSP_WORDS];
    const int E = a.E, K = a.K, T = a.T, tid = threadIdx.x;
    const int sub = tid / DSP_TOK, tl = tid % DSP_TOK;
    /* the token's K expert ids, loaded together (indices clamped; a load
     * under a branch is waited for alone) while the masks are cleared, then
     * marked */
    int ek[KM];
#pragma unroll
    for (int k = 0; k < KM; k++) ek[k] = a.idx[min(tid, T - 1) * K + min(k, K - 1)];
    for (int i = tid; i < DSP1_SUB * E * DSP_WORDS; i += DSP_THREADS) mask[i] = 0;
    lds_barrier();
#pragma unroll
    for (int k = 0; k < KM; k++) {
        if (k >= K || tid >= T) ek[k] = -1;
        if (ek[k] >= 0) atomicOr(&mask[(sub * E + ek[k]) * DSP_WORDS + (tl >> 5)], 1u << (tl & 31));
    }
    lds_barrier();
    uint32_t run = 0;
    if (tid < E) { /* word prefixes from 0, and the expert's count */
        uint32_t m[DSP1_SUB * DSP_WORDS];
#pragma unroll
        for (int sc = 0; sc < DSP1_SUB; sc++)
#pragma unroll
            for (int w = 0; w < DSP_WORDS; w++) m[sc * DSP_WORDS + w] = mask[(sc * E + tid) * DSP_WORDS + w];
#pragma unroll
        for (int sc = 0; sc < DSP1_SUB; sc++)
#pragma unroll
            for (int w = 0; w < DSP_WORDS; w++) {
                wpre[(sc * E + tid) * DSP_WORDS + w] = run;
                run += __popc(m[sc * DSP_WORDS + w]);
            }
    }
    dispatch_lists(a, run, xo, wsum, tiles_s, tiles_b, has_shared);
    lds_barrier();
    const uint32_t below = (1u << (tl & 31)) - 1u;
    uint32_t pk[KM];
#pragma unroll
    for (int k = 0; k < KM; k++)
        if (ek[k] >= 0) {
            const int e = ek[k], i = (sub * E + e) * DSP_WORDS + (tl >> 5);
            pk[k] = xo[e] + wpre[i] + __popc(mask[i] & below);
            a.pairs[pk[k]] = (uint32_t)(tid * K + k);
        }
    /* the token's K inverse positions: contiguous, written as 16-byte runs
     * when K = 8 */
    if (KM == 8 && K == 8) {
        if (tid < T) {
            *(u4 *)(a.pos + tid * 8) = u4{pk[0], pk[1], pk[2], pk[3]};
            *(u4 *)(a.pos + tid * 8 + 4) = u4{pk[4], pk[5], pk[6], pk[7]};
        }
    } else {
#pragma unroll
        for (int k = 0; k < KM; k++)
            if (ek[k] >= 0) a.pos[tid * K + k] = pk[k];
    }
}

/* RMSNorm (inference/src/shaders.metal:128-149) with the canonical sum of
 * squares: x = (h * (1 / sqrt(ss/H + eps))) * bf16(w); one wave per token. */
template <int NIM>
__global__ __launch_bounds__(64) void k_rmsnorm(const float *h, const float *w, int H, float eps,
                                                float *x) {
    const int lane = threadIdx.x, t = blockIdx.x;
    const float *ht = h + (size_t)t * H;
    const int NI = H / 256;
    /* every load unconditional (row index clamped) and issued before the
     * first use: a load under a branch, or one behind a store, is waited
     * for alone */
    f4 v[NIM], wv[NIM];
#pragma unroll
    for (int i = 0; i < NIM; i++) v[i] = *(const f4 *)(ht + 256 * min(i, NI - 1) + 4 * lane);
#pragma unroll
    for (int i = 0; i < NIM; i++) wv[i] = *(const f4 *)((w ? w : ht) + 256 * min(i, NI - 1) + 4 * lane);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NIM; i++)
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
    for (int i = 0; i < NIM; i++)
        if (i < NI) {
            const int j = 256 * i + 4 * lane;
            const f4 wq = w ? wv[i] : f4{1, 1, 1, 1};
            f4 o;
            o.x = (v[i].x * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wq.x) & 0xFFFF0000u);
            o.y = (v[i].y * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wq.y) & 0xFFFF0000u);
            o.z = (v[i].z * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wq.z) & 0xFFFF0000u);
            o.w = (v[i].w * scale) * __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, wq.w) & 0xFFFF0000u);
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
        case 1: KLAUNCH(KERNEL<1>, __VA_ARGS__); break;        \
        case 2: KLAUNCH(KERNEL<2>, __VA_ARGS__); break;        \
        case 4: KLAUNCH(KERNEL<4>, __VA_ARGS__); break;        \
        case 8: KLAUNCH(KERNEL<8>, __VA_ARGS__); break;        \
        case 16: KLAUNCH(KERNEL<16>, __VA_ARGS__); break;      \
        default: return -2;                                               \
    }

int route_small_folds(const RouteArgs &a) {
    return a.T >= 1 && a.T <= 16 && a.T * a.K <= 256 && a.H % 256 == 0 && a.H <= 256 * 8 && epl_for(a.E) == 4;
}

int launch_route_small(const RouteArgs &a, hipStream_t s, int fold_topk) {
    if (a.T < 1 || a.T > 16 || a.T * a.K > 256 || a.H % 256 || a.H > 4096) return -2;
    if (fold_topk && !route_small_folds(a)) return -2;
    const dim3 g((a.E + 1 + 3) / 4), g2((a.E + 1 + 1) / 2), g4((unsigned)(a.E + 1));
#define RS_LAUNCH(TM, NIMV, RSV, G)                                                                      \
    do {                                                                                                 \
        if (fold_topk && NIMV == 8) {                                                                    \
            const dim3 gf((unsigned)((a.E + 1 + 8 / (RSV) - 1) / (8 / (RSV))));                          \
            if (a.norm_h) KLAUNCH((k_route_small<true, TM, 8, RSV, 4>), gf, dim3(512), 0, s, a);         \
            else KLAUNCH((k_route_small<false, TM, 8, RSV, 4>), gf, dim3(512), 0, s, a);                 \
        } else if (a.norm_h) KLAUNCH((k_route_small<true, TM, NIMV, RSV, 0>), G, dim3(256), 0, s, a);    \
        else KLAUNCH((k_route_small<false, TM, NIMV, RSV, 0>), G, dim3(256), 0, s, a);                   \
    } while (0)
#define RS_T(NIMV)                                \
    do {                                          \
        if (a.T == 1) RS_LAUNCH(1, NIMV, 1, g);   \
        else if (a.T <= 4) RS_LAUNCH(4, NIMV, 1, g); \
        else if (a.T <= 8) RS_LAUNCH(4, NIMV, 2, g2); \
        else RS_LAUNCH(4, NIMV, 4, g4);           \
    } while (0)
    if (a.H <= 256 * 8) RS_T(8);
    else RS_T(CANON_NI);
#undef RS_T
#undef RS_LAUNCH
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
    KLAUNCH(k_route_logits, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk(const RouteArgs &a, hipStream_t s) {
    dim3 grid((a.T + 3) / 4);
    EPL_SWITCH(a.E, k_topk, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

void route_eps_coeffs(int H, float *c1, float *c2) {
    const double u = 0x1p-23, g = H * u / (1.0 - H * u);
    /* 9/8: room for the rounding of the bound arithmetic itself (eps, the
     * bounds and the norms: a few ulps, against eps >= 2^-10 |w||x|) */
    *c1 = (float)(1.125 * (0x1p-10 + 0x1p-21 + 0x1p-28 * sqrt((double)H) + 2.0 * g));
    *c2 = (float)(1.125 * 0x1p-14 * sqrt((double)H));
}

int launch_pack_router(const float *W, int E, int H, _Float16 *W16, float *wscale, float *wnorm, hipStream_t s) {
    if (E < 1 || H < 1) return -2;
    KLAUNCH(k_pack_router, dim3(E), dim3(256), 0, s, W, H, W16, wscale, wnorm);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* the approximation pass, 8 waves a block: 16 tokens a block up to 1024
 * tokens, 32 below 2048, 64 from 2048 (one block per CU there: T = 2048
 * approximation 14.6 -> 12.2 us against 32-token blocks, 14.6 with 128) */
int launch_route_approx(const RouteArgs &a, hipStream_t s) {
    if (!a.W16 || !a.wscale || !a.part || a.H % 256 || a.H > 4096 || a.T < 1) return -2;
    const int tts = a.T <= 1024 ? 1 : a.T < 2048 ? 2 : 4;
    const dim3 grid((unsigned)((a.T + 16 * tts - 1) / (16 * tts) * 8));
#define SK_LAUNCH(TTS, KSM)                                                                          \
    do {                                                                                            \
        if (a.x16in) KLAUNCH((k_route_approx<TTS, 2, 8, true, KSM>), grid, dim3(512), 0, s, a);  \
        else KLAUNCH((k_route_approx<TTS, 2, 8, false, KSM>), grid, dim3(512), 0, s, a);         \
    } while (0)
#define SK_H(TTS)                            \
    do {                                     \
        if (a.H <= 2048) SK_LAUNCH(TTS, 256); \
        else SK_LAUNCH(TTS, 512);            \
    } while (0)
    if (tts == 1) SK_H(1);
    else if (tts == 2) SK_H(2);
    else SK_H(4);
#undef SK_H
#undef SK_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_topk_exact(const RouteArgs &a, hipStream_t s) {
    if (!a.wnorm || !a.part || !a.wscale || a.H % 256 || a.H > 4096 || a.K > 64 || a.K > a.E) return -2;
    const int ni = a.H / 256;
    /* up to 1024 tokens a token's candidates spread over 4 waves (more waves
     * in flight); beyond, one wave per token already fills the chip */
    const int wpt = a.T <= 1024 ? 4 : 1;
    const dim3 grid((a.T * wpt + 3) / 4);
#define TKX(NIV, WPTV)                                                                                   \
    switch (epl_for(a.E)) {                                                                              \
        case 1: KLAUNCH((k_topk_exact<1, NIV, WPTV>), grid, dim3(256), 0, s, a); break;   \
        case 2: KLAUNCH((k_topk_exact<2, NIV, WPTV>), grid, dim3(256), 0, s, a); break;   \
        case 4: KLAUNCH((k_topk_exact<4, NIV, WPTV>), grid, dim3(256), 0, s, a); break;   \
        case 8: KLAUNCH((k_topk_exact<8, NIV, WPTV>), grid, dim3(256), 0, s, a); break;   \
        case 16: KLAUNCH((k_topk_exact<16, NIV, WPTV>), grid, dim3(256), 0, s, a); break; \
        default: return -2;                                                                              \
    }
#define TKW(NIV)                      \
    do {                              \
        if (wpt == 4) { TKX(NIV, 4) } \
        else { TKX(NIV, 1) }          \
    } while (0)
    if (ni <= 2) TKW(2);
    else if (ni <= 4) TKW(4);
    else if (ni <= 8) TKW(8);
    else TKW(16);
#undef TKW
#undef TKX
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int dispatch_blocks(int T) { return (T + DSP_TOK - 1) / DSP_TOK; }

#ifndef DISPATCH_ONE
#define DISPATCH_ONE 1
#endif
bool dispatch_three_launches(const RouteArgs &a) { return !(DISPATCH_ONE && a.E <= 256 && a.T <= DSP_THREADS); }

/* counted: cnt already holds the per-block expert counts (the exact top-k
 * added them), so the count launch is skipped */
int launch_dispatch(const RouteArgs &a, uint32_t *tiles_s, uint32_t *tiles_b, int has_shared, uint32_t *cnt,
                    hipStream_t s, int counted) {
    const size_t lds = sizeof(uint32_t) * (size_t)a.E * DSP_WORDS * 2;
    /* one scan lane per expert; 16-bit fields for the pair counts */
    if (lds > 64 * 1024 || a.E > DSP_THREADS || a.K > OROME_MAXK || (long)a.T * a.K > 32768) return -2;
    if (!dispatch_three_launches(a)) {
        if (a.K <= 8) KLAUNCH(k_dispatch_one<8>, dim3(1), dim3(DSP_THREADS), 0, s, a, tiles_s, tiles_b, has_shared);
        else KLAUNCH(k_dispatch_one<OROME_MAXK>, dim3(1), dim3(DSP_THREADS), 0, s, a, tiles_s, tiles_b, has_shared);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const int G = dispatch_blocks(a.T);
    if (counted && a.E <= DSP_TOK) { /* scan and scatter together */
        if (a.K <= 8) KLAUNCH(k_dispatch_scan_scatter<8>, dim3(G), dim3(DSP_TOK), lds, s, a, cnt, G, tiles_s, tiles_b, has_shared);
        else KLAUNCH(k_dispatch_scan_scatter<OROME_MAXK>, dim3(G), dim3(DSP_TOK), lds, s, a, cnt, G, tiles_s, tiles_b, has_shared);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    if (counted) {
    } else if (a.K <= 8) KLAUNCH(k_dispatch_count<8>, dim3(G), dim3(DSP_TOK), lds / 2, s, a, cnt);
    else KLAUNCH(k_dispatch_count<OROME_MAXK>, dim3(G), dim3(DSP_TOK), lds / 2, s, a, cnt);
    KLAUNCH(k_dispatch_scan, dim3(1), dim3(DSP_THREADS), 0, s, a, cnt, G, tiles_s, tiles_b, has_shared);
    if (a.K <= 8) KLAUNCH(k_dispatch_scatter<8>, dim3(G), dim3(DSP_TOK), lds, s, a, (const uint32_t *)cnt);
    else KLAUNCH(k_dispatch_scatter<OROME_MAXK>, dim3(G), dim3(DSP_TOK), lds, s, a, (const uint32_t *)cnt);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x, hipStream_t s) {
    if (H % 256 || H > 256 * CANON_NI) return -2;
    if (H <= 256 * 8) KLAUNCH(k_rmsnorm<8>, dim3(T), dim3(64), 0, s, h, w, H, eps, x);
    else KLAUNCH(k_rmsnorm<CANON_NI>, dim3(T), dim3(64), 0, s, h, w, H, eps, x);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
