/* route_dev.h -- device-side expert selection shared by the routing and
 * decode kernels.
 *
 * Selection restates softmax_topk_route (inference/src/shaders.metal:
 * 1141-1234): K rounds of argmax, ties to the lower expert index, softmax over
 * the K winners.  It runs as a wave64 max over 64-bit keys (order-preserving
 * float bits, then the complemented index), so one reduction settles value
 * and tie.  Dispatch is a stable counting sort of pairs p = t*K + k by expert.
 */
#pragma once
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
template <int EPL, bool COH = false>
DEV void wave_topk(const float *l, const float *bias, int E, int K, int lane, int32_t *idx_out,
                   float *w_out, float *sgl_out, int *e_out) {
    /* all loads first and unconditional (index clamped, then masked), so
     * they are in flight together instead of one round trip each */
    float v[EPL], bv[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = min(lane + 64 * j, E - 1);
        v[j] = COH ? ld_coh(l + e) : l[e];
    }
    if (bias)
#pragma unroll
        for (int j = 0; j < EPL; j++) bv[j] = bias[min(lane + 64 * j, E - 1)];
    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + 64 * j;
        key[j] = e < E ? route_key(bias ? v[j] + bv[j] : v[j], e) : 0;
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
        *sgl_out = COH ? ld_coh(l + E) : l[E];
    }
}

/* Block-wide exclusive scan of one 32-bit value per thread (256 threads):
 * wave inclusive scans by shuffles, then the four wave totals.  Returns the
 * exclusive prefix; *total receives the block sum. */
DEV uint32_t block_excl_scan256(uint32_t v, uint32_t *wsum /* LDS [4] */, uint32_t *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)inc, off, 64);
        if (lane >= off) inc += o;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    uint32_t base = 0;
    for (int w = 0; w < wv; w++) base += wsum[w];
    *total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    return base + inc - v;
}

/* Small-batch selection and dispatch (T*K <= 256) by one block of 256
 * threads: a wave per token for the top-k, then the stable counting sort of
 * the T*K pairs by expert.  Each expert keeps an LDS membership mask over
 * the pairs (8 words); its popcount is the expert's count, a block scan of
 * the counts gives the offsets and the active-expert ranks, and a pair's
 * rank inside its expert is the popcount of the mask below it. */
template <int EPL, bool COH>
DEV void topk_dispatch_block(const RouteArgs &a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tid = threadIdx.x;
    const int E = a.E, T = a.T, K = a.K, NP = T * K;
    __shared__ int s_e[256];
    __shared__ uint32_t mask[64 * EPL * 8]; /* experts (< 64 EPL) x 8 words of pair bits */
    __shared__ uint32_t eoff[64 * EPL];
    __shared__ uint32_t wsum[4];
    for (int i = tid; i < 64 * EPL * 8; i += 256) mask[i] = 0;
    for (int t = wv; t < T; t += 4)
        wave_topk<EPL, COH>(a.logits + (size_t)t * (E + 1), a.bias, E, K, lane, a.idx + t * K,
                            a.w + t * K, a.sgl + t, s_e + t * K);
    __syncthreads();
    if (tid < NP) atomicOr(&mask[s_e[tid] * 8 + (tid >> 5)], 1u << (tid & 31));
    __syncthreads();
    /* thread tid owns experts [tid*EPT, tid*EPT + EPT), EPT = EPL/4 (E <= 64 EPL) */
    constexpr int EPT = EPL >= 4 ? EPL / 4 : 1;
    uint32_t cnt[EPT], packed = 0;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid * EPT + j;
        uint32_t c = 0;
        if (e < E)
#pragma unroll
            for (int w = 0; w < 8; w++) c += __popc(mask[e * 8 + w]);
        cnt[j] = c;
        packed += (c << 16) | (c != 0); /* count <= 256 in the high half, active count low */
    }
    uint32_t total;
    const uint32_t ex = block_excl_scan256(packed, wsum, &total);
    uint32_t off = ex >> 16, rank = ex & 0xFFFFu;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid * EPT + j;
        if (e < E) {
            eoff[e] = off;
            a.offsets[e] = off;
            if (cnt[j]) {
                ACT_E(a.list, rank) = (uint32_t)e;
                ACT_OFF(a.list, E, rank) = off;
                rank++;
            }
            off += cnt[j];
        }
    }
    if (tid == 0) {
        const uint32_t n = total & 0xFFFFu;
        a.offsets[E] = (uint32_t)NP;
        ACT_N(a.list) = n;
        ACT_OFF(a.list, E, n) = (uint32_t)NP;
    }
    __syncthreads();
    if (tid < NP) {
        const int e = s_e[tid], wd = tid >> 5;
        uint32_t r = __popc(mask[e * 8 + wd] & ((1u << (tid & 31)) - 1u));
        for (int w = 0; w < wd; w++) r += __popc(mask[e * 8 + w]);
        const uint32_t pos = eoff[e] + r;
        a.pairs[pos] = (uint32_t)tid;
        a.pos[tid] = pos;
    }
}

/* Block-local routing for T*K <= 256 by one block of 256 threads: the
 * top-k of every token and the dispatch of its pairs, all in LDS.  With
 * `publish` the block also writes the call's routing outputs (idx, w, sgl,
 * offsets, pairs, pos, active list) for later kernels. */
struct RouteLds {
    int e[256];        /* expert of pair p = t*K + k */
    float w[256];      /* weight of pair p */
    float sgl[16];     /* shared-gate logit per token */
    int pairs[256];    /* sorted position -> pair */
    int pos[256];      /* pair -> sorted position */
    int head[256];
    int act_e[256];    /* active slot -> expert (ascending) */
    int act_off[257];  /* active slot -> first sorted position */
    int nact;
};

template <int EPL>
DEV void route_block_lds(const RouteArgs &a, RouteLds &r, bool publish) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int E = a.E, T = a.T, K = a.K, NP = T * K, p = threadIdx.x;
    for (int t = wv; t < T; t += 4)
        wave_topk<EPL, false>(a.logits + (size_t)t * (E + 1), a.bias, E, K, lane, r.e + t * K,
                              r.w + t * K, r.sgl + t, nullptr);
    __syncthreads();
    int e = 0, less = 0, before = 0;
    if (p < NP) {
        e = r.e[p];
        for (int q = 0; q < NP; q++) {
            const int eq = r.e[q];
            less += eq < e;
            before += (q < p) & (eq == e);
        }
        const int ps = less + before;
        r.pairs[ps] = p;
        r.pos[p] = ps;
        r.head[p] = before == 0;
    }
    __syncthreads();
    if (p < NP && r.head[p]) {
        int rank = 0;
        for (int q = 0; q < NP; q++) rank += r.head[q] & (r.e[q] < e);
        r.act_e[rank] = e;
        r.act_off[rank] = less;
    }
    if (p == 0) {
        int n = 0;
        for (int q = 0; q < NP; q++) n += r.head[q];
        r.nact = n;
        r.act_off[n] = NP;
    }
    __syncthreads();
    if (!publish) return;
    if (p < NP) {
        a.idx[p] = r.e[p];
        a.w[p] = r.w[p];
        a.pairs[p] = (uint32_t)r.pairs[p];
        a.pos[p] = (uint32_t)r.pos[p];
    }
    if (p < T) a.sgl[p] = r.sgl[p];
    if (p <= r.nact) ACT_OFF(a.list, E, p) = (uint32_t)r.act_off[p];
    if (p < r.nact) ACT_E(a.list, p) = (uint32_t)r.act_e[p];
    if (p == 0) ACT_N(a.list) = (uint32_t)r.nact;
    for (int ee = p; ee <= E; ee += 256) {
        int c = 0;
        for (int q = 0; q < NP; q++) c += r.e[q] < ee;
        a.offsets[ee] = (uint32_t)c;
    }
}
