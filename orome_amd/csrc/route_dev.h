/* route_dev.h -- device-side expert selection shared by the routing and
 * decode kernels.
 *
 * Selection restates softmax_topk_route (inference/src/shaders.metal:
 * 1141-1234): K rounds of argmax, exact ties to the lower expert index (the
 * contract's rule; the reference's shuffle-down tree, 1166-1200, settles an
 * exact tie by tree position instead), softmax over
 * the K winners.  A round is a wave64 max over order-preserving 32-bit images
 * of the values; the lowest lane holding the maximum (lane order is expert
 * order) settles ties.
 */
#pragma once
#include "dev_common.h"
#include "kernels.h"

/* -------------------------------------------------------- key helpers */
/* Order-preserving 32-bit image of a float (larger float -> larger key);
 * -0 is folded into +0 so the two tie, as in an IEEE compare.  Key 0 (the
 * image of one NaN pattern, outside the contract) marks taken or absent
 * entries. */
DEV uint32_t route_ord(float v) {
    if (v == 0.0f) v = 0.0f;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
DEV float ord_value(uint32_t ord) {
    const uint32_t b = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
    return __builtin_bit_cast(float, b);
}

/* wave64 maximum of a 32-bit key, returned wave-uniform: DPP maxima within
 * rows of 16 lanes, then the four row maxima */
DEV uint32_t wave_max_u32(uint32_t m) {
    m = max(m, dppu<DPP_XOR1>(m));
    m = max(m, dppu<DPP_XOR2>(m));
    m = max(m, dppu<DPP_HALF_MIRROR>(m));
    m = max(m, dppu<DPP_MIRROR>(m));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)m, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)m, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)m, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)m, 48);
    /* on the scalar unit (left to itself the compiler copies b and d back
     * into vector registers for one v_max3); s_max writes SCC */
    uint32_t ab, cd, r;
    asm("s_max_u32 %0, %1, %2" : "=s"(ab) : "s"(a), "s"(b) : "scc");
    asm("s_max_u32 %0, %1, %2" : "=s"(cd) : "s"(c), "s"(d) : "scc");
    asm("s_max_u32 %0, %1, %2" : "=s"(r) : "s"(ab), "s"(cd) : "scc");
    return r;
}

/* One token's top-K on one wave.  Lane L owns the EPL consecutive experts
 * EPL*L .. EPL*L + EPL-1, so lane order is expert order.  Each lane first
 * sorts its keys (adjacent compare-exchanges that swap only on a strictly
 * larger right-hand key, hence stable: equal keys keep index order); a
 * round then takes the wave maximum of the lanes' heads and the lowest lane
 * holding it -- the lowest expert index among equal values, the contract's
 * rule for exact ties -- and that lane pops its head.  All round state
 * except the lane's list is wave-uniform (scalar registers), and the rounds
 * form a rolled loop (each wave runs them once: unrolled, every round would
 * be fetched cold).  Lane k < K ends with the k-th expert and its softmax
 * weight (softmax over the winners, summed in k order as the reference's
 * loop does); lanes < K write idx_out/w_out/e_out (each may be NULL) and
 * lane 0 the shared-gate logit. */
struct TopkLane {
    int id;
    float w;
};
template <int EPL>
DEV TopkLane wave_topk_keys(uint32_t *key, float sg, int K, int lane, int32_t *idx_out, float *w_out,
                            float *sgl_out, int *e_out);
template <int EPL, bool COH = false>
DEV TopkLane wave_topk(const float *l, const float *bias, int E, int K, int lane, int32_t *idx_out,
                       float *w_out, float *sgl_out, int *e_out) {
    /* all loads first and unconditional (index clamped, then masked), so
     * they are in flight together instead of one round trip each */
    float v[EPL], bv[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = min(lane * EPL + j, E - 1);
        v[j] = COH ? ld_coh(l + e) : l[e];
    }
    const float sg = COH ? ld_coh(l + E) : l[E];
    if (bias)
#pragma unroll
        for (int j = 0; j < EPL; j++) bv[j] = bias[min(lane * EPL + j, E - 1)];
    uint32_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) key[j] = lane * EPL + j < E ? route_ord(bias ? v[j] + bv[j] : v[j]) : 0u;
    return wave_topk_keys<EPL>(key, sg, K, lane, idx_out, w_out, sgl_out, e_out);
}

/* The selection of wave_topk from the lanes' keys (key 0: not eligible). */
template <int EPL>
DEV TopkLane wave_topk_keys(uint32_t *key, float sg, int K, int lane, int32_t *idx_out, float *w_out,
                            float *sgl_out, int *e_out) {
    int kj[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) kj[j] = j;
    /* odd-even transposition sort, descending */
#pragma unroll
    for (int pass = 0; pass < EPL; pass++)
#pragma unroll
        for (int j = pass & 1; j + 1 < EPL; j += 2)
            if (key[j + 1] > key[j]) {
                const uint32_t tk = key[j]; key[j] = key[j + 1]; key[j + 1] = tk;
                const int tj = kj[j]; kj[j] = kj[j + 1]; kj[j + 1] = tj;
            }
    int id = 0;
    float val = 0.0f, v0 = 0.0f;
#pragma unroll 1
    for (int k = 0; k < K; k++) {
        const uint32_t m = wave_max_u32(key[0]);
        const int wl = (int)__builtin_ctzll(__ballot(key[0] == m));
        const int e = wl * EPL + __builtin_amdgcn_readlane(kj[0], wl);
        const float vk = ord_value(m);
        if (lane == k) { id = e; val = vk; }
        if (k == 0) v0 = vk;
        if (lane == wl) {
#pragma unroll
            for (int j = 0; j + 1 < EPL; j++) { key[j] = key[j + 1]; kj[j] = kj[j + 1]; }
            key[EPL - 1] = 0u;
        }
    }
    const float tw = lane < K ? expf(val - v0) : 0.0f;
    float sum = 0.0f;
#pragma unroll 1
    for (int k = 0; k < K; k++)
        sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tw), k));
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    const float w = tw * inv;
    if (lane < K) {
        if (idx_out) idx_out[lane] = id;
        if (w_out) w_out[lane] = w;
        if (e_out) e_out[lane] = id;
    }
    if (lane == 0 && sgl_out) *sgl_out = sg;
    return TopkLane{id, w};
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
    if (lane == 63 && wv < 4) wsum[wv] = inc;
    lds_barrier();
    uint32_t base = 0;
    for (int w = 0; w < min(wv, 4); w++) base += wsum[w];
    *total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    return base + inc - v;
}

/* Small-batch selection and dispatch (T*K <= 256) by one block of 256 or
 * more threads (the first 256 count and scan; threads past them only take
 * part in the selection): a wave per token for the top-k, then the stable
 * counting sort of
 * the T*K pairs by expert.  Each expert keeps an LDS membership mask over
 * the pairs (8 words); its popcount is the expert's count, a block scan of
 * the counts gives the offsets and the active-expert ranks, and a pair's
 * rank inside its expert is the popcount of the mask below it. */
template <int EPL, bool COH>
DEV void topk_dispatch_block(const RouteArgs &a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tid = threadIdx.x, nw = (int)(blockDim.x >> 6);
    const int E = a.E, T = a.T, K = a.K, NP = T * K;
    __shared__ int s_e[256];
    __shared__ uint32_t mask[64 * EPL * 8]; /* experts (< 64 EPL) x 8 words of pair bits */
    __shared__ uint32_t eoff[64 * EPL];
    __shared__ uint32_t wsum[4];
    for (int i = tid; i < 64 * EPL * 8; i += (int)blockDim.x) mask[i] = 0;
    for (int t = wv; t < T; t += nw)
        wave_topk<EPL, COH>(a.logits + (size_t)t * (E + 1), a.bias, E, K, lane, a.idx + t * K,
                            a.w + t * K, a.sgl + t, s_e + t * K);
    lds_barrier();
    if (tid < NP) atomicOr(&mask[s_e[tid] * 8 + (tid >> 5)], 1u << (tid & 31));
    lds_barrier();
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
                if (a.tiles_s) { /* T <= 16 rows: one small tile */
                    a.tiles_s[1 + 3 * rank] = (uint32_t)e;
                    a.tiles_s[2 + 3 * rank] = off;
                    a.tiles_s[3 + 3 * rank] = cnt[j];
                }
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
        if (a.tiles_s) {
            if (a.has_shared) {
                a.tiles_s[1 + 3 * n] = (uint32_t)E;
                a.tiles_s[2 + 3 * n] = 0u;
                a.tiles_s[3 + 3 * n] = (uint32_t)T;
            }
            a.tiles_s[0] = n + (a.has_shared ? 1u : 0u);
        }
    }
    lds_barrier();
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

/* Canonical dots of one wave over H (H % 256 == 0, H <= 256 NIM) for up to
 * TMAX tokens, with NORM x = RMSNorm(h) computed in place (RMSNorm of
 * inference/src/shaders.metal:128-149, the same arithmetic and canonical sum
 * of squares as k_rmsnorm, so x is bit-identical to that kernel's output;
 * write_x stores it for the later kernels).  Tokens go in chunks of up to 4
 * whose row loads are issued together with the router row's; every load is
 * unconditional (indices clamped, values past T or H unused), since a load
 * under a branch is waited for alone.  A NULL wrow gives zeros. */
template <int TMAX, int NIM, bool NORM>
DEV void canon_dots(const float *wrow, const RouteArgs &a, int lane, bool write_x, float *acc, int tb = 0,
                    f4 *xlds = nullptr, const f4 *xpart = nullptr) {
    /* tokens tb .. tb + TMAX - 1 (acc[t - tb]) */
    /* write_x also stages fp16(x) into a.x16 when set (round to nearest
     * even, each 4-group stored (0,2,1,3), the grouped GEMMs' layout) */
    constexpr int TC = TMAX < 4 ? TMAX : 4;
    const int NI = a.H / 256, H = a.H, T = a.T - tb;
    const float *xs = (NORM ? a.norm_h : a.x) + (size_t)tb * a.H;
    f4 wv[NIM], nw[NIM];
#pragma unroll
    for (int i = 0; i < NIM; i++) {
        const int ic = 256 * min(i, NI - 1) + 4 * lane;
        wv[i] = *(const f4 *)((wrow ? wrow : xs) + ic);
        if (NORM) nw[i] = *(const f4 *)((a.norm_w ? a.norm_w : xs) + ic);
    }
    /* xlds (one token, H <= 2048, every wave of the block calls this): the
     * block's threads hold x (or the norm input) in xpart, two 16-byte
     * pieces each; it is stored into LDS once and read back from there
     * (the waves would otherwise each fetch the whole row) */
    if (xlds) {
        const int q = threadIdx.x;
        xlds[q] = xpart[0];
        xlds[q + 256] = xpart[1];
        lds_barrier();
    }
#pragma unroll
    for (int t0 = 0; t0 < TMAX; t0 += TC) {
        if (t0 >= T) break;
        f4 hv[TC][NIM];
#pragma unroll
        for (int c = 0; c < TC; c++)
#pragma unroll
            for (int i = 0; i < NIM; i++)
                hv[c][i] = xlds ? xlds[(256 * min(i, NI - 1) + 4 * lane) >> 2]
                                : *(const f4 *)(xs + (size_t)min(t0 + c, T - 1) * H + 256 * min(i, NI - 1) + 4 * lane);
        if (t0 == 0) {
#pragma unroll
            for (int i = 0; i < NIM; i++) {
                if (!wrow) wv[i] = f4{0, 0, 0, 0};
                if (NORM) {
                    const f4 w = a.norm_w ? nw[i] : f4{1, 1, 1, 1};
                    nw[i] = f4{__builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.x) & 0xFFFF0000u),
                               __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.y) & 0xFFFF0000u),
                               __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.z) & 0xFFFF0000u),
                               __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w.w) & 0xFFFF0000u)};
                }
            }
        }
#pragma unroll
        for (int c = 0; c < TC; c++) {
            const int t = t0 + c;
            acc[t] = 0.0f;
            if (t >= T || (!NORM && !wrow)) continue;
            float scale = 1.0f;
            if (NORM) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < NIM; i++)
                    if (i < NI) {
                        ss = __builtin_fmaf(hv[c][i].x, hv[c][i].x, ss);
                        ss = __builtin_fmaf(hv[c][i].y, hv[c][i].y, ss);
                        ss = __builtin_fmaf(hv[c][i].z, hv[c][i].z, ss);
                        ss = __builtin_fmaf(hv[c][i].w, hv[c][i].w, ss);
                    }
                ss = wave_sum_canon(ss);
                scale = 1.0f / sqrtf(ss / (float)H + a.norm_eps);
            }
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < NIM; i++)
                if (i < NI) {
                    f4 x = hv[c][i];
                    if (NORM) {
                        x = f4{(x.x * scale) * nw[i].x, (x.y * scale) * nw[i].y, (x.z * scale) * nw[i].z,
                               (x.w * scale) * nw[i].w};
                        if (write_x) *(f4 *)(a.xnorm + (size_t)(tb + t) * H + 256 * i + 4 * lane) = x;
                    }
                    if (write_x && a.x16)
                        *(h4 *)(a.x16 + (size_t)(tb + t) * H + 256 * i + 4 * lane) =
                            h4{(_Float16)x.x, (_Float16)x.z, (_Float16)x.y, (_Float16)x.w};
                    d = __builtin_fmaf(wv[i].x, x.x, d);
                    d = __builtin_fmaf(wv[i].y, x.y, d);
                    d = __builtin_fmaf(wv[i].z, x.z, d);
                    d = __builtin_fmaf(wv[i].w, x.w, d);
                }
            acc[t] = wave_sum_canon(d);
        }
    }
}
