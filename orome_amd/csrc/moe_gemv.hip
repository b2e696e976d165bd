/*
 * moe_gemv.hip -- decode-path (T <= 8) expert products: fused dequant GEMV.
 *
 * Bandwidth-bound: every weight byte is read once per call, the expert set
 * is deduplicated across the batch (one pass per active expert, over the
 * tokens routed to it), and no matrix cores are used.
 *
 * Work unit ("chunk") = 32 weights of one row, held by one lane:
 *   Q4_K  a 16-byte run of quant bytes (16 low + 16 high nibbles) plus the
 *         super-block header (d, dmin, scales; eight lanes share it);
 *   Q6_K  8 positions l of one 128-weight half: 4 x 8 weights at l, l+32,
 *         l+64, l+96 (ql/qh bytes, four int8 scales);
 *   Q8_0  one 34-byte block.
 * Quants become exact fp16 values (v_perm into the 0x64xx exponent, minus
 * the bias), are multiplied with fp16 activations by v_dot2_f32_f16 (exact
 * products, fp32 sums), and the per-sub-block scale/min is applied in fp32:
 *   sum_j (a*q_j - b) x_j = a * sum_j q_j x_j - b * sum_j x_j.
 * Activations are rounded to fp16 exactly as the reference stages them
 * (half(x): inference/src/shaders.metal:2252-2255, 2612-2613).
 *
 * Restates batch_expert_gate_up_swiglu_q4k_dyn (shaders.metal:2232-2310),
 * shared_gate_up_swiglu_q4k/_q8_0 (2316-2445), batch_expert_down_q4k_dyn
 * (2590-2668), dequant_matvec_q6k/_q8_0 (1888-1988, 1627-1701) and
 * moe_combine_copy_sq_k8 (1079-1135).
 */
#include "dev_common.h"
#include "kernels.h"
#include "route_dev.h"


enum { FQ4K = 0, FQ5K = 1, FQ6K = 2, FQ8 = 3 };

static __host__ __device__ __forceinline__ size_t row_bytes(int fmt, int n) {
    return fmt == FQ4K ? (size_t)(n / 256) * 144 : fmt == FQ5K ? (size_t)(n / 256) * 176
           : fmt == FQ6K ? (size_t)(n / 256) * 210 : (size_t)(n / 32) * 34;
}

/* 16 consecutive fp32 -> 8 fp16 pairs (RNE) and the sum of the rounded values */
DEV float load_x16_f32(const float *p, h2 *o) {
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        f4 a = *(const f4 *)(p + 4 * v);
        o[2 * v] = h2{(_Float16)a.x, (_Float16)a.y};
        o[2 * v + 1] = h2{(_Float16)a.z, (_Float16)a.w};
    }
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int v = 0; v < 8; v++) s = dot2(o[v], one, s);
    return s;
}
/* load_x16_f32 on 16 floats already loaded */
DEV float cvt_x16_f32(const f4 *a, h2 *o) {
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        o[2 * v] = h2{(_Float16)a[v].x, (_Float16)a[v].y};
        o[2 * v + 1] = h2{(_Float16)a[v].z, (_Float16)a[v].w};
    }
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int v = 0; v < 8; v++) s = dot2(o[v], one, s);
    return s;
}
/* 8 consecutive fp16 (16 bytes) -> 4 pairs; LX: p points into LDS */
template <bool LX = false>
DEV void load_h8(const _Float16 *p, h2 *o) {
    u4 v;
    if constexpr (LX) v = *(const __attribute__((address_space(3))) u4 *)p;
    else v = ld_u4((const uint8_t *)p);
    o[0] = as_h2(v.x); o[1] = as_h2(v.y); o[2] = as_h2(v.z); o[3] = as_h2(v.w);
}
DEV float hsum(const h2 *o, int n) {
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
    float s = 0.0f;
    for (int v = 0; v < n; v++) s = dot2(o[v], one, s);
    return s;
}

/* Q4_K chunk: raw bytes */
struct Q4Raw {
    u4 q, hdr;
};
DEV Q4Raw q4_load(const uint8_t *row, int c) {
    const uint8_t *sb = row + (c >> 3) * 144;
    return Q4Raw{ld_u4(sb + 16 + (c & 7) * 16), ld_u4(sb)};
}
/* the same with streaming loads (`nt`), for the routed experts of the
 * one-token gate/up: read once, they would push the shared expert, the
 * touched down rows and the router out of the last-level cache */
DEV Q4Raw q4_load_nt(const uint8_t *row, int c) {
    const uint8_t *sb = row + (c >> 3) * 144;
    return Q4Raw{ld_u4_nt(sb + 16 + (c & 7) * 16), ld_u4_nt(sb)};
}
DEV void q4_pos(int c, int &klo) { klo = (c >> 3) * 256 + ((c & 7) >> 1) * 64 + (c & 1) * 16; }
DEV float q4_dot(const Q4Raw &r, int c, const h2 *xl, const h2 *xh, float Xl, float Xh) {
    Q4Affine af = q4k_affine(r.hdr, (c & 7) >> 1);
    float sl = 0.0f, sh = 0.0f;
    uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        h2 l01, l23, h01, h23;
        q4_nibbles_h2(w[d], l01, l23, h01, h23);
        sl = dot2(l01, xl[2 * d], sl);
        sl = dot2(l23, xl[2 * d + 1], sl);
        sh = dot2(h01, xh[2 * d], sh);
        sh = dot2(h23, xh[2 * d + 1], sh);
    }
    return (af.a_lo * sl + af.a_hi * sh) - (af.b_lo * Xl + af.b_hi * Xh);
}

/* Q5_K chunk: the same positions as a Q4_K chunk (16 ql bytes, the 16 qh
 * bytes of those positions, the header) */
struct Q5Raw {
    u4 q, qh, hdr;
};
DEV Q5Raw q5_load(const uint8_t *row, int c) {
    const uint8_t *sb = row + (c >> 3) * 176;
    return Q5Raw{ld_u4(sb + 48 + (c & 7) * 16), ld_u4(sb + 16 + (c & 1) * 16), ld_u4(sb)};
}
DEV float q5_dot(const Q5Raw &r, int c, const h2 *xl, const h2 *xh, float Xl, float Xh) {
    const int g = (c & 7) >> 1;
    Q4Affine af = q4k_affine(r.hdr, g);
    float sl = 0.0f, sh = 0.0f;
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, hb[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        h2 l01, l23, h01, h23;
        q5_bias_h2(w[d], hb[d], g, l01, l23, h01, h23);
        sl = dot2(l01 - bias, xl[2 * d], sl);
        sl = dot2(l23 - bias, xl[2 * d + 1], sl);
        sh = dot2(h01 - bias, xh[2 * d], sh);
        sh = dot2(h23 - bias, xh[2 * d + 1], sh);
    }
    return (af.a_lo * sl + af.a_hi * sh) - (af.b_lo * Xl + af.b_hi * Xh);
}

/* Q8_0 chunk = block c */
struct Q8Raw {
    u4 q0, q1;
    uint32_t d;
};
DEV Q8Raw q8_load(const uint8_t *row, int c) {
    const uint8_t *b = row + c * 34;
    return Q8Raw{ld_u32x4_a2(b + 2), ld_u32x4_a2(b + 18), ld_u32_a2(b)};
}
DEV float q8_dot(const Q8Raw &r, const h2 *x /*16 pairs*/) {
    uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float s = 0.0f;
#pragma unroll
    for (int d = 0; d < 8; d++) {
        h2 p01, p23;
        q8_h2(w[d], p01, p23);
        s = dot2(p01, x[2 * d], s);
        s = dot2(p23, x[2 * d + 1], s);
    }
    return f16_bits_to_f32(r.d) * s;
}

/* Q6_K chunk c: sb = c>>3, half h = (c>>2)&1, positions l0 = 8*(c&3) .. +7 */
struct Q6Raw {
    u2 qa, qb, qh, sc;
    uint32_t d;
};
DEV Q6Raw q6_load(const uint8_t *row, int c) {
    const uint8_t *sb = row + (c >> 3) * 210;
    const int h = (c >> 2) & 1, l0 = 8 * (c & 3);
    return Q6Raw{ld_u32x2_a2(sb + h * 64 + l0), ld_u32x2_a2(sb + h * 64 + 32 + l0),
                 ld_u32x2_a2(sb + 128 + h * 32 + l0), ld_u32x2_a2(sb + 192 + h * 8),
                 ld_u32_a2(sb + 208)};
}
DEV void q6_pos(int c, int &k0) { k0 = (c >> 3) * 256 + ((c >> 2) & 1) * 128 + 8 * (c & 3); }
DEV float sc8(u2 sc, int i) {
    uint32_t w = i < 4 ? sc.x : sc.y;
    return (float)(int8_t)((w >> (8 * (i & 3))) & 0xFF);
}
/* x: 4 groups (offsets 0, 32, 64, 96) of 4 pairs */
DEV float q6_dot(const Q6Raw &r, int c, const h2 *x) {
    float s[4] = {0, 0, 0, 0};
    uint32_t qa[2] = {r.qa.x, r.qa.y}, qb[2] = {r.qb.x, r.qb.y}, qh[2] = {r.qh.x, r.qh.y};
#pragma unroll
    for (int m = 0; m < 2; m++) {
        h2 p01, p23;
        q6_h2(qa[m], qh[m], 0, 0, p01, p23);
        s[0] = dot2(p01, x[0 * 4 + 2 * m], s[0]);
        s[0] = dot2(p23, x[0 * 4 + 2 * m + 1], s[0]);
        q6_h2(qb[m], qh[m], 0, 2, p01, p23);
        s[1] = dot2(p01, x[1 * 4 + 2 * m], s[1]);
        s[1] = dot2(p23, x[1 * 4 + 2 * m + 1], s[1]);
        q6_h2(qa[m], qh[m], 4, 4, p01, p23);
        s[2] = dot2(p01, x[2 * 4 + 2 * m], s[2]);
        s[2] = dot2(p23, x[2 * 4 + 2 * m + 1], s[2]);
        q6_h2(qb[m], qh[m], 4, 6, p01, p23);
        s[3] = dot2(p01, x[3 * 4 + 2 * m], s[3]);
        s[3] = dot2(p23, x[3 * 4 + 2 * m + 1], s[3]);
    }
    const int is = (c & 3) >> 1;
    float d = f16_bits_to_f32(r.d);
    return d * (sc8(r.sc, is) * s[0] + sc8(r.sc, is + 2) * s[1] + sc8(r.sc, is + 4) * s[2] +
                sc8(r.sc, is + 6) * s[3]);
}

/* =================================================================== */
/* gate/up + SiLU-GLU.  Block = 4 waves x RPW rows (gate and up of each row).
 * Grid = [routed blocks: Umax slots x M/(4*RPW)] + [shared: S/(4*RPW)]. */
struct GUArgs {
    const uint8_t *gate, *up;
    size_t gate_stride, up_stride;
    const uint8_t *sh_gate, *sh_up;
    int sh_fmt, S;
    const float *x;
    int T, H, M, K, E;
    const uint32_t *list, *pairs;
    _Float16 *act, *act_sh;
    int routed_blocks;
    unsigned long long *kt; /* per-block launch stamps (KT_BEGIN / KT_END) or NULL */
    /* T = 1: the down matrices the next kernel reads (row-major, pf_rb bytes
     * a row, H rows), touched one 4-byte load per 128-byte line so that they
     * are on their way to the caches while this kernel waits; NULL: none */
    const uint8_t *pf_down, *pf_sh_down;
    size_t pf_down_stride;
    int pf_rb, pf_sh_rb;
    /* T = 1: act row k holds the expert of selection round k (slot order)
     * instead of its sorted position, so the down + combine kernel can load
     * the act rows without waiting for the routing */
    int act_by_slot;
};

/* One 4-byte load per 128-byte line of two of the 8-row groups g = i,
 * i + step, i + 2 step, ... (< H / 8) of a row-major matrix, the pair
 * starting at group slot s0: the rows that the T = 1 down kernel's blocks g
 * read, from a block on the same XCD as they are (g = i mod 8).  The value
 * lands in `sink`, which the caller keeps until a wait for it. */
DEV void touch_rows8(const uint8_t *m, int rb, int H, int i, int step, int s0, int lane, uint32_t &sink) {
    const int nl = (8 * rb + 127) / 128, g = i + step * (s0 + lane / nl);
    if (lane / nl >= 2 || g >= H / 8) return;
    const uint8_t *p = m + (size_t)g * 8 * rb + min((lane % nl) * 128, 8 * rb - 4);
    asm volatile("global_load_dword %0, %1, off" : "=v"(sink) : "v"(p) : "memory");
}

/* One wave: RPW gate rows and RPW up rows for the n tokens of a slot.  Raw
 * weight chunks of all rows are loaded first; the token loop is a runtime
 * loop (register use does not grow with the batch), and each (row, token)
 * sum is reduced across the wave at once.  Lane 0 keeps running totals in
 * `red` when a row needs more than one pass of 64 chunks (H > 2048). */
template <int RPW, int SFMT>
DEV void gu_body(const GUArgs &a, const uint8_t *gbase, const uint8_t *ubase, int r0, int n,
                 const int *tok, _Float16 *out, int out_ld, int lane, float *red) {
    const int H = a.H, NC = H / 32;
    const size_t rb = SFMT == FQ8 ? row_bytes(FQ8, H) : row_bytes(FQ4K, H);
    for (int c0 = 0; c0 < NC; c0 += 64) {
        const int c = c0 + lane;
        const bool live = c < NC;
        const int cc = live ? c : c0;
        int klo, khi;
        if (SFMT == FQ8) { klo = cc * 32; khi = klo + 16; }
        else { q4_pos(cc, klo); khi = klo + 32; }
        if (SFMT == FQ8) {
            Q8Raw g[RPW], u[RPW];
#pragma unroll
            for (int i = 0; i < RPW; i++) {
                g[i] = q8_load(gbase + (size_t)(r0 + i) * rb, cc);
                u[i] = q8_load(ubase + (size_t)(r0 + i) * rb, cc);
            }
            for (int j = 0; j < n; j++) {
                h2 x[16];
                load_x16_f32(a.x + (size_t)tok[j] * H + klo, x);
                load_x16_f32(a.x + (size_t)tok[j] * H + khi, x + 8);
#pragma unroll
                for (int i = 0; i < RPW; i++) {
                    float pg = live ? q8_dot(g[i], x) : 0.0f, pu = live ? q8_dot(u[i], x) : 0.0f;
                    pg = wave_sum_fast(pg);
                    pu = wave_sum_fast(pu);
                    if (lane == 0) {
                        red[(i * 2) * 16 + j] += pg;
                        red[(i * 2 + 1) * 16 + j] += pu;
                    }
                }
            }
        } else {
            Q4Raw g[RPW], u[RPW];
#pragma unroll
            for (int i = 0; i < RPW; i++) {
                g[i] = q4_load(gbase + (size_t)(r0 + i) * rb, cc);
                u[i] = q4_load(ubase + (size_t)(r0 + i) * rb, cc);
            }
            for (int j = 0; j < n; j++) {
                h2 xl[8], xh[8];
                float Xl = load_x16_f32(a.x + (size_t)tok[j] * H + klo, xl);
                float Xh = load_x16_f32(a.x + (size_t)tok[j] * H + khi, xh);
#pragma unroll
                for (int i = 0; i < RPW; i++) {
                    float pg = live ? q4_dot(g[i], cc, xl, xh, Xl, Xh) : 0.0f;
                    float pu = live ? q4_dot(u[i], cc, xl, xh, Xl, Xh) : 0.0f;
                    pg = wave_sum_fast(pg);
                    pu = wave_sum_fast(pu);
                    if (lane == 0) {
                        red[(i * 2) * 16 + j] += pg;
                        red[(i * 2 + 1) * 16 + j] += pu;
                    }
                }
            }
        }
    }
    if (lane == 0)
        for (int j = 0; j < n; j++)
#pragma unroll
            for (int i = 0; i < RPW; i++)
                out[(size_t)j * out_ld + r0 + i] =
                    glu_f16(red[(i * 2) * 16 + j], red[(i * 2 + 1) * 16 + j]);
}

/* One token, H = 2048 (one 32-weight chunk per lane): x arrives already
 * converted (loaded before the routing), so only the weight bytes are
 * waited for once the experts are known.  Same sums as gu_body. */
template <int RPW>
DEV void gu_body1(const GUArgs &a, const uint8_t *gbase, const uint8_t *ubase, int r0, const h2 *xl,
                  const h2 *xh, float Xl, float Xh, _Float16 *out, int lane) {
    const size_t rb = row_bytes(FQ4K, a.H);
    Q4Raw g[RPW], u[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        g[i] = q4_load(gbase + (size_t)(r0 + i) * rb, lane);
        u[i] = q4_load(ubase + (size_t)(r0 + i) * rb, lane);
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const float pg = wave_sum_fast(q4_dot(g[i], lane, xl, xh, Xl, Xh));
        const float pu = wave_sum_fast(q4_dot(u[i], lane, xl, xh, Xl, Xh));
        if (lane == 0) out[r0 + i] = glu_f16(pg, pu);
    }
}

#ifndef GU_RPW
#define GU_RPW 2
#endif
/* Decode gate/up with the routing folded in: routed blocks select the
 * experts themselves from the router logits (block 0 publishes the routing
 * for the down kernel); shared-expert blocks start at once. */
template <int EPL, bool ROUTE>
DEV void k_gemv_gate_up_body(GUArgs a, RouteArgs ra) {
    __shared__ float red_all[4][GU_RPW * 2 * 16];
    __shared__ int tok[16];
    __shared__ RouteLds r;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int rows_blk = 4 * GU_RPW;
    float *red = red_all[wv];
    for (int i = lane; i < GU_RPW * 2 * 16; i += 64) red[i] = 0.0f;
    int b = blockIdx.x;
    if (b < a.routed_blocks) {
        const int bpe = a.M / rows_blk;
        const int u = b / bpe, tile = b % bpe;
        int e, s0, n;
        if constexpr (ROUTE) {
            route_block_lds<EPL>(ra, r, b == 0);
            if (u >= r.nact) return;
            e = r.act_e[u];
            s0 = r.act_off[u];
            n = r.act_off[u + 1] - s0;
            if (threadIdx.x < n) tok[threadIdx.x] = r.pairs[s0 + threadIdx.x] / a.K;
        } else {
            if ((uint32_t)u >= ACT_N(a.list)) return;
            e = (int)ACT_E(a.list, u);
            s0 = (int)ACT_OFF(a.list, a.E, u);
            n = (int)ACT_OFF(a.list, a.E, u + 1) - s0;
            if (threadIdx.x < n) tok[threadIdx.x] = (int)(a.pairs[s0 + threadIdx.x] / (uint32_t)a.K);
        }
        __syncthreads();
        gu_body<GU_RPW, FQ4K>(a, a.gate + (size_t)e * a.gate_stride, a.up + (size_t)e * a.up_stride,
                              tile * rows_blk + wv * GU_RPW, n, tok, a.act + (size_t)s0 * a.M, a.M, lane, red);
    } else {
        const int tile = b - a.routed_blocks;
        if (threadIdx.x < a.T) tok[threadIdx.x] = threadIdx.x;
        __syncthreads();
        const int r0 = tile * rows_blk + wv * GU_RPW;
        if (a.sh_fmt == FQ8)
            gu_body<GU_RPW, FQ8>(a, a.sh_gate, a.sh_up, r0, a.T, tok, a.act_sh, a.S, lane, red);
        else
            gu_body<GU_RPW, FQ4K>(a, a.sh_gate, a.sh_up, r0, a.T, tok, a.act_sh, a.S, lane, red);
    }
}

template <int EPL, bool ROUTE>
__global__ __launch_bounds__(256) void k_gemv_gate_up(GUArgs a, RouteArgs ra) {
    KT_BEGIN(a.kt);
    k_gemv_gate_up_body<EPL, ROUTE>(a, ra);
    KT_END(a.kt);
}

/* a lane's EPL in-lane positions, four bits each */
template <int EPL>
struct PosPack {
    typedef uint32_t type;
};
template <>
struct PosPack<16> {
    typedef uint64_t type;
};
/* One-token gate/up with the routing folded in (H = 2048, E <= 64 EPL): no
 * separate top-k kernel.  In each block one wave runs the selection rounds
 * on the router's logits; the block's waves, all for selection rank u, wait
 * at a barrier that it passes as soon as round u has named the expert, and
 * then issue their weight loads for it.  The remaining rounds, the expert's
 * sorted position (the number of smaller selected ids: its act row, unless
 * act rows go in slot order) and, in block 0, the call's selections and
 * weights overlap those loads; block 0's waves write the dispatch after
 * their products.  Selection and softmax restate softmax_topk_route
 * (inference/src/shaders.metal:1141-1234) exactly as wave_topk does. */
template <int EPL>
DEV void k_gemv_gate_up1_body(GUArgs a, RouteArgs ra) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int rows_blk = 4 * GU_RPW, b = blockIdx.x;
    const int E = a.E, K = a.K;
    int klo;
    q4_pos(lane, klo);
    if (b >= a.routed_blocks) { /* shared expert (Q4_K): needs no routing */
        f4 xr[8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            xr[q] = *(const f4 *)(a.x + klo + 4 * q);
            xr[4 + q] = *(const f4 *)(a.x + klo + 32 + 4 * q);
        }
        h2 xl[8], xh[8];
        const float Xl = cvt_x16_f32(xr, xl), Xh = cvt_x16_f32(xr + 4, xh);
        const int r0 = (b - a.routed_blocks) * rows_blk + wv * GU_RPW;
        uint32_t sink = 0;
        /* waves 1 and 2 touch the group slots 0..3 of this block's rows (the
         * H / 8 groups of 8 rows over S / (4 GU_RPW) blocks: 4 each at
         * H = 2048, S = 512) */
        if ((wv == 1 || wv == 2) && a.pf_sh_down)
            touch_rows8(a.pf_sh_down, a.pf_sh_rb, a.H, b - a.routed_blocks, a.S / rows_blk, 2 * (wv - 1), lane, sink);
        gu_body1<GU_RPW>(a, a.sh_gate, a.sh_up, r0, xl, xh, Xl, Xh, a.act_sh, lane);
        asm volatile("s_waitcnt vmcnt(0)" : : "v"(sink));
        return;
    }
    /* x reaches the block once: wave w converts a quarter of it to fp16 into
     * LDS (each wave loading all of x made 576 blocks x 4 waves x 8 KB of L2
     * reads that held back the logits); the selecting wave also loads the
     * logits (and bias), in the same round trip */
    __shared__ __attribute__((aligned(16))) _Float16 s_x16[2048];
    const int sel = (b >> 8) & 3;
    const int xq = (wv * 64 + lane) * 8; /* this thread's 8 elements of x (H = 2048) */
    const f4 xa = *(const f4 *)(a.x + xq), xb = *(const f4 *)(a.x + xq + 4);
    const float *l = ra.logits, *bias = ra.bias ? ra.bias : ra.logits;
    float v[EPL], bv[EPL], sg = 0.0f;
    if (wv == sel) {
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            v[j] = l[min(lane * EPL + j, E - 1)];
            bv[j] = bias[min(lane * EPL + j, E - 1)];
        }
        sg = l[E];
    }
    *(h8 *)(s_x16 + xq) = h8{(_Float16)xa.x, (_Float16)xa.y, (_Float16)xa.z, (_Float16)xa.w,
                             (_Float16)xb.x, (_Float16)xb.y, (_Float16)xb.z, (_Float16)xb.w};
    const int bpe = a.M / rows_blk, u = b / bpe, r0 = (b % bpe) * rows_blk + wv * GU_RPW;
    const size_t rb = row_bytes(FQ4K, a.H);
    /* one wave of the block selects; the others wait at a barrier that it
     * passes right after round u has named the block's expert (and by which
     * every wave has stored its quarter of x).  The selecting wave is wave
     * (b / 256) % 4, so the blocks that share a CU (b, b + 256, b + 512 with
     * one block per CU and round) select on different SIMDs. */
    __shared__ int s_eu, s_rank, s_ids[64];
    Q4Raw g[GU_RPW], w2[GU_RPW];
    auto issue = [&](int e) {
        const uint8_t *gb = a.gate + (size_t)e * a.gate_stride, *ub = a.up + (size_t)e * a.up_stride;
#pragma unroll
        for (int i = 0; i < GU_RPW; i++) {
            g[i] = q4_load_nt(gb + (size_t)(r0 + i) * rb, lane);
            w2[i] = q4_load_nt(ub + (size_t)(r0 + i) * rb, lane);
        }
    };
    int rank = 0;
    if (wv == sel) {
        uint32_t key[EPL];
        int kj[EPL];
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            key[j] = lane * EPL + j < E ? route_ord(ra.bias ? v[j] + bv[j] : v[j]) : 0u;
            kj[j] = j;
        }
#pragma unroll
        for (int pass = 0; pass < EPL; pass++)
#pragma unroll
            for (int j = pass & 1; j + 1 < EPL; j += 2)
                if (key[j + 1] > key[j]) {
                    const uint32_t tk = key[j]; key[j] = key[j + 1]; key[j + 1] = tk;
                    const int tj = kj[j]; kj[j] = kj[j + 1]; kj[j + 1] = tj;
                }
        /* lane k keeps the k-th winner.  A round is a serial chain on one
         * wave, so it carries only what the next round needs: the lanes'
         * lists (the in-lane positions packed four bits each, popped by one
         * shift) and the winner's key; keys become values after the
         * rounds. */
        typedef typename PosPack<EPL>::type PK;
        PK kjp = 0;
#pragma unroll
        for (int j = 0; j < EPL; j++) kjp |= (PK)kj[j] << (4 * j);
        int myid = 0, eu = 0;
        uint32_t mykey = 0u, key0 = 0u;
        /* a rolled loop: each wave runs these rounds once */
#pragma unroll 1
        for (int k = 0; k < K; k++) {
            const uint32_t m = wave_max_u32(key[0]);
            const int wl = (int)__builtin_ctzll(__ballot(key[0] == m));
            const int id = wl * EPL + (int)((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kjp, wl) & 0xFu);
            if (lane == k) { myid = id; mykey = m; }
            if (k == 0) key0 = m;
            if (lane == wl) {
#pragma unroll
                for (int j = 0; j + 1 < EPL; j++) key[j] = key[j + 1];
                key[EPL - 1] = 0u;
                kjp >>= 4;
            }
            if (k == u) {
                eu = id;
                if (lane == 0) s_eu = id;
                lds_barrier();
                issue(eu);
            }
        }
        const float myval = ord_value(mykey), v0 = ord_value(key0);
        rank = __popcll(__ballot(lane < K && myid < eu));
        if (lane == 0) s_rank = rank;
        if (b == 0) { /* the call's selections and weights; the block's
                       * waves write the rest of the routing at the end */
            const float tw = lane < K ? expf(myval - v0) : 0.0f;
            float sum = 0.0f;
#pragma unroll 1
            for (int k = 0; k < K; k++)
                sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tw), k));
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            if (lane < K) {
                ra.idx[lane] = myid;
                ra.w[lane] = tw * inv;
                s_ids[lane] = myid;
            }
            if (lane == 0) ra.sgl[0] = sg;
        }
    } else {
        lds_barrier();
        issue(s_eu);
    }
    /* the two waves after the selecting one touch the selected expert's
     * down rows that this block's XCD will read (group slots 0..3) */
    uint32_t sink = 0;
    const int tw = (wv - sel) & 3;
    if ((tw == 1 || tw == 2) && a.pf_down)
        touch_rows8(a.pf_down + (size_t)s_eu * a.pf_down_stride, a.pf_rb, a.H, b % bpe, bpe, 2 * (tw - 1), lane, sink);
    /* this lane's 32 values of x (k = klo .. klo + 15, klo + 32 .. + 47) */
    h2 xl[8], xh[8];
    float Xl = 0.0f, Xh = 0.0f;
    {
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        const u4 q0 = *(const u4 *)(s_x16 + klo), q1 = *(const u4 *)(s_x16 + klo + 8);
        const u4 q2 = *(const u4 *)(s_x16 + klo + 32), q3 = *(const u4 *)(s_x16 + klo + 40);
        const uint32_t wl[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t wh[8] = {q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
        for (int v2 = 0; v2 < 8; v2++) {
            xl[v2] = as_h2(wl[v2]);
            xh[v2] = as_h2(wh[v2]);
        }
#pragma unroll
        for (int v2 = 0; v2 < 8; v2++) Xl = dot2(xl[v2], one, Xl);
#pragma unroll
        for (int v2 = 0; v2 < 8; v2++) Xh = dot2(xh[v2], one, Xh);
    }
    float pg[GU_RPW], pu[GU_RPW];
#pragma unroll
    for (int i = 0; i < GU_RPW; i++) {
        pg[i] = wave_sum_fast(q4_dot(g[i], lane, xl, xh, Xl, Xh));
        pu[i] = wave_sum_fast(q4_dot(w2[i], lane, xl, xh, Xl, Xh));
    }
    /* the act row: the block's selection round (act_by_slot), else the
     * expert's rank among the selected ids, which the selecting wave knows
     * once its rounds are done */
    asm volatile("s_waitcnt vmcnt(0)" : : "v"(sink));
    if (a.act_by_slot) {
        rank = u; /* block u's expert was named by round u */
    } else {
        lds_barrier();
        if (wv != sel) rank = s_rank;
    }
    _Float16 *out = a.act + (size_t)rank * a.M;
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < GU_RPW; i++) out[r0 + i] = glu_f16(pg[i], pu[i]);
    if (b == 0) {
        /* the dispatch of the call's routing for the down kernel, from the
         * selected ids the selecting wave left in LDS before its products:
         * sorted positions (pairs, pos), the active list and offsets[e] =
         * the number of selected ids below e, one entry per thread.  Here,
         * after every wave's products, it adds no time to the selecting
         * wave (done there, it made block 0 end ~0.9 us after the rest). */
        lds_barrier();
        const int tid = threadIdx.x;
        if (tid < K) {
            const int id = s_ids[tid];
            int rkk = 0;
            for (int k = 0; k < K; k++) rkk += s_ids[k] < id;
            ra.pairs[rkk] = (uint32_t)tid;
            ra.pos[tid] = (uint32_t)rkk;
            ACT_E(ra.list, rkk) = (uint32_t)id;
            ACT_OFF(ra.list, E, rkk) = (uint32_t)rkk;
        }
        if (tid == 0) {
            ACT_N(ra.list) = (uint32_t)K;
            ACT_OFF(ra.list, E, K) = (uint32_t)K;
        }
        for (int ee = tid; ee <= E; ee += 256) {
            int c = 0;
            for (int k = 0; k < K; k++) c += s_ids[k] < ee;
            ra.offsets[ee] = (uint32_t)c;
        }
    }
}

template <int EPL>
__global__ __launch_bounds__(256) void k_gemv_gate_up1(GUArgs a, RouteArgs ra) {
    /* the arguments the first loads and branches depend on, in one round of
     * scalar loads: left alone, the compiler fetched them in four dependent
     * rounds (each branch on an argument waited for its own loads) ahead of
     * the logits' load */
    asm volatile("" ::"s"(a.kt), "s"(a.routed_blocks), "s"(a.x), "s"(a.gate), "s"(a.up), "s"(a.gate_stride),
                 "s"(a.up_stride), "s"(a.M), "s"(a.E), "s"(a.K), "s"(ra.logits), "s"(ra.bias));
    KT_BEGIN(a.kt);
    k_gemv_gate_up1_body<EPL>(a, ra);
    KT_END(a.kt);
}

/* Batched gate/up, 2 <= T <= 8, H = 2048, Q4_K.  One 16-lane DPP row per
 * weight row: lane cl owns chunks 4cl..4cl+3 of the row (64 contiguous
 * quant bytes, one super-block header, sub-block pairs 2(cl&1) and
 * 2(cl&1)+1, k = 128cl .. 128cl+127), so a row's sum is one 16-lane DPP
 * reduction.  A block = 4 waves over GB_ITER tiles of 16 rows (gate and up)
 * of one slot -- an active expert, or the shared expert over all T tokens
 * (the shared slot's blocks come first in the grid: they carry the most
 * tokens) -- with a two-deep weight ring: tile i+1's bytes are in flight
 * while tile i computes.  The slot's tokens are staged once in LDS as fp16
 * (half(x), as the reference stages it) with the sums of each 16
 * consecutive rounded values (the Q4_K min term).  ROUTE: the block selects
 * and dispatches itself (route_block_lds); else it reads the routing written
 * by k_topk_dispatch_small in one round trip. */
#define GB_ROWS 16
#define GB_ITER 4
/* LDS: per token, 16 segments of 128 k (lane cl reads segment cl) padded to
 * GB_SEG halves, and per segment the 8 sums padded to GB_SUM floats, so the
 * 16 lanes of a row hit distinct banks */
#define GB_SEG 136
#define GB_SUM 12
#define GB_TOK_BYTES (16 * GB_SEG * 2 + 16 * GB_SUM * 4 + GB_ROWS * GB_ITER * 2)
struct GbTile {
    u4 hg, hu, qg[4], qu[4];
    MDEV void load(const uint8_t *pg, const uint8_t *pu, int cl) {
        hg = ld_u4(pg);
        hu = ld_u4(pu);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            qg[p] = ld_u4(pg + 16 + 64 * (cl & 1) + 16 * p);
            qu[p] = ld_u4(pu + 16 + 64 * (cl & 1) + 16 * p);
        }
    }
};
/* One tile: 4 rows per wave (one per DPP row) of gate and up, every token
 * of the slot; results (act = silu(gate) * up, fp16) go to obuf[j][row].
 * Quant dwords become biased exact fp16 images (q4_bias_h2) and meet x,
 * which sits in LDS in the matching (0,2,1,3) order.  Per sub-block pair g
 * (scales a = d sc, mins b = dmin m) and token:
 *   a_lo (S_lo - 1024 X_lo) + a_hi (S_hi - 1024 X_hi) / 16 - b_lo X_lo - b_hi X_hi
 * folded as  a_lo S_lo + (a_hi/16) S_hi - (1024 a_lo + b_lo) X_lo - (64 a_hi + b_hi) X_hi. */
DEV void gb_tile(const GbTile &tl, int it, int cl, int q, int wv, int n, const _Float16 *xs, const float *xsum,
                 _Float16 *obuf) {
    float A[2][4], B[2][4]; /* [g][gate lo, gate hi, up lo, up hi] */
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const Q4Affine fg = q4k_affine(tl.hg, 2 * (cl & 1) + g), fu = q4k_affine(tl.hu, 2 * (cl & 1) + g);
        A[g][0] = fg.a_lo; A[g][1] = fg.a_hi * 0.0625f; A[g][2] = fu.a_lo; A[g][3] = fu.a_hi * 0.0625f;
        B[g][0] = fmaf(1024.0f, fg.a_lo, fg.b_lo); B[g][1] = fmaf(64.0f, fg.a_hi, fg.b_hi);
        B[g][2] = fmaf(1024.0f, fu.a_lo, fu.b_lo); B[g][3] = fmaf(64.0f, fu.a_hi, fu.b_hi);
    }
    const int rr = it * GB_ROWS + wv * 4 + q;
#pragma unroll 1
    for (int j = 0; j < n; j++) {
        const _Float16 *xj = xs + (size_t)j * (16 * GB_SEG) + cl * GB_SEG;
        const float *sj = xsum + j * (16 * GB_SUM) + cl * GB_SUM;
        float cg = 0.0f, cu = 0.0f;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            float gl = 0.0f, gh = 0.0f, ul = 0.0f, uh = 0.0f;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                h2 xl[8], xh[8];
                load_h8<true>(xj + g * 64 + c * 16, xl);
                load_h8<true>(xj + g * 64 + c * 16 + 8, xl + 4);
                load_h8<true>(xj + g * 64 + 32 + c * 16, xh);
                load_h8<true>(xj + g * 64 + 32 + c * 16 + 8, xh + 4);
                const u4 wq = tl.qg[2 * g + c], uq = tl.qu[2 * g + c];
                uint32_t gw[4] = {wq.x, wq.y, wq.z, wq.w}, uw[4] = {uq.x, uq.y, uq.z, uq.w};
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    /* opaque per token: keeps the split inside the token loop
                     * instead of hoisting 128 registers of it */
                    asm volatile("" : "+v"(gw[d]), "+v"(uw[d]));
                    h2 l02, l13, h02, h13;
                    q4_bias_h2(gw[d], l02, l13, h02, h13);
                    gl = dot2(l02, xl[2 * d], gl);
                    gl = dot2(l13, xl[2 * d + 1], gl);
                    gh = dot2(h02, xh[2 * d], gh);
                    gh = dot2(h13, xh[2 * d + 1], gh);
                    q4_bias_h2(uw[d], l02, l13, h02, h13);
                    ul = dot2(l02, xl[2 * d], ul);
                    ul = dot2(l13, xl[2 * d + 1], ul);
                    uh = dot2(h02, xh[2 * d], uh);
                    uh = dot2(h13, xh[2 * d + 1], uh);
                }
            }
            const float Xl = sj[4 * g] + sj[4 * g + 1], Xh = sj[4 * g + 2] + sj[4 * g + 3];
            cg += (A[g][0] * gl + A[g][1] * gh) - (B[g][0] * Xl + B[g][1] * Xh);
            cu += (A[g][2] * ul + A[g][3] * uh) - (B[g][2] * Xl + B[g][3] * Xh);
        }
        const float tg = row_sum16(cg), tu = row_sum16(cu);
        if (cl == 0) obuf[j * (GB_ROWS * GB_ITER) + rr] = glu_f16(tg, tu);
    }
}

/* The slot's tiles through a two-deep weight ring (t0 holds tile 0 on entry). */
DEV void gb_run(GbTile &t0, GbTile &t1, const uint8_t *wg, const uint8_t *wu, size_t tile_step, int ntile, int cl,
                int q, int wv, int n, const _Float16 *xs, const float *xsum, _Float16 *obuf) {
#pragma unroll 1
    for (int it = 0; it < ntile; it += 2) {
        /* every load unconditional (clamped tile): a skipped load would
         * leave the wait counts unknown and a tile would wait for every load
         * in flight */
        const int n1 = it + 1 < ntile ? it + 1 : it, n2 = it + 2 < ntile ? it + 2 : ntile - 1;
        t1.load(wg + n1 * tile_step, wu + n1 * tile_step, cl);
        gb_tile(t0, it, cl, q, wv, n, xs, xsum, obuf);
        t0.load(wg + n2 * tile_step, wu + n2 * tile_step, cl);
        if (it + 1 < ntile) gb_tile(t1, it + 1, cl, q, wv, n, xs, xsum, obuf);
    }
}

template <int EPL, bool ROUTE>
DEV void k_gemv_gu_b_body(GUArgs a, RouteArgs ra) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gb_dyn[];
    __shared__ RouteLds r;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tid = threadIdx.x;
    const int cl = lane & 15, q = lane >> 4;
    const int T = a.T, K = a.K, H = 2048;
    _Float16 *xs = (_Float16 *)gb_dyn;
    float *xsum = (float *)(gb_dyn + (size_t)T * 16 * GB_SEG * 2);
    const int sh_blocks = a.S / GB_ROWS; /* one tile each: the shared slot carries all T tokens */
    const int b = blockIdx.x;
    const bool sh = b < sh_blocks;
    const int bpe = a.M / (GB_ROWS * GB_ITER);
    int n, s0 = 0, base;
    int tk[8];
    const uint8_t *wg, *wu;
    if (!sh) {
        const int br = b - sh_blocks, u = br / bpe;
        base = (br % bpe) * (GB_ROWS * GB_ITER);
        int e;
        if constexpr (ROUTE) {
            route_block_lds<EPL>(ra, r, br == 0);
            if (u >= r.nact) return;
            e = r.act_e[u];
            s0 = r.act_off[u];
            n = r.act_off[u + 1] - s0;
#pragma unroll
            for (int j = 0; j < 8; j++) tk[j] = j < n ? r.pairs[s0 + j] / K : 0;
        } else {
            const uint32_t nact = ACT_N(a.list);
            const uint32_t eu = ACT_E(a.list, u), o0 = ACT_OFF(a.list, a.E, u), o1 = ACT_OFF(a.list, a.E, u + 1);
            const uint32_t pr = lane < T * K ? a.pairs[lane] : 0u;
            if ((uint32_t)u >= nact) return;
            e = (int)eu;
            s0 = (int)o0;
            n = (int)(o1 - o0);
#pragma unroll
            for (int j = 0; j < 8; j++)
                tk[j] = j < n ? (int)((uint32_t)__builtin_amdgcn_readlane((int)pr, s0 + j) / (uint32_t)K) : 0;
        }
        wg = a.gate + (size_t)e * a.gate_stride;
        wu = a.up + (size_t)e * a.up_stride;
    } else {
        base = b * GB_ROWS;
        n = T;
#pragma unroll
        for (int j = 0; j < 8; j++) tk[j] = j;
        wg = a.sh_gate;
        wu = a.sh_up;
    }
    const size_t rb = row_bytes(FQ4K, H);
    const size_t wave_row = (size_t)(base + wv * 4 + q) * rb + (cl >> 1) * 144;
    wg += wave_row;
    wu += wave_row;
    const size_t tile_step = (size_t)GB_ROWS * rb;
    GbTile t0, t1;
    t0.load(wg, wu, cl); /* weight bytes first */
    /* stage the tokens: thread t converts x[tok][8t .. 8t+8), four tokens
     * per pass; loads are unconditional (clamped token) so they stay in
     * flight together */
    const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += 4) {
        if (j0 < n) {
            f4 xv[4][2];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float *src = a.x + (size_t)tk[j0 + jj < n ? j0 + jj : j0] * H + 8 * tid;
                xv[jj][0] = *(const f4 *)src;
                xv[jj][1] = *(const f4 *)(src + 4);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = j0 + jj;
                h2 o[4] = {h2{(_Float16)xv[jj][0].x, (_Float16)xv[jj][0].y}, h2{(_Float16)xv[jj][0].z, (_Float16)xv[jj][0].w},
                           h2{(_Float16)xv[jj][1].x, (_Float16)xv[jj][1].y}, h2{(_Float16)xv[jj][1].z, (_Float16)xv[jj][1].w}};
                float s8 = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; v++) s8 = dot2(o[v], one, s8);
                const float s16 = s8 + dppf<DPP_XOR1>(s8);
                if (j < n) { /* each 4-group stored (0,2,1,3) */
                    const h2 p0 = {o[0].x, o[1].x}, p1 = {o[0].y, o[1].y}, p2 = {o[2].x, o[3].x}, p3 = {o[2].y, o[3].y};
                    *(u4 *)(xs + (size_t)j * (16 * GB_SEG) + (tid >> 4) * GB_SEG + 8 * (tid & 15)) =
                        u4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
                    if ((tid & 1) == 0) xsum[j * (16 * GB_SUM) + (tid >> 4) * GB_SUM + ((tid & 15) >> 1)] = s16;
                }
            }
        }
    }
    __syncthreads();
    /* outputs wait in LDS (no global stores between the ring's loads) */
    _Float16 *obuf = xs + (size_t)T * 16 * GB_SEG + (size_t)T * 16 * GB_SUM * 2;
    const int ntile = sh ? 1 : GB_ITER;
    gb_run(t0, t1, wg, wu, tile_step, ntile, cl, q, wv, n, xs, xsum, obuf);
    __syncthreads();
    /* obuf[j][r] holds act for token j, block row r (GB_ITER * 16 rows) */
    _Float16 *out = sh ? a.act_sh : a.act + (size_t)s0 * a.M;
    const int ld = sh ? a.S : a.M;
    for (int i = tid; i < n * GB_ROWS * GB_ITER; i += 256) {
        if (sh && i % (GB_ROWS * GB_ITER) >= GB_ROWS) continue;
        const int j = i / (GB_ROWS * GB_ITER), rr = i % (GB_ROWS * GB_ITER);
        out[(size_t)j * ld + base + rr] = obuf[i];
    }
}

template <int EPL, bool ROUTE>
__global__ __launch_bounds__(256) void k_gemv_gu_b(GUArgs a, RouteArgs ra) {
    KT_BEGIN(a.kt);
    k_gemv_gu_b_body<EPL, ROUTE>(a, ra);
    KT_END(a.kt);
}

/* =================================================================== */
/* down.  One block = one active slot (routed expert or the shared expert) x
 * 8 output rows; each wave covers 4 rows with 16 lanes per row (a row pass
 * is 16 x 32 = 512 weights; in_dim % 512 == 0).  Results go to
 * y[sorted pair position][H] and ysh[t][H]; the combine kernel applies the
 * routing weights (kernel boundaries order the two, no cross-block fences). */
struct DownArgs {
    const uint8_t *down;
    size_t down_stride;
    int fmt;
    const uint8_t *sh_down;
    int sh_fmt, S;
    const _Float16 *act, *act_sh;
    int T, H, M, K, E;
    const uint32_t *list;
    float *y, *ysh;
    const float *pf_router; /* T = 1, H = 2048: rows E x H to touch (the next layer's router) or NULL */
};

template <int NT, int FMT>
DEV void down_slot(const uint8_t *row, int in_dim, int cl, int n, const _Float16 *const *xrow,
                   float *acc) {
    for (int c = cl; c < in_dim / 32; c += 16) {
        if (FMT == FQ4K) {
            Q4Raw r = q4_load(row, c);
            int klo;
            q4_pos(c, klo);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                if (j >= n) break;
                h2 xl[8], xh[8];
                load_h8(xrow[j] + klo, xl);
                load_h8(xrow[j] + klo + 8, xl + 4);
                load_h8(xrow[j] + klo + 32, xh);
                load_h8(xrow[j] + klo + 40, xh + 4);
                acc[j] += q4_dot(r, c, xl, xh, hsum(xl, 8), hsum(xh, 8));
            }
        } else if (FMT == FQ5K) {
            Q5Raw r = q5_load(row, c);
            int klo;
            q4_pos(c, klo);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                if (j >= n) break;
                h2 xl[8], xh[8];
                load_h8(xrow[j] + klo, xl);
                load_h8(xrow[j] + klo + 8, xl + 4);
                load_h8(xrow[j] + klo + 32, xh);
                load_h8(xrow[j] + klo + 40, xh + 4);
                acc[j] += q5_dot(r, c, xl, xh, hsum(xl, 8), hsum(xh, 8));
            }
        } else if (FMT == FQ6K) {
            Q6Raw r = q6_load(row, c);
            int k0;
            q6_pos(c, k0);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                if (j >= n) break;
                h2 x[16];
#pragma unroll
                for (int gq = 0; gq < 4; gq++) load_h8(xrow[j] + k0 + 32 * gq, x + 4 * gq);
                acc[j] += q6_dot(r, c, x);
            }
        } else {
            Q8Raw r = q8_load(row, c);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                if (j >= n) break;
                h2 x[16];
#pragma unroll
                for (int gq = 0; gq < 4; gq++) load_h8(xrow[j] + c * 32 + 8 * gq, x + 4 * gq);
                acc[j] += q8_dot(r, x);
            }
        }
    }
}

template <int NT>
__global__ __launch_bounds__(128) void k_gemv_down(DownArgs a) {
    const int T = a.T, H = a.H;
    const int ntile = H / 8;
    const int u = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    const int n_act = (int)ACT_N(a.list);
    const int has_sh = a.sh_down != nullptr;
    if (u >= n_act + has_sh) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int rl = wv * 4 + (lane >> 4), cl = lane & 15;
    const int r = tile * 8 + rl;
    const bool sh = u == n_act;
    const _Float16 *xrow[NT];
    float acc[NT];
    int n, s0 = 0, fmt, in_dim;
    const uint8_t *row;
    if (!sh) {
        const int e = (int)ACT_E(a.list, u);
        s0 = (int)ACT_OFF(a.list, a.E, u);
        n = (int)ACT_OFF(a.list, a.E, u + 1) - s0;
        fmt = a.fmt;
        in_dim = a.M;
        row = a.down + (size_t)e * a.down_stride + (size_t)r * row_bytes(fmt, in_dim);
#pragma unroll
        for (int j = 0; j < NT; j++) xrow[j] = a.act + (size_t)(s0 + (j < n ? j : 0)) * a.M;
    } else {
        n = T;
        fmt = a.sh_fmt;
        in_dim = a.S;
        row = a.sh_down + (size_t)r * row_bytes(fmt, in_dim);
#pragma unroll
        for (int j = 0; j < NT; j++) xrow[j] = a.act_sh + (size_t)(j < n ? j : 0) * a.S;
    }
#pragma unroll
    for (int j = 0; j < NT; j++) acc[j] = 0.0f;
    if (fmt == FQ4K) down_slot<NT, FQ4K>(row, in_dim, cl, n, xrow, acc);
    else if (fmt == FQ5K) down_slot<NT, FQ5K>(row, in_dim, cl, n, xrow, acc);
    else if (fmt == FQ6K) down_slot<NT, FQ6K>(row, in_dim, cl, n, xrow, acc);
    else down_slot<NT, FQ8>(row, in_dim, cl, n, xrow, acc);
#pragma unroll
    for (int j = 0; j < NT; j++) {
        if (j >= n) break;
        float v = row_sum16(acc[j]);
        if (cl == 0) {
            if (sh) a.ysh[(size_t)j * H + r] = v;
            else a.y[(size_t)(s0 + j) * H + r] = v;
        }
    }
}

/* One-token down + combine.  For T = 1 every routed expert holds one pair,
 * so a block of 8 output rows can take all K routed slots and the shared
 * slot itself and write h_out directly (k_combine's order: h_in + sum_k
 * w_k y_k, then + sigmoid(s) y_shared), with no y round trip and one launch
 * fewer.  Raw weight chunks of every slot are loaded before any is used, so
 * all of a lane's loads are in flight together.  in_dim = 512: one chunk
 * per lane (16 lanes per row). */
#define DC_K 8
template <int FMT>
struct DnRaw;
template <>
struct DnRaw<FQ4K> {
    Q4Raw r;
    MDEV void load(const uint8_t *row, int c) { r = q4_load(row, c); }
    MDEV float dot(int c, const _Float16 *x) const {
        int klo;
        q4_pos(c, klo);
        h2 xl[8], xh[8];
        load_h8(x + klo, xl);
        load_h8(x + klo + 8, xl + 4);
        load_h8(x + klo + 32, xh);
        load_h8(x + klo + 40, xh + 4);
        return q4_dot(r, c, xl, xh, hsum(xl, 8), hsum(xh, 8));
    }
};
template <>
struct DnRaw<FQ5K> {
    Q5Raw r;
    MDEV void load(const uint8_t *row, int c) { r = q5_load(row, c); }
};
template <>
struct DnRaw<FQ6K> {
    Q6Raw r;
    MDEV void load(const uint8_t *row, int c) { r = q6_load(row, c); }
    MDEV float dot(int c, const _Float16 *x) const {
        int k0;
        q6_pos(c, k0);
        h2 xv[16];
#pragma unroll
        for (int gq = 0; gq < 4; gq++) load_h8(x + k0 + 32 * gq, xv + 4 * gq);
        return q6_dot(r, c, xv);
    }
};
template <>
struct DnRaw<FQ8> {
    Q8Raw r;
    MDEV void load(const uint8_t *row, int c) { r = q8_load(row, c); }
    MDEV float dot(int c, const _Float16 *x) const {
        h2 xv[16];
#pragma unroll
        for (int gq = 0; gq < 4; gq++) load_h8(x + c * 32 + 8 * gq, xv + 4 * gq);
        return q8_dot(r, xv);
    }
};

/* Activation values of chunk c of one token, loaded once and used for
 * every weight row of the lane (the DnRaw<FMT> chunk layouts).  offs gives
 * the four 8-value runs a lane reads, set fills the values from those runs
 * (so a kernel can issue the loads of many chunks before using any). */
template <int FMT>
struct DnX;
template <>
struct DnX<FQ4K> {
    h2 xl[8], xh[8];
    float Xl, Xh;
    static MDEV void offs(int c, int (&o)[4]) {
        int klo;
        q4_pos(c, klo);
        o[0] = klo; o[1] = klo + 8; o[2] = klo + 32; o[3] = klo + 40;
    }
    MDEV void set(const u4 (&q)[4]) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            xl[4 * j] = as_h2(q[j].x); xl[4 * j + 1] = as_h2(q[j].y); xl[4 * j + 2] = as_h2(q[j].z); xl[4 * j + 3] = as_h2(q[j].w);
            xh[4 * j] = as_h2(q[2 + j].x); xh[4 * j + 1] = as_h2(q[2 + j].y);
            xh[4 * j + 2] = as_h2(q[2 + j].z); xh[4 * j + 3] = as_h2(q[2 + j].w);
        }
        Xl = hsum(xl, 8);
        Xh = hsum(xh, 8);
    }
    MDEV void load(int c, const _Float16 *x) {
        int o[4];
        offs(c, o);
        load_h8(x + o[0], xl);
        load_h8(x + o[1], xl + 4);
        load_h8(x + o[2], xh);
        load_h8(x + o[3], xh + 4);
        Xl = hsum(xl, 8);
        Xh = hsum(xh, 8);
    }
    MDEV float dot(const DnRaw<FQ4K> &r, int c) const { return q4_dot(r.r, c, xl, xh, Xl, Xh); }
};
/* Q5_K chunks cover the positions of Q4_K chunks: the same activation runs
 * and sums, a five-bit dot */
template <>
struct DnX<FQ5K> : DnX<FQ4K> {
    MDEV float dot(const DnRaw<FQ5K> &r, int c) const { return q5_dot(r.r, c, xl, xh, Xl, Xh); }
};
template <>
struct DnX<FQ6K> {
    h2 x[16];
    static MDEV void offs(int c, int (&o)[4]) {
        int k0;
        q6_pos(c, k0);
#pragma unroll
        for (int gq = 0; gq < 4; gq++) o[gq] = k0 + 32 * gq;
    }
    MDEV void set(const u4 (&q)[4]) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
            x[4 * gq] = as_h2(q[gq].x); x[4 * gq + 1] = as_h2(q[gq].y);
            x[4 * gq + 2] = as_h2(q[gq].z); x[4 * gq + 3] = as_h2(q[gq].w);
        }
    }
    MDEV void load(int c, const _Float16 *xr) {
        int o[4];
        offs(c, o);
#pragma unroll
        for (int gq = 0; gq < 4; gq++) load_h8(xr + o[gq], x + 4 * gq);
    }
    MDEV float dot(const DnRaw<FQ6K> &r, int c) const { return q6_dot(r.r, c, x); }
};
template <>
struct DnX<FQ8> {
    h2 x[16];
    static MDEV void offs(int c, int (&o)[4]) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) o[gq] = c * 32 + 8 * gq;
    }
    MDEV void set(const u4 (&q)[4]) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
            x[4 * gq] = as_h2(q[gq].x); x[4 * gq + 1] = as_h2(q[gq].y);
            x[4 * gq + 2] = as_h2(q[gq].z); x[4 * gq + 3] = as_h2(q[gq].w);
        }
    }
    MDEV void load(int c, const _Float16 *xr) {
        int o[4];
        offs(c, o);
#pragma unroll
        for (int gq = 0; gq < 4; gq++) load_h8(xr + o[gq], x + 4 * gq);
    }
    MDEV float dot(const DnRaw<FQ8> &r, int) const { return q8_dot(r.r, x); }
};

/* SLOT: act row k belongs to slot k (the gate/up wrote them in selection
 * order), so the activation loads go out with the routing loads instead of
 * after them.
 *
 * A block holds 8 output rows as two halves of 4 rows (a 16-lane group per
 * row), and each half's nine dots (8 routed slots, then the shared expert)
 * are spread over DC_SG waves: wave g of a half takes slots g, g + DC_SG,
 * g + 2 DC_SG (slot 8 is the shared expert's).  One wave per half running
 * all nine dots one after the other was bound by that wave's instruction
 * chain (~1200 instructions after its loads arrived).  The dots are
 * unchanged, and the sums go through LDS to the half's first wave, which
 * combines them in k_combine's order: h_in + sum_k w_k y_k (k ascending),
 * then + sigmoid(s) y_shared. */
#define DC_SG 3
template <int EFMT, int SFMT, bool SLOT>
__global__ __launch_bounds__(128 * DC_SG) void k_gemv_down_combine1(DownArgs a, RouteArgs ra, const float *h_in,
                                                                   float *h_out, float *res) {
    constexpr int NS = (DC_K + 1 + DC_SG - 1) / DC_SG; /* slots per wave */
    static_assert(NS * DC_SG == DC_K + 1, "nine slots over the waves of a half");
    __shared__ float ys[2][DC_K + 1][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int half = wv / DC_SG, g = wv % DC_SG;
    const int cl = lane & 15, rq = lane >> 4, r = blockIdx.x * 8 + half * 4 + rq;
    const int K = a.K;
    const size_t rb = row_bytes(EFMT, a.M);
    const bool has_sh = a.sh_down != nullptr;
    const bool sh_here = g == DC_SG - 1; /* this wave's last slot is the shared expert's */
    /* every load up front and unconditional, in dependence order: the slots'
     * experts, positions and weights; then the weight chunks; then the
     * activation chunks, the residual and the gate (a load under a branch,
     * or one made inside a slot's dot, is waited for alone) */
    /* the 8 slots' experts, positions and weights as three 32-byte reads
     * (the context sizes these buffers for 16 per token); a slot k >= K
     * takes slot 0's expert and position (a valid address) and is not summed */
    static_assert(DC_K == 8 && OROME_MAXK >= 8, "slot reads");
    typedef int i4v __attribute__((ext_vector_type(4)));
    const i4v e0 = *(const i4v *)ra.idx, e1 = *(const i4v *)(ra.idx + 4);
    const u4 p0 = *(const u4 *)ra.pos, p1 = *(const u4 *)(ra.pos + 4);
    int o[4], osh[4];
    DnX<EFMT>::offs(cl, o);
    DnX<SFMT>::offs(cl, osh);
    /* this wave's routed slots: k = g + DC_SG j (j < NS, and the shared
     * expert's in place of k = 8); a slot past 8 reads slot 0's rows */
    int kk[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) kk[j] = min(g + DC_SG * j, DC_K - 1);
    u4 xq[NS][4], sq[4];
    const _Float16 *xs = has_sh ? a.act_sh : a.act;
    if constexpr (SLOT) {
#pragma unroll
        for (int j = 0; j < NS; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) xq[j][q] = ld_u4((const uint8_t *)(a.act + (size_t)(kk[j] < K ? kk[j] : 0) * a.M + o[q]));
#pragma unroll
        for (int q = 0; q < 4; q++) sq[q] = ld_u4((const uint8_t *)(xs + osh[q]));
    }
    const int ev[DC_K] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
    const int pv[DC_K] = {(int)p0.x, (int)p0.y, (int)p0.z, (int)p0.w, (int)p1.x, (int)p1.y, (int)p1.z, (int)p1.w};
    int e[NS], ps[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) {
        /* kk[j] is wave-uniform: a select over the eight slots */
        int ej = ev[0], pj = pv[0];
#pragma unroll
        for (int k = 1; k < DC_K; k++)
            if (kk[j] == k && k < K) { ej = ev[k]; pj = pv[k]; }
        e[j] = ej;
        ps[j] = pj;
    }
    DnRaw<EFMT> raw[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) raw[j].load(a.down + (size_t)e[j] * a.down_stride + (size_t)r * rb, cl);
    DnRaw<SFMT> rsh;
    rsh.load(has_sh ? a.sh_down + (size_t)r * row_bytes(SFMT, a.S) : a.down + (size_t)r * rb, cl);
    if constexpr (!SLOT) {
#pragma unroll
        for (int j = 0; j < NS; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) xq[j][q] = ld_u4((const uint8_t *)(a.act + (size_t)ps[j] * a.M + o[q]));
#pragma unroll
        for (int q = 0; q < 4; q++) sq[q] = ld_u4((const uint8_t *)(xs + osh[q]));
    }
    /* what the combine needs, loaded with the rest */
    const f4 w0 = *(const f4 *)ra.w, w1 = *(const f4 *)(ra.w + 4);
    const float hb = (h_in ? h_in : h_out)[r];
    const float sgv = ra.sgl[0];
    /* the next layer's router (one wave per 4-row block of 2048 fp32, the
     * T = 1 router's blocks): block j touches row 4 (x + 8 (s / 4)) + s % 4,
     * x = j % 8, s = j / 8, so the rows reach the XCD whose router block
     * reads them; one 4-byte load per 128-byte line */
    uint32_t sink = 0;
    if (a.pf_router && wv == 1) {
        const int x8 = blockIdx.x & 7, sl = blockIdx.x >> 3, row = 4 * (x8 + 8 * (sl >> 2)) + (sl & 3);
        if (row < a.E) {
            const float *p = a.pf_router + (size_t)row * 2048 + lane * 32;
            asm volatile("global_load_dword %0, %1, off" : "=v"(sink) : "v"(p) : "memory");
        }
    }
#pragma unroll
    for (int j = 0; j < NS; j++) {
        if (sh_here && j == NS - 1) break; /* the shared expert's slot, below */
        DnX<EFMT> xv;
        xv.set(xq[j]);
        const float y = row_sum16(xv.dot(raw[j], cl));
        if (cl == 0) ys[half][g + DC_SG * j][rq] = y;
    }
    if (sh_here) {
        float ysh = 0.0f;
        if (has_sh) {
            DnX<SFMT> xv;
            xv.set(sq);
            ysh = row_sum16(xv.dot(rsh, cl));
        }
        if (cl == 0) ys[half][DC_K][rq] = ysh;
    }
    __syncthreads();
    if (g == 0 && cl == 0) {
        const float wk[DC_K] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float moe = 0.0f;
#pragma unroll
        for (int k = 0; k < DC_K; k++)
            if (k < K) moe += wk[k] * ys[half][k][rq];
        float ov = (h_in ? hb : 0.0f) + moe;
        if (has_sh) ov = ov + sigmoid_f(sgv) * ys[half][DC_K][rq];
        h_out[r] = ov;
        if (res) res[r] = ov;
    }
    asm volatile("s_waitcnt vmcnt(0)" : : "v"(sink));
}

/* Batched down (T <= 8, in_dim = 512): a block = 4 waves = 64 output rows of
 * one slot (an active routed expert, or the shared expert over all T
 * tokens, last); a 16-lane DPP row takes DB_R consecutive weight rows, lane
 * cl chunk cl of each (all DB_R chunks loaded at once), and walks the slot's
 * tokens with each token's activation chunk loaded once for all its rows.
 * Same sums as k_gemv_down; results go to y[sorted position][H] and
 * ysh[t][H]. */
#ifndef DB_R
#define DB_R 2
#endif
#define DB_ROWS (4 * 4 * DB_R)
template <int FMT>
DEV void db_run(const uint8_t *w, size_t rb, int r0, int cl, int n, const _Float16 *x0, int x_ld, float *out,
                int H) {
    DnRaw<FMT> raw[DB_R];
#pragma unroll
    for (int r = 0; r < DB_R; r++) raw[r].load(w + (size_t)(r0 + r) * rb, cl);
#pragma unroll 1
    for (int j = 0; j < n; j++) {
        DnX<FMT> xv;
        xv.load(cl, x0 + (size_t)j * x_ld);
#pragma unroll
        for (int r = 0; r < DB_R; r++) {
            const float v = row_sum16(xv.dot(raw[r], cl));
            if (cl == 0) out[(size_t)j * H + r0 + r] = v;
        }
    }
}
template <int EFMT, int SFMT>
__global__ __launch_bounds__(256) void k_gemv_down_b(DownArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, cl = lane & 15, q = lane >> 4;
    const int bps = a.H / DB_ROWS, u = blockIdx.x / bps;
    const int r0 = (blockIdx.x % bps) * DB_ROWS + wv * (4 * DB_R) + q * DB_R;
    const uint32_t nact = ACT_N(a.list), eu = ACT_E(a.list, u), o0 = ACT_OFF(a.list, a.E, u),
                   o1 = ACT_OFF(a.list, a.E, u + 1);
    const bool has_sh = a.sh_down != nullptr;
    if ((uint32_t)u > nact || ((uint32_t)u == nact && !has_sh)) return;
    if ((uint32_t)u == nact)
        db_run<SFMT>(a.sh_down, row_bytes(SFMT, a.S), r0, cl, a.T, a.act_sh, a.S, a.ysh, a.H);
    else
        db_run<EFMT>(a.down + (size_t)eu * a.down_stride, row_bytes(EFMT, a.M), r0, cl, (int)(o1 - o0),
                     a.act + (size_t)o0 * a.M, a.M, a.y + (size_t)o0 * a.H, a.H);
}

/* ------------------------------------------------------------ launch */

static int epl_of(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : E <= 1024 ? 16 : 0; }

bool gemv_gate_up1_path(int route_in_block, int T, int H, const SharedSide &sh) {
    return route_in_block && T == 1 && H == 2048 && (!sh.gate || sh.gate_fmt == FQ4K);
}

int launch_gemv_gate_up(const ExpertSide &ex, const SharedSide &sh, const RouteArgs &ra, int route_in_block,
                        const float *x, int T, int H, int M, int K, int E, _Float16 *act, _Float16 *act_sh,
                        hipStream_t s, unsigned long long *kt, int kt_cap, int act_by_slot) {
    const int rows_blk = 4 * GU_RPW;
    if (T < 1 || T > 16 || T * K > 256 || H % 256 || ex.gate_fmt != FQ4K || !epl_of(E)) return -2;
    if (M % rows_blk || (sh.gate && sh.S % rows_blk)) return -2;
    if (sh.gate && sh.gate_fmt != FQ4K && sh.gate_fmt != FQ8) return -2;
    GUArgs a;
    a.gate = ex.gate; a.up = ex.up; a.gate_stride = ex.gate_stride; a.up_stride = ex.up_stride;
    a.sh_gate = sh.gate; a.sh_up = sh.up; a.sh_fmt = sh.gate_fmt; a.S = sh.gate ? sh.S : 0;
    a.x = x; a.T = T; a.H = H; a.M = M; a.K = K; a.E = E; a.list = ra.list; a.pairs = ra.pairs;
    a.act = act; a.act_sh = act_sh;
    a.pf_down = a.pf_sh_down = nullptr; a.pf_down_stride = 0; a.pf_rb = a.pf_sh_rb = 0;
    a.act_by_slot = 0;
    if (T == 1) {
        a.pf_down = ex.down; a.pf_down_stride = ex.down_stride; a.pf_rb = (int)row_bytes(ex.down_fmt, M);
        if (sh.gate) { a.pf_sh_down = sh.down; a.pf_sh_rb = (int)row_bytes(sh.down_fmt, sh.S); }
    }
    const int umax = T * K < E ? T * K : E;
    a.routed_blocks = umax * (M / rows_blk);
    const int blocks = a.routed_blocks + (sh.gate ? sh.S / rows_blk : 0);
    a.kt = kt && blocks <= kt_cap ? kt : nullptr;
    const int gb_rows = GB_ROWS * GB_ITER;
    if (T >= 2 && T <= 8 && H == 2048 && M % gb_rows == 0 && (!sh.gate || (sh.gate_fmt == FQ4K && sh.S % gb_rows == 0))) {
        a.routed_blocks = umax * (M / gb_rows);
        const int gblocks = a.routed_blocks + (sh.gate ? sh.S / GB_ROWS : 0);
        const size_t lds = (size_t)T * GB_TOK_BYTES;
        a.kt = kt && gblocks <= kt_cap ? kt : nullptr;
#define GB_LAUNCH(EPLV)                                                                                       \
    do {                                                                                                      \
        if (route_in_block)                                                                                   \
            KLAUNCH((k_gemv_gu_b<EPLV, true>), dim3(gblocks), dim3(256), lds, s, a, ra);           \
        else                                                                                                  \
            KLAUNCH((k_gemv_gu_b<EPLV, false>), dim3(gblocks), dim3(256), lds, s, a, ra);          \
    } while (0)
        switch (epl_of(E)) {
            case 1: GB_LAUNCH(1); break;
            case 2: GB_LAUNCH(2); break;
            case 4: GB_LAUNCH(4); break;
            case 8: GB_LAUNCH(8); break;
            default: GB_LAUNCH(16); break;
        }
#undef GB_LAUNCH
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    if (act_by_slot && !gemv_gate_up1_path(route_in_block, T, H, sh)) return -1;
    if (gemv_gate_up1_path(route_in_block, T, H, sh)) {
        a.act_by_slot = act_by_slot;
#define GU1_LAUNCH(EPLV) KLAUNCH((k_gemv_gate_up1<EPLV>), dim3(blocks), dim3(256), 0, s, a, ra)
        switch (epl_of(E)) {
            case 1: GU1_LAUNCH(1); break;
            case 2: GU1_LAUNCH(2); break;
            case 4: GU1_LAUNCH(4); break;
            case 8: GU1_LAUNCH(8); break;
            default: GU1_LAUNCH(16); break;
        }
#undef GU1_LAUNCH
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
#define GU_LAUNCH(EPLV)                                                                          \
    do {                                                                                          \
        if (route_in_block)                                                                       \
            KLAUNCH((k_gemv_gate_up<EPLV, true>), dim3(blocks), dim3(256), 0, s, a, ra);  \
        else                                                                                      \
            KLAUNCH((k_gemv_gate_up<EPLV, false>), dim3(blocks), dim3(256), 0, s, a, ra); \
    } while (0)
    switch (epl_of(E)) {
        case 1: GU_LAUNCH(1); break;
        case 2: GU_LAUNCH(2); break;
        case 4: GU_LAUNCH(4); break;
        case 8: GU_LAUNCH(8); break;
        default: GU_LAUNCH(16); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}


/* MACRO(EF, SF) for the runtime pair (routed down format in {Q4_K, Q5_K,
 * Q6_K}, shared down format in {Q4_K, Q5_K, Q6_K, Q8_0}) */
#define DOWN_SF_SWITCH(EF, SF, MACRO)       \
    do {                                    \
        if ((SF) == FQ4K) MACRO(EF, FQ4K);  \
        else if ((SF) == FQ5K) MACRO(EF, FQ5K); \
        else if ((SF) == FQ6K) MACRO(EF, FQ6K); \
        else MACRO(EF, FQ8);                \
    } while (0)
#define DOWN_FMT_SWITCH(EFR, SFR, MACRO)                    \
    do {                                                    \
        if ((EFR) == FQ4K) DOWN_SF_SWITCH(FQ4K, SFR, MACRO); \
        else if ((EFR) == FQ5K) DOWN_SF_SWITCH(FQ5K, SFR, MACRO); \
        else DOWN_SF_SWITCH(FQ6K, SFR, MACRO);              \
    } while (0)

static int nt_for(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 0; }

int launch_gemv_down(const ExpertSide &ex, const SharedSide &sh, const _Float16 *act,
                     const _Float16 *act_sh, int T, int H, int M, int K, int E, const uint32_t *list,
                     float *y, float *ysh, hipStream_t s) {
    const int NT = nt_for(T);
    if (!NT || H % 8 || M % 512 || (sh.gate && sh.S % 512)) return -2;
    if (ex.down_fmt != FQ4K && ex.down_fmt != FQ5K && ex.down_fmt != FQ6K) return -2;
    if (sh.gate && sh.down_fmt != FQ4K && sh.down_fmt != FQ5K && sh.down_fmt != FQ6K && sh.down_fmt != FQ8) return -2;
    DownArgs a = {};
    a.down = ex.down; a.down_stride = ex.down_stride; a.fmt = ex.down_fmt;
    a.sh_down = sh.gate ? sh.down : nullptr; a.sh_fmt = sh.down_fmt; a.S = sh.S;
    a.act = act; a.act_sh = act_sh; a.T = T; a.H = H; a.M = M; a.K = K; a.E = E;
    a.list = list; a.y = y; a.ysh = ysh;
    const int umax = T * K < E ? T * K : E;
    if (M == 512 && (!sh.gate || sh.S == 512) && H % DB_ROWS == 0) {
        const dim3 g((unsigned)((umax + (sh.gate ? 1 : 0)) * (H / DB_ROWS)));
        const int sf = sh.gate ? sh.down_fmt : FQ4K;
#define DB_LAUNCH(EF, SF) KLAUNCH((k_gemv_down_b<EF, SF>), g, dim3(256), 0, s, a)
        DOWN_FMT_SWITCH(ex.down_fmt, sf, DB_LAUNCH);
#undef DB_LAUNCH
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    dim3 grid((umax + (sh.gate ? 1 : 0)) * (H / 8));
    switch (NT) {
        case 1: KLAUNCH(k_gemv_down<1>, grid, dim3(128), 0, s, a); break;
        case 2: KLAUNCH(k_gemv_down<2>, grid, dim3(128), 0, s, a); break;
        case 4: KLAUNCH(k_gemv_down<4>, grid, dim3(128), 0, s, a); break;
        default: KLAUNCH(k_gemv_down<8>, grid, dim3(128), 0, s, a); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_gemv_down_combine1(const ExpertSide &ex, const SharedSide &sh, const RouteArgs &ra,
                              const _Float16 *act, const _Float16 *act_sh, int H, int M, int K,
                              const float *h_in, float *h_out, float *res, hipStream_t s,
                              const float *next_router, int act_by_slot) {
    if (K < 1 || K > DC_K || H % 8 || M != 512 || (sh.gate && sh.S != 512)) return -2;
    if (ex.down_fmt != FQ4K && ex.down_fmt != FQ5K && ex.down_fmt != FQ6K) return -2;
    const int sf = sh.gate ? sh.down_fmt : FQ4K;
    if (sf != FQ4K && sf != FQ5K && sf != FQ6K && sf != FQ8) return -2;
    DownArgs a = {};
    a.down = ex.down; a.down_stride = ex.down_stride; a.fmt = ex.down_fmt;
    a.sh_down = sh.gate ? sh.down : nullptr; a.sh_fmt = sf; a.S = sh.gate ? sh.S : 0;
    a.act = act; a.act_sh = act_sh; a.T = 1; a.H = H; a.M = M; a.K = K; a.E = ra.E;
    a.pf_router = H == 2048 ? next_router : nullptr;
#define DC_LAUNCH(EF, SF)                                                                                                     \
    do {                                                                                                                      \
        if (act_by_slot) KLAUNCH((k_gemv_down_combine1<EF, SF, true>), dim3(H / 8), dim3(128 * DC_SG), 0, s, a, ra, h_in, h_out, res); \
        else KLAUNCH((k_gemv_down_combine1<EF, SF, false>), dim3(H / 8), dim3(128 * DC_SG), 0, s, a, ra, h_in, h_out, res);           \
    } while (0)
    DOWN_FMT_SWITCH(ex.down_fmt, sf, DC_LAUNCH);
#undef DC_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
