/*
 * moe_gemm.hip -- prefill-path grouped expert GEMMs on the matrix cores.
 *
 * Work list: the dispatch kernel emits two tile lists (expert, first row,
 * rows <= GEMM_TILE_SMALL or GEMM_TILE_BIG), each launched with its tile size,
 * over the expert-sorted pair list; the shared expert is expert E over the
 * token order.  One block computes one tile x NB output rows:
 *   gate/up  D[row][token] = W_{gate,up}[e][row] . x16[token]      (K = H)
 *   down     y[pos][row]   = W_down[e][row]    . act[pos]         (K = M)
 * with v_mfma_f32_16x16x32_f16 (A = 16 weight rows x 32 k, B = 32 k x 16
 * tokens, fp32 accumulate).  Each of the 8 waves owns RPW blocks of 16
 * weight rows (of gate and of up for the first GEMM, one block; of down,
 * four) for all TB = ceil(rows/16) token blocks of the tile, so one
 * dequantised A fragment feeds TB matrix instructions.
 *
 * Weights are dequantised straight into A fragments with packed fp16
 * arithmetic on exactly factored terms (q arrives as the exact fp16 1024+q by
 * OR-ing the quant bits under the 0x64 exponent byte):
 *   Q4_K  t = fma(1024+q, sc, -1024 sc) = q sc   (exact, <= 945)
 *         w = fma(t, d, -fp16(dmin m))          one rounding, plus the
 *         rounding of dmin*m (~7% of |w|): within one fp16 ulp of exact
 *   Q6_K  w = (q sc) d   exact product when |q sc| <= 2048, else two roundings
 *   Q8_0  w = q d        one rounding
 * The B operand (activations, fp16 as the reference stages half(x) and
 * half(act)) sits in LDS in fragment order: the 8 k values lane (i, kg) needs
 * at step s of a 128-wide k stage are 16 contiguous bytes at (4 s + kg) * 8,
 * so a B fragment is one ds_read_b128; the staging store applies the
 * per-format k permutation.  Stages are double-buffered: the next stage's
 * activations and weight bytes are fetched to registers before the current
 * stage's matrix work.
 */
#include <cstdlib>
#include "dev_common.h"
#include "kernels.h"

/* FQ4KT, FQ5KT, FQ6KT, FQ8T: Q4_K / Q5_K / Q6_K / Q8_0 repacked tile-major
 * (launch_pack_q4k, _q5k, _q6k, _q8), same values */
enum { FQ4K = 0, FQ5K = 1, FQ6K = 2, FQ8 = 3, FQ4KT = GEMM_FMT_Q4K_TILED, FQ6KT = GEMM_FMT_Q6K_TILED, FQ8T = GEMM_FMT_Q8_TILED,
       FQ5KT = GEMM_FMT_Q5K_TILED };

typedef float f4v __attribute__((ext_vector_type(4)));

/* Block shape per tile size.  Small tiles (<= 32 tokens: the HBM-bound
 * regime) run 4-wave blocks with a 2-deep weight ring, so four waves share
 * a SIMD; big tiles run 8-wave blocks with a 4-deep ring (their LDS tile
 * allows one block per CU). */
#ifndef GEMM_BIG_W
#define GEMM_BIG_W 8
#endif
#ifndef GEMM_BIG_DEPTH
#define GEMM_BIG_DEPTH 4
#endif
template <int TBM>
struct Shape {
    static constexpr int W = TBM <= 2 ? 4 : GEMM_BIG_W;         /* waves per block */
    static constexpr int DEPTH = TBM <= 2 ? 2 : GEMM_BIG_DEPTH; /* weight stages in flight per wave */
    /* activation chunk: TBM*16 rows of 32 16-byte vectors, NV per thread;
     * when the last pass runs past the tile its rows land in one spare LDS
     * row (XR = rows per chunk buffer) */
    static constexpr int NV = (TBM * 16 * 32 + W * 64 - 1) / (W * 64);
    static constexpr int XR = NV * W * 2 > TBM * 16 ? TBM * 16 + 1 : TBM * 16;
};
#define KC 128                          /* k per stage (one A fragment set) */
#define KCH 256                         /* k per LDS activation chunk */
#define BLD (KCH + 16)                  /* chunk row pitch (halves): 544 bytes, B-fragment reads conflict-free */

DEV size_t gemm_row_bytes(int fmt, int n) {
    return fmt == FQ4K || fmt == FQ4KT ? (size_t)(n / 256) * 144
           : fmt == FQ5K || fmt == FQ5KT ? (size_t)(n / 256) * 176
           : fmt == FQ6K || fmt == FQ6KT ? (size_t)(n / 256) * 210
                                         : (size_t)(n / 32) * 34;
}
/* offset of lane row i of the 16-row block starting at row0: a row of its
 * own, or (tile-major Q4_K) the block base plus the lane's 16-byte column */
template <int FMT>
DEV size_t lane_row(int row0, int i, size_t rbytes) {
    return FMT == FQ4KT || FMT == FQ5KT || FMT == FQ6KT ? (size_t)row0 * rbytes + (size_t)i * 16
           : FMT == FQ8T                 ? (size_t)row0 * rbytes
                                         : (size_t)(row0 + i) * rbytes;
}
/* weight loads: streaming (`nt`) in the big-tile kernels and the 16-row
 * tiles of small batches, where each weight is read by one unit, and cached
 * in the 32-row tiles, where the tiles of a popular expert (and of the
 * shared expert) read the same weights again */
template <bool NT>
DEV u4 ld_w(const uint8_t *p) { return NT ? ld_u4_nt(p) : ld_u4(p); }
DEV uint32_t u4_at(u4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
DEV h2 splat(_Float16 v) { return h2{v, v}; }
DEV h2 hfma(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }
DEV h2 or_bias(uint32_t v) { return as_h2(v | 0x64006400u); }
DEV h8 cat4(h2 a, h2 b, h2 c, h2 d) { return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y}; }
/* exact fp16 pairs (q0, q2) and (q1, q3) of four 6-bit (minus 32) or int8
 * quants: the (0,2,1,3) order every activation row is stored in */
DEV void q6_h2_0213(uint32_t ql, uint32_t qh, int shift, int qshift, h2 &p02, h2 &p13) {
    const uint32_t v = ((ql >> shift) & 0x0F0F0F0Fu) | (((qh >> qshift) & 0x03030303u) << 4);
    const h2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    p02 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04020400u)) - bias;
    p13 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04030401u)) - bias;
}
DEV void q8_h2_0213(uint32_t w, h2 &p02, h2 &p13) {
    const uint32_t v = w ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    p02 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04020400u)) - bias;
    p13 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04030401u)) - bias;
}

/* ------------------------------------------------- k order in LDS */
/* Position (halves) inside a stage row of the 4 k values [4c, 4c+4), i.e. of
 * fragment (s, kg) elements j0..j0+3.  Mirrors the lane -> k mapping of each
 * Span below.  Activation rows (x16, act, act_sh) are kept in global memory
 * with every 4-group stored (0,2,1,3) -- the order the Q4_K nibble split
 * yields; the Q6_K and Q8_0 spans produce the same order -- so a 4-group is
 * copied into LDS unchanged. */
template <int FMT>
DEV int frag_pos(int c) {
    if (FMT == FQ4K || FMT == FQ4KT || FMT == FQ5K || FMT == FQ5KT) { /* lane kg, step s: k = 64(kg>>1) + 16(kg&1) + 4s (+32 high nibbles) */
        const int g = c >> 4, r = c & 15, hi = r >> 3, rr = r & 7;
        return (((rr & 3) * 4 + 2 * g + (rr >> 2)) * 8) + 4 * hi;
    } else if (FMT == FQ6K || FMT == FQ6KT) { /* k = 32(kg&1) + 16(kg>>1) + 4s (+64 high nibbles) */
        const int hi = c >> 4, r = c & 15, odd = r >> 3, q = r & 7;
        return (((q & 3) * 4 + 2 * (q >> 2) + odd) * 8) + 4 * hi;
    } else { /* k = 32s + 8kg .. +7 */
        return ((c >> 3) * 4 + ((c & 7) >> 1)) * 8 + 4 * (c & 1);
    }
}

/* ------------------------------------------------------------ spans */
/* One weight row's share of a 128-wide k stage j for lane group kg (0..3):
 * raw bytes (load), per-stage constants (prepare), A fragment at step s. */
template <int FMT>
struct Span;

template <>
struct Span<FQ4K> {
    u4 hdr, q;
    MDEV void init(int) {}
    template <bool NT = false>
    MDEV void load(const uint8_t *row, int j, int kg) {
        const uint8_t *p = row + (size_t)(j >> 1) * 144;
        hdr = ld_w<NT>(p);
        q = ld_w<NT>(p + 16 + 16 * (kg + 4 * (j & 1)));
    }
    h2 d, sc, nc, mb; /* (lo, hi) sub-block pairs: sc = (sl, sh/16), nc = (-1024 sl, -64 sh), mb = -(dmin m) */
    MDEV void prepare(int j, int kg) {
        /* the first half-block never reads hdr.w: consume it here so its
         * register is not recycled (a write-after-write wait on the load
         * still in flight) before this unit */
        asm volatile("" ::"v"(hdr.w));
        /* 6-bit scale/min pairs of sub-blocks 2g, 2g+1 (g = 2(j&1) + kg/2),
         * packed as (lo | hi << 16): bytes 2hb, 2hb+1 of the scale and min
         * words, plus for g >= 2 the 4-bit parts from byte 8+hb / 10+hb
         * (inference/src/format.m:41-64) */
        const uint32_t hb = (uint32_t)kg >> 1, sel = 0x0C010C00u + hb * 0x00020002u;
        uint32_t s2, m2;
        if ((j & 1) == 0) {
            s2 = __builtin_amdgcn_perm(0u, hdr.y, sel) & 0x003F003Fu;
            m2 = __builtin_amdgcn_perm(0u, hdr.z, sel) & 0x003F003Fu;
        } else {
            const uint32_t sp = (hdr.w >> (8 * hb)) & 0xFFu, mp = (hdr.w >> (8 * hb + 16)) & 0xFFu;
            s2 = ((sp | (sp << 12)) & 0x000F000Fu) | ((__builtin_amdgcn_perm(0u, hdr.y, sel) >> 2) & 0x00300030u);
            m2 = ((mp | (mp << 12)) & 0x000F000Fu) | ((__builtin_amdgcn_perm(0u, hdr.z, sel) >> 2) & 0x00300030u);
        }
        const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 S = or_bias(s2) - bias, M = or_bias(m2) - bias; /* exact small integers */
        sc = S * h2{(_Float16)1.0f, (_Float16)0.0625f};
        nc = S * h2{(_Float16)-1024.0f, (_Float16)-64.0f};
        const _Float16 dmin = __builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
        mb = M * h2{-dmin, -dmin}; /* RN(dmin m), as fp16 of the exact fp32 product */
        d = splat(__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu)));
    }
    /* k order of the result: l, l+2, l+1, l+3, l+32, l+34, l+33, l+35 */
    MDEV h8 frag(int s) const {
        const uint32_t w = u4_at(q, s);
        /* bytes 1 and 3 under the 0x64 exponent byte: (0x64 b1, 0x64 b3);
         * bytes 0 and 2 masked and OR-ed under it in one three-input op
         * (truth table 0xEA: (a & b) | c) */
        const uint32_t p13 = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);
        const h2 t0 = hfma(as_h2(__builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA)), splat(sc.x), splat(nc.x));
        const h2 t1 = hfma(as_h2(p13 & 0xFF0FFF0Fu), splat(sc.x), splat(nc.x));
        const h2 t2 = hfma(as_h2(__builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x64006400u, 0xEA)), splat(sc.y), splat(nc.y));
        const h2 t3 = hfma(as_h2(p13 & 0xFFF0FFF0u), splat(sc.y), splat(nc.y));
        return cat4(hfma(t0, d, splat(mb.x)), hfma(t1, d, splat(mb.x)), hfma(t2, d, splat(mb.y)),
                    hfma(t3, d, splat(mb.y)));
    }
};

/* Tile-major Q4_K: per 16-row block and 256-wide super-block, 2304 bytes =
 * the 16 rows' 16-byte headers (d, dmin, scales), then for each 128-k half
 * the 64 lanes' 16 quant bytes in lane order (kg * 16 + i).  A wave's quant
 * load is one contiguous 1 KB and its header load 256 B, where the row-major
 * layout touches 16 rows 1152 B apart.  `p` is the block base plus 16 i. */
template <>
struct Span<FQ4KT> : Span<FQ4K> {
    template <bool NT = false>
    MDEV void load(const uint8_t *p, int j, int kg) {
        const uint8_t *b = p + (size_t)(j >> 1) * 2304;
        hdr = ld_w<NT>(b);
        q = ld_w<NT>(b + 256 + (j & 1) * 1024 + kg * 256);
    }
};

/* Q5_K (176-byte super-blocks: header as Q4_K, qh[32] @16, ql[128] @48):
 * the lane mapping of Q4_K, with bit 2g (low values) or 2g+1 (high) of
 * qh[l] as the fifth bit (inference/src/format.m:110-141).  The values are
 * moved to the low bits, so the exact q*sc (<= 31*63 < 2048) takes the
 * scales unscaled. */
template <>
struct Span<FQ5K> {
    u4 hdr, q, qh;
    MDEV void init(int) {}
    template <bool NT = false>
    MDEV void load(const uint8_t *row, int j, int kg) {
        const uint8_t *p = row + (size_t)(j >> 1) * 176;
        hdr = ld_w<NT>(p);
        q = ld_w<NT>(p + 48 + 16 * (kg + 4 * (j & 1)));
        qh = ld_w<NT>(p + 16 + 16 * (kg & 1));
    }
    h2 d, sc, nc, mb;
    int sh_lo; /* qh bit of the low values: 2g, g = 2(j&1) + kg/2 */
    MDEV void prepare(int j, int kg) {
        asm volatile("" ::"v"(hdr.w));
        const uint32_t hb = (uint32_t)kg >> 1, sel = 0x0C010C00u + hb * 0x00020002u;
        uint32_t s2, m2;
        if ((j & 1) == 0) {
            s2 = __builtin_amdgcn_perm(0u, hdr.y, sel) & 0x003F003Fu;
            m2 = __builtin_amdgcn_perm(0u, hdr.z, sel) & 0x003F003Fu;
        } else {
            const uint32_t sp = (hdr.w >> (8 * hb)) & 0xFFu, mp = (hdr.w >> (8 * hb + 16)) & 0xFFu;
            s2 = ((sp | (sp << 12)) & 0x000F000Fu) | ((__builtin_amdgcn_perm(0u, hdr.y, sel) >> 2) & 0x00300030u);
            m2 = ((mp | (mp << 12)) & 0x000F000Fu) | ((__builtin_amdgcn_perm(0u, hdr.z, sel) >> 2) & 0x00300030u);
        }
        const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 S = or_bias(s2) - bias, M = or_bias(m2) - bias;
        sc = S;
        nc = S * h2{(_Float16)-1024.0f, (_Float16)-1024.0f};
        const _Float16 dmin = __builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
        mb = M * h2{-dmin, -dmin};
        d = splat(__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu)));
        sh_lo = 2 * (2 * (j & 1) + (kg >> 1));
    }
    /* k order of the result: l, l+2, l+1, l+3, l+32, l+34, l+33, l+35 */
    MDEV h8 frag(int s) const {
        const uint32_t w = u4_at(q, s), h = u4_at(qh, s);
        const uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> sh_lo) & 0x01010101u) << 4);
        const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (sh_lo + 1)) & 0x01010101u) << 4);
        const h2 t0 = hfma(as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04020400u)), splat(sc.x), splat(nc.x));
        const h2 t1 = hfma(as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030401u)), splat(sc.x), splat(nc.x));
        const h2 t2 = hfma(as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04020400u)), splat(sc.y), splat(nc.y));
        const h2 t3 = hfma(as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030401u)), splat(sc.y), splat(nc.y));
        return cat4(hfma(t0, d, splat(mb.x)), hfma(t1, d, splat(mb.x)), hfma(t2, d, splat(mb.y)),
                    hfma(t3, d, splat(mb.y)));
    }
};

/* Tile-major Q5_K: per 16-row block and super-block, 2816 bytes = the 16
 * rows' 16-byte headers, the 64 lanes' 16 quant bytes per 128-k half in lane
 * order (as Q4_K), then the qh bytes: for g = kg & 1, the 16 rows' bytes
 * 16g .. 16g+15 of qh.  `p` is the block base plus 16 i. */
template <>
struct Span<FQ5KT> : Span<FQ5K> {
    template <bool NT = false>
    MDEV void load(const uint8_t *p, int j, int kg) {
        const uint8_t *b = p + (size_t)(j >> 1) * 2816;
        hdr = ld_w<NT>(b);
        q = ld_w<NT>(b + 256 + (j & 1) * 1024 + kg * 256);
        qh = ld_w<NT>(b + 2304 + (kg & 1) * 256);
    }
};

template <>
struct Span<FQ6K> {
    u4 ql, qh;
    u2 sc8;
    uint32_t dw;
    int odd2;
    MDEV void init(int kg) { odd2 = 2 * (kg & 1); }
    template <bool NT = false>
    MDEV void load(const uint8_t *row, int j, int kg) {
        const uint8_t *p = row + (size_t)(j >> 1) * 210;
        const int h = j & 1, lq = 16 * (kg >> 1);
        ql = ld_u32x4_a2(p + h * 64 + 32 * (kg & 1) + lq);
        qh = ld_u32x4_a2(p + 128 + h * 32 + lq);
        sc8 = ld_u32x2_a2(p + 192 + h * 8);
        dw = ld_u32_a2(p + 208);
    }
    h2 d, scl, sch;
    MDEV void prepare(int, int kg) {
        const int b = (kg >> 1) + 2 * (kg & 1); /* scale is + 2 odd, is = l / 16 = kg >> 1 */
        d = splat(__builtin_bit_cast(_Float16, (uint16_t)(dw & 0xFFFFu)));
        scl = splat((_Float16)(float)(int8_t)((sc8.x >> (8 * b)) & 0xFF));
        sch = splat((_Float16)(float)(int8_t)((sc8.y >> (8 * b)) & 0xFF));
    }
    /* k order of the result: l, l+2, l+1, l+3, then the same 64 further */
    MDEV h8 frag(int s) const {
        const uint32_t a = u4_at(ql, s), b = u4_at(qh, s);
        h2 p02, p13, r02, r13;
        q6_h2_0213(a, b, 0, odd2, p02, p13);
        q6_h2_0213(a, b, 4, 4 + odd2, r02, r13);
        return cat4((p02 * scl) * d, (p13 * scl) * d, (r02 * sch) * d, (r13 * sch) * d);
    }
};

/* Tile-major Q6_K: per 16-row block and super-block, 3360 bytes (16 rows of
 * 210) = for each 128-k half the 64 lanes' 16 low-bit bytes in lane order
 * (kg * 16 + i), then for each half the high-bit bytes of lane groups
 * (kg >> 1) * 16 + i, then each row's 16 scales, then the 16 rows' d.  All
 * but d are aligned 16-, 8-byte loads.  `p` is the block base plus 16 i. */
template <>
struct Span<FQ6KT> : Span<FQ6K> {
    template <bool NT = false>
    MDEV void load(const uint8_t *p, int j, int kg) {
        const uint8_t *b = p + (size_t)(j >> 1) * 3360;
        const int h = j & 1, i = (int)(threadIdx.x & 15);
        ql = ld_w<NT>(b + h * 1024 + kg * 256);
        qh = ld_w<NT>(b + 2048 + h * 512 + (kg >> 1) * 256);
        sc8 = *(const u2 *)(b + 3072 + h * 8);
        dw = *(const uint16_t *)(b + 3328 - 14 * i);
    }
};

template <>
struct Span<FQ8> {
    u2 qv[4];
    uint32_t dd[4];
    MDEV void init(int) {}
    template <bool NT = false>
    MDEV void load(const uint8_t *row, int j, int kg) {
        const uint8_t *p = row + (size_t)(4 * j) * 34;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            qv[s] = ld_u32x2_a2(p + s * 34 + 2 + 8 * kg);
            dd[s] = ld_u32_a2(p + s * 34);
        }
    }
    MDEV void prepare(int, int) {}
    MDEV h8 frag(int s) const {
        const h2 d = splat(__builtin_bit_cast(_Float16, (uint16_t)(dd[s] & 0xFFFFu)));
        h2 p02, p13, p46, p57; /* k order l, l+2, l+1, l+3, l+4, l+6, l+5, l+7 */
        q8_h2_0213(qv[s].x, p02, p13);
        q8_h2_0213(qv[s].y, p46, p57);
        return cat4(p02 * d, p13 * d, p46 * d, p57 * d);
    }
};

/* Tile-major Q8_0: per 16-row block and 128-k stage, 2176 bytes = the 64
 * lanes' 32 quant bytes in lane order (lane kg * 16 + i: row i, blocks 4j..4j+3,
 * bytes 8kg..8kg+7 of each), then the 16 rows' four fp16 scales.  Aligned
 * 16-byte loads (row-major Q8_0 blocks are 34 bytes, 2-byte aligned) and
 * half the registers per stage.  `p` is the 16-row block base. */
template <>
struct Span<FQ8T> {
    u4 q0, q1;
    u2 dd;
    MDEV void init(int) {}
    template <bool NT = false>
    MDEV void load(const uint8_t *p, int j, int) {
        const int ln = threadIdx.x & 63;
        const uint8_t *b = p + (size_t)j * 2176;
        q0 = ld_w<NT>(b + 32 * ln);
        q1 = ld_w<NT>(b + 32 * ln + 16);
        typedef const __attribute__((address_space(1))) u2 *gp2;
        dd = *(gp2)(uintptr_t)(b + 2048 + 8 * (ln & 15));
    }
    MDEV void prepare(int, int) {}
    MDEV h8 frag(int s) const {
        const uint32_t dw = s < 2 ? dd.x : dd.y;
        const h2 d = splat(__builtin_bit_cast(_Float16, (uint16_t)((s & 1) ? dw >> 16 : dw & 0xFFFFu)));
        const uint32_t w0 = s == 0 ? q0.x : s == 1 ? q0.z : s == 2 ? q1.x : q1.z;
        const uint32_t w1 = s == 0 ? q0.y : s == 1 ? q0.w : s == 2 ? q1.y : q1.w;
        h2 p02, p13, p46, p57; /* k order l, l+2, l+1, l+3, l+4, l+6, l+5, l+7 */
        q8_h2_0213(w0, p02, p13);
        q8_h2_0213(w1, p46, p57);
        return cat4(p02 * d, p13 * d, p46 * d, p57 * d);
    }
};

DEV f4v mfma(h8 a, h8 b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

/* ------------------------------------------------------- B chunks */
/* A chunk is KCH (256) k of the tile's token rows in LDS, row pitch BLD
 * halves (136 dwords; measured conflict-free for the B-fragment reads, where
 * a 132-dword pitch doubles the LDS cycles),
 * each 128-k half in the fragment order of FMT.  A thread's vector n covers
 * token 16n + tid/32, k 8 (tid%32) .. +7.  Every thread loads and stores all
 * TBM vectors: rows past the tile read an all-zero row, so the code stays
 * straight-line (exact wait counts for the weight ring) and needs no
 * select. */
template <int TBM>
struct Chunk {
    static constexpr int W = Shape<TBM>::W, NV = Shape<TBM>::NV, TR = TBM * 16;
    u4 v[NV];
    /* chunk row of this thread's vector n, clamped to `lim` only where the
     * last pass runs past the tile */
    MDEV int row(int n, int lim) const {
        const int r = (W * 2) * n + (int)(threadIdx.x >> 5);
        return NV * W * 2 > TR ? min(r, lim) : r;
    }
    MDEV void fetch(const _Float16 *src, const int *rowoff, int ld, int k0) {
        const int cc = (threadIdx.x & 31) * 8;
#pragma unroll
        for (int n = 0; n < NV; n++)
            v[n] = ld_u4((const uint8_t *)(src + (size_t)rowoff[row(n, TR - 1)] * ld + k0 + cc));
    }
    template <int FMT>
    MDEV void store(_Float16 *xs) const {
        const int col = threadIdx.x & 31, half = col >> 4, c0 = (col & 15) * 2;
        const int p0 = half * KC + frag_pos<FMT>(c0), p1 = half * KC + frag_pos<FMT>(c0 + 1);
#pragma unroll
        for (int n = 0; n < NV; n++) {
            _Float16 *row = xs + this->row(n, TR) * BLD;
            *(u2 *)(row + p0) = u2{v[n].x, v[n].y};
            *(u2 *)(row + p1) = u2{v[n].z, v[n].w};
        }
    }
};

/* ------------------------------------------------------------- tile */
/* One block: Shape<TBM>::W waves, wave w owns RPW row blocks of 16 rows (rows
 * yb*NB + (w*RPW + rb)*16 ..) of NMAT matrices (gate+up, or down).
 * A wave walks units u = (rb, stage j) in order, stage j = 128 k; weight
 * bytes for unit u+DEPTH are in flight while unit u computes.  Activation
 * chunks (256 k) sit in two LDS buffers: with <= 2 chunks both stay resident
 * (one barrier in all); with more, chunk c+2 is written into c's buffer
 * after the barrier that ends chunk c (RPW must be 1 then). */
template <int FMT, int NMAT, int RPW, int DEPTH, int NST, int TBM, bool NT, typename Epi, typename Fill>
DEV void tile_run(const uint8_t *w0, const uint8_t *w1, int in_dim, const _Float16 *src, int ld,
                  const int *rowoff, int rows, int yb, _Float16 *xs, const Epi &epi, const Fill &fill) {
    const int tb = (rows + 15) >> 4;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kg = lane >> 4, i = lane & 15;
    const size_t rbytes = gemm_row_bytes(FMT, in_dim);
    /* NST > 0: stage count fixed at compile time, so the unit loop unrolls
     * completely and the prefetch ring never crosses a loop back-edge (where
     * the register copies would wait for every load in flight) */
    const int nst = NST ? NST : in_dim / KC, nch = nst / 2, U = RPW * nst;
    const int rbase = yb * (Shape<TBM>::W * 16 * RPW) + wv * 16 * RPW;
    const uint8_t *rw0 = w0 + lane_row<FMT>(rbase, i, rbytes);
    const uint8_t *rw1 = NMAT > 1 ? w1 + lane_row<FMT>(rbase, i, rbytes) : nullptr;

    /* U is a multiple of DEPTH (checked by the launchers); the last DEPTH
     * units reload unit U-1 instead of branching */
    Span<FMT> ring[DEPTH][NMAT];
#pragma unroll
    for (int d = 0; d < DEPTH; d++) {
        const int rb = d / nst, j = d - rb * nst;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            ring[d][m].init(kg);
            ring[d][m].template load<NT>((m ? rw1 : rw0) + (size_t)rb * 16 * rbytes, j, kg);
        }
    }

    /* the tile's token rows (rowoff), formed while the first weight stages
     * are in flight; fill ends with a block barrier */
    fill();
    Chunk<TBM> ch;
    ch.fetch(src, rowoff, ld, 0);
    ch.template store<FMT>(xs);
    if (nch > 1) {
        ch.fetch(src, rowoff, ld, KCH);
        ch.template store<FMT>(xs + Shape<TBM>::XR * BLD);
    }
    if (nch > 2) ch.fetch(src, rowoff, ld, 2 * KCH);
    __syncthreads();

    f4v c[NMAT][TBM];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int t = 0; t < TBM; t++) c[m][t] = f4v{0, 0, 0, 0};

#pragma unroll
    for (int u0 = 0; u0 < U; u0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
            const int u = u0 + d;
            const int rb = u / nst, j = u - rb * nst;
            /* keep units apart (register pressure): no scheduling across
             * them, and no reuse of B fragments loaded by an earlier unit
             * (row blocks of one wave read the same LDS addresses) */
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");
            Span<FMT> cur[NMAT];
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                cur[m] = ring[d][m];
                cur[m].prepare(j, kg);
            }
            {
                const int u2 = min(u + DEPTH, U - 1), rb2 = u2 / nst, j2 = u2 - rb2 * nst;
#pragma unroll
                for (int m = 0; m < NMAT; m++) ring[d][m].template load<NT>((m ? rw1 : rw0) + (size_t)rb2 * 16 * rbytes, j2, kg);
            }
            const _Float16 *bp = xs + ((j >> 1) & 1) * (Shape<TBM>::XR * BLD) + (j & 1) * KC + i * BLD + kg * 8;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                h8 a[NMAT];
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    a[m] = cur[m].frag(s);
                }
                /* B reads for every token block (rows past the tile hold
                 * zeros): straight-line LDS traffic the scheduler can hoist */
                h8 b[TBM];
#pragma unroll
                for (int t = 0; t < TBM; t++) {
                    b[t] = *(const h8 *)(bp + t * 16 * BLD + s * 32);
                }
                /* every token block, also past the tile (zero rows): no
                 * branches between the matrix instructions, so the scheduler
                 * can interleave them with the next step's dequant */
#pragma unroll
                for (int t = 0; t < TBM; t++)
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        c[m][t] = mfma(a[m], b[t], c[m][t]);
                    }
            }
            if (j == nst - 1) {
                epi.template operator()<TBM>(c, rbase + rb * 16 + 4 * kg, tb);
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int t = 0; t < TBM; t++) c[m][t] = f4v{0, 0, 0, 0};
            }
            if (nch > 2 && (j & 1) && (j >> 1) + 2 < nch) {
                __syncthreads();
                ch.template store<FMT>(xs + ((j >> 1) & 1) * (Shape<TBM>::XR * BLD));
                if ((j >> 1) + 3 < nch) ch.fetch(src, rowoff, ld, ((j >> 1) + 3) * KCH);
            } else if (nch > 2 && (j & 1) && (j >> 1) + 1 < nch) {
                __syncthreads(); /* chunk c+1 was stored before the previous barrier */
            }
        }
    }
}

/* Block -> (tile, row block).  Work-groups go to the 8 XCDs round-robin by
 * linear id, so the NYB row blocks of one tile are given ids 8 apart: same
 * XCD (one L2 for the tile's gathered activation rows) and dispatched close
 * together.  The grid holds ceil(tiles/8)*8*NYB blocks. */
DEV void block_tile(int nyb, int &tile, int &yb) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    tile = (slot / nyb) * 8 + xcd;
    yb = slot % nyb;
}
struct GemmArgs {
    const uint8_t *wa, *wb;   /* gate/up (wb NULL for down) of expert 0 */
    size_t stride_a, stride_b;
    const uint8_t *sh_a, *sh_b;
    const _Float16 *src;      /* x16 [T][H] (gate/up) or act [pairs][M] (down) */
    const _Float16 *src_sh;   /* down: act_sh [T][S] */
    int T, H, M, S, K, E;
    int zrow, zrow_sh;        /* all-zero rows of src / src_sh (rows past a tile read them) */
    int nyb;                  /* row blocks per tile */
    int uwin;                 /* tiles walked: all (0), the last uwin (> 0) or all but the last -uwin (< 0) */
    const uint32_t *tiles, *pairs;
    _Float16 *act, *act_sh;   /* gate/up outputs */
    unsigned long long *kt;   /* gate/up: per-block launch stamps (KT_BEGIN / KT_END) or NULL */
    float *y, *ysh;           /* down outputs */
    /* self-dispatch (the gate/up over the small-tile list, sd set; sd_tile) */
    int sd, sd_g, nsh;        /* on; rows of dcnt; the shared expert's tiles at the list's end */
    const uint32_t *dcnt;     /* [sd_g][E] expert counts per 256-token block (the exact top-k's) */
    const uint8_t *tmask;     /* [E][TMASK_LD(T)] token marks per expert (the exact top-k's) */
    const int32_t *idx;       /* [T][K] the selections */
    uint32_t *offsets, *pos, *pairs_out, *tiles_out;
};

/* Self-dispatch of the 32-row tile list (T K <= 32 E, E <= the block's 256
 * threads, T <= 1024), in place of the dispatch kernel.  Every gate/up
 * block forms the list that kernel would write from the exact top-k's
 * per-256-token-block expert counts (order-free atomic adds): expert e's
 * pairs 32 at a time, experts ascending, then the shared expert's
 * ceil(T/32) tiles.  Its tile's token rows come from expert e's token marks
 * (a byte per token, set by the top-k) in token order, which is the
 * dispatch kernel's order (pair id ascending within an expert).  The
 * yb = 0 block of a tile writes the tile's list entry and its pairs' sorted
 * positions (pairs, pos) for the down projection and the combine; block
 * (0, 0) writes the count and the offsets.  sd_locate finds the block's
 * tile (false: a block past the list); every thread of the block calls it.
 * At T = 512 this took the layer from 156.8-157.3 to 150.6-152.1 us. */
DEV bool sd_locate(const GemmArgs &a, int ti, int yb, uint32_t &e, uint32_t &first, uint32_t &rows, uint32_t &base) {
    __shared__ uint32_t wsum[32], sel[4];
    const int tid = threadIdx.x, E = a.E;
    uint32_t cg[4];
#pragma unroll
    for (int g = 0; g < 4; g++) cg[g] = a.dcnt[(size_t)min(g, a.sd_g - 1) * E + min(tid, E - 1)];
    uint32_t c = 0;
#pragma unroll
    for (int g = 0; g < 4; g++)
        if (g < a.sd_g) c += cg[g];
    if (tid >= E) c = 0;
    const uint32_t nt = (c + 31u) >> 5;
    uint32_t x = c, y = nt, tx, ty;
    scan2_block(x, y, wsum, tx, ty);
    /* counts that do not add up to T K (state not cleared) give an empty
     * list rather than tiles past the buffers */
    const uint32_t off = x - c, t0 = y - nt, ntiles = tx == (uint32_t)(a.T * a.K) ? ty + (uint32_t)a.nsh : 0u;
    if (ti == 0 && yb == 0) {
        if (tid < E) a.offsets[tid] = off;
        if (tid == 0) {
            a.offsets[E] = tx;
            a.tiles_out[0] = ntiles;
        }
    }
    if ((uint32_t)ti >= ntiles) return false;
    if (tid < E && nt && (uint32_t)ti >= t0 && (uint32_t)ti < t0 + nt) {
        const uint32_t b = ((uint32_t)ti - t0) * 32u;
        sel[0] = (uint32_t)tid;
        sel[1] = off + b;
        sel[2] = min(32u, c - b);
        sel[3] = b;
    }
    if ((uint32_t)ti >= ty && tid == 0) {
        const uint32_t f = ((uint32_t)ti - ty) * 32u;
        sel[0] = (uint32_t)E;
        sel[1] = f;
        sel[2] = min(32u, (uint32_t)a.T - f);
        sel[3] = 0;
    }
    lds_barrier();
    e = __builtin_amdgcn_readfirstlane(sel[0]);
    first = __builtin_amdgcn_readfirstlane(sel[1]);
    rows = __builtin_amdgcn_readfirstlane(sel[2]);
    base = __builtin_amdgcn_readfirstlane(sel[3]);
    if (yb == 0 && tid == 0) {
        a.tiles_out[1 + 3 * ti] = e;
        a.tiles_out[2 + 3 * ti] = first;
        a.tiles_out[3 + 3 * ti] = rows;
    }
    return true;
}

/* The located tile's token rows into rowoff (rows past the tile: the zero
 * row), then a block barrier; the yb = 0 block then writes the pairs'
 * sorted positions.  Every thread of the block calls it. */
DEV void sd_rows(const GemmArgs &a, int yb, uint32_t e, uint32_t first, uint32_t rows, uint32_t base, int *rowoff) {
    const int tid = threadIdx.x;
    const bool sh = e == (uint32_t)a.E;
    if (sh) {
        if (tid < 32) rowoff[tid] = (uint32_t)tid < rows ? (int)first + tid : a.zrow;
    } else if (tid < 64) {
        /* wave 0: lane l holds the marks of tokens 16 l .. 16 l + 15 (T <=
         * 1024); a token's rank is the marks of the lanes below plus those
         * below it in its lane */
        const u4 v = *(const u4 *)(a.tmask + (size_t)e * TMASK_LD(a.T) + min(16 * tid, TMASK_LD(a.T) - 16));
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < 16; j++)
            if ((u4_at(v, j >> 2) >> (8 * (j & 3))) & 0xFFu) m |= 1u << j;
        if (16 * tid >= a.T) m = 0u;
        uint32_t incl = (uint32_t)__builtin_popcount(m);
        /* inclusive prefix over the wave's lanes (DPP), as in scan2_block */
#define SD_SCAN(CTRL, ROWS) incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, CTRL, ROWS, 0xF, false)
        SD_SCAN(0x111, 0xF);
        SD_SCAN(0x112, 0xF);
        SD_SCAN(0x114, 0xF);
        SD_SCAN(0x118, 0xF);
        SD_SCAN(0x142, 0xA);
        SD_SCAN(0x143, 0xC);
#undef SD_SCAN
        if (tid < 32) rowoff[tid] = a.zrow;
        int r = (int)(incl - (uint32_t)__builtin_popcount(m)) - (int)base;
        uint32_t mm = m;
        while (mm) {
            const int j = __builtin_ctz(mm);
            mm &= mm - 1u;
            if (r >= 0 && r < (int)rows) rowoff[r] = tid * 16 + j;
            r++;
        }
    }
    lds_barrier();
    if (!sh && yb == 0 && (uint32_t)tid < rows) {
        /* the pair of row tid: the slot in which its token picked e */
        const uint32_t t = (uint32_t)rowoff[tid];
        uint32_t k = 0;
        for (int q = 0; q < a.K; q++)
            if (a.idx[(size_t)t * a.K + q] == (int32_t)e) k = (uint32_t)q;
        const uint32_t pr = t * (uint32_t)a.K + k;
        a.pairs_out[first + tid] = pr;
        a.pos[pr] = first + tid;
    }
}

/* D layout: lane (i, kg) holds token 16t + i, rows r..r+3 (r = 4kg + block base) */
struct GuEpi {
    _Float16 *out;
    int out_ld, first, rows;
    template <int TBM>
    MDEV void operator()(const f4v (&c)[2][TBM], int r, int tb) const {
        const int i = threadIdx.x & 15;
#pragma unroll
        for (int t = 0; t < TBM; t++) {
            const int tok = t * 16 + i;
            if (t >= tb || tok >= rows) continue;
            h4 v; /* act rows are stored (0,2,1,3) within each 4-group */
#pragma unroll
            for (int q = 0; q < 4; q++) v[(q & 1) * 2 + (q >> 1)] = glu_f16(c[0][t][q], c[1][t][q]);
            *(h4 *)(out + (size_t)(first + tok) * out_ld + r) = v;
        }
    }
};

struct DnEpi {
    float *out;
    int out_ld, first, rows;
    template <int TBM>
    MDEV void operator()(const f4v (&c)[1][TBM], int r, int tb) const {
        const int i = threadIdx.x & 15;
#pragma unroll
        for (int t = 0; t < TBM; t++) {
            const int tok = t * 16 + i;
            if (t >= tb || tok >= rows) continue;
            *(f4v *)(out + (size_t)(first + tok) * out_ld + r) = c[0][t];
        }
    }
};

/* row blocks per wave and weight stages in flight per wave */
#define GU_RPW 1
#define DN_RPW 4

/* --------------------------------------------------- persistent stream */
/* A unit is one (tile, row block) of a tile list; uniform over the block. */
struct UnitDesc {
    int valid, sh, first, rows, yb;
    uint32_t e;
};

/* The n-th unit of this block.  Units of tiles t = xcd (mod 8) go to the
 * blocks of that XCD (work-groups are dealt to the 8 XCDs round-robin by
 * linear id), so the row blocks of one tile share an L2 and run at about the
 * same time; within an XCD, block `slot` takes units slot, slot + bpx, ... */
DEV UnitDesc unit_desc(const uint32_t *tiles, int nyb, int E, int n, int uwin) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, bpx = gridDim.x >> 3;
    const int q = slot + n * bpx, ti = 8 * (q / nyb) + xcd;
    /* the list is read-only here: constant address space, so the uniform
     * reads are scalar loads and do not wait behind the weight loads */
    typedef const __attribute__((address_space(4))) uint32_t cu32;
    cu32 *tl = (cu32 *)(uintptr_t)tiles;
    /* the window of tiles walked (the shared expert's tiles end the list) */
    const uint32_t nall = tl[0];
    uint32_t base = 0, cnt = nall;
    if (uwin > 0) {
        cnt = nall < (uint32_t)uwin ? nall : (uint32_t)uwin;
        base = nall - cnt;
    } else if (uwin < 0) {
        cnt = nall > (uint32_t)-uwin ? nall - (uint32_t)-uwin : 0u;
    }
    UnitDesc u;
    u.valid = (uint32_t)ti < cnt;
    u.yb = q % nyb;
    const int tc = u.valid ? (int)base + ti : 0; /* entry 0 exists whenever the list is read */
    u.e = u.valid ? tl[1 + 3 * tc] : 0u;
    u.first = u.valid ? (int)tl[2 + 3 * tc] : 0;
    u.rows = u.valid ? (int)tl[3 + 3 * tc] : 0;
    u.sh = u.e == (uint32_t)E;
    return u;
}

/* Persistent form of tile_run: the block walks its units back to back and
 * the weight ring and the activation chunk stream run on across unit
 * boundaries, so only the first unit waits for its loads.  Per unit the
 * arithmetic is exactly tile_run's (same fragments, same MFMA order).
 *   - weight stage u + DEPTH of unit n is unit n+1's stage u + DEPTH - U;
 *   - global chunk C = n * nch + c sits in LDS buffer C % 3.  Before the
 *     barrier that ends chunk C, chunk C + 2 is stored (its buffer held
 *     C - 1, which every wave finished before the previous barrier) and
 *     C + 3 fetched into registers, so nothing waits after the barrier and
 *     chunk C + 1 is readable a whole chunk before it is used;
 *   - B fragments are read one MFMA step ahead (across stages, chunks and
 *     units), so the LDS latency hides behind the current step's work;
 *   - token row offsets of unit n sit in LDS slot n % 3, written at the end
 *     of unit n - 2's first chunk (units past the end point every row at the
 *     zero row, so loads and stores stay unconditional).
 * P supplies the unit's weight and source pointers, row offsets and
 * epilogue. */
template <int FMT, int NMAT, int RPW, int DEPTH, int NST, int TBM, typename P>
DEV void tile_stream(const P &pol, _Float16 *xs, int *rowoff) {
    constexpr int W = Shape<TBM>::W, TR = TBM * 16, nst = NST, nch = NST / 2, U = RPW * NST, CB = Shape<TBM>::XR * BLD;
    static_assert(NST % 4 == 0 && U % DEPTH == 0 && (RPW == 1 || nch == 2), "stream shape");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kg = lane >> 4, i = lane & 15;
    const size_t rbytes = gemm_row_bytes(FMT, pol.in_dim());
    UnitDesc cu = pol.desc(0), nu = pol.desc(1);
    if (!cu.valid) return;
    /* this lane's weight row in matrix m of unit u (row block 0, stage 0);
     * a unit past the end reuses `other` (its loads are never consumed) */
    auto wrow = [&](const UnitDesc &u, int m, const uint8_t *other) -> const uint8_t * {
        return u.valid ? pol.weights(u, m) + lane_row<FMT>(u.yb * (W * 16 * RPW) + wv * 16 * RPW, i, rbytes) : other;
    };
    if (threadIdx.x < TR) {
        rowoff[threadIdx.x] = pol.row_fin(cu, pol.row_raw(cu, (int)threadIdx.x));
        rowoff[TR + threadIdx.x] = pol.row_fin(nu, pol.row_raw(nu, (int)threadIdx.x));
    }
    __syncthreads();

    const uint8_t *cw[NMAT], *nw[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        cw[m] = wrow(cu, m, nullptr);
        nw[m] = wrow(nu, m, cw[m]);
    }
    Span<FMT> ring[DEPTH][NMAT];
#pragma unroll
    for (int d = 0; d < DEPTH; d++) {
        const int rb = d / nst, j = d - rb * nst;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            ring[d][m].init(kg);
            ring[d][m].template load<(TBM >= 5)>(cw[m] + (size_t)rb * 16 * rbytes, j, kg);
        }
    }
    /* chunks 0, 1 of the stream into buffers 0, 1, chunk 2 (unit 0's when
     * nch > 2, else unit 1's chunk 0) into registers */
    Chunk<TBM> ch;
    ch.fetch(pol.src(cu), rowoff, pol.ld(), 0);
    ch.template store<FMT>(xs);
    ch.fetch(pol.src(cu), rowoff, pol.ld(), KCH);
    ch.template store<FMT>(xs + CB);
    if (nch > 2) ch.fetch(pol.src(cu), rowoff, pol.ld(), 2 * KCH);
    else ch.fetch(pol.src(nu), rowoff + TR, pol.ld(), 0);
    __syncthreads();

    /* B fragment of token block t, step s of a stage whose chunk sits in
     * buffer `buf` (j & 1 picks the chunk's 128-k half) */
    const _Float16 *bl = xs + i * BLD + kg * 8;
    auto bfrag = [&](int buf, int j, int s, int t) -> h8 {
        return *(const h8 *)(bl + buf * CB + (j & 1) * KC + t * 16 * BLD + s * 32);
    };
    h8 b[TBM];
#pragma unroll
    for (int t = 0; t < TBM; t++) b[t] = bfrag(0, 0, 0, t);

    f4v c[NMAT][TBM];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int t = 0; t < TBM; t++) c[m][t] = f4v{0, 0, 0, 0};

    for (int n = 0;; n++) {
        /* unit n + 2: its row offsets are read here (a global load for
         * routed gate/up rows) and stored into LDS slot (n + 2) % 3 at the
         * end of this unit's first chunk, so the load's wait comes stages
         * later.  That slot was last read by fetches issued in unit n - 1. */
        const UnitDesc fu = pol.desc(n + 2);
        const int s1 = (n + 1) % 3, s2 = (n + 2) % 3;
        const uint32_t ro = threadIdx.x < TR ? pol.row_raw(fu, (int)threadIdx.x) : 0u;
        const int bb = (n * nch) % 3; /* buffer of this unit's chunk 0 */
#pragma unroll
        for (int u0 = 0; u0 < U; u0 += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; d++) {
                const int u = u0 + d;
                const int rb = u / nst, j = u - rb * nst;
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("" ::: "memory");
                Span<FMT> cur[NMAT];
#pragma unroll
                for (int m = 0; m < NMAT; m++) {
                    cur[m] = ring[d][m];
                    cur[m].prepare(j, kg);
                }
                {
                    /* stage u + DEPTH: of this unit, else of the next */
                    const bool here = u + DEPTH < U;
                    const int u2 = here ? u + DEPTH : u + DEPTH - U;
                    const int rb2 = u2 / nst, j2 = u2 - rb2 * nst;
#pragma unroll
                    for (int m = 0; m < NMAT; m++) ring[d][m].template load<(TBM >= 5)>((here ? cw[m] : nw[m]) + (size_t)rb2 * 16 * rbytes, j2, kg);
                }
                /* the stage after this one: next row block or next unit
                 * restart at stage 0, whose chunk 0 is this unit's (row
                 * blocks) or the next unit's */
                const int jn = j + 1 < nst ? j + 1 : 0;
                const int cnext = j + 1 < nst ? (j + 1) >> 1 : rb + 1 < RPW ? 0 : nch;
                const int bufc = (bb + (j >> 1)) % 3, bufn = (bb + cnext) % 3;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    /* next step's B reads first, pinned above this step's
                     * work (the scheduler would otherwise sink each read next
                     * to its use and wait for it there) */
                    h8 bn[TBM];
#pragma unroll
                    for (int t = 0; t < TBM; t++) bn[t] = s < 3 ? bfrag(bufc, j, s + 1, t) : bfrag(bufn, jn, 0, t);
                    __builtin_amdgcn_sched_barrier(0);
                    h8 a[NMAT];
#pragma unroll
                    for (int m = 0; m < NMAT; m++) a[m] = cur[m].frag(s);
#pragma unroll
                    for (int t = 0; t < TBM; t++)
#pragma unroll
                        for (int m = 0; m < NMAT; m++) c[m][t] = mfma(a[m], b[t], c[m][t]);
#pragma unroll
                    for (int t = 0; t < TBM; t++) b[t] = bn[t];
                }
                if (j == nst - 1) {
                    pol.epilogue(cu, c, cu.yb * (W * 16 * RPW) + wv * 16 * RPW + rb * 16 + 4 * kg, (cu.rows + 15) >> 4);
#pragma unroll
                    for (int m = 0; m < NMAT; m++)
#pragma unroll
                        for (int t = 0; t < TBM; t++) c[m][t] = f4v{0, 0, 0, 0};
                }
                if (rb == RPW - 1 && (j & 1)) {
                    /* end of chunk C = n nch + cc: store chunk C + 2, fetch
                     * chunk C + 3 (of unit n + off), then the barrier */
                    const int cc = j >> 1, c3 = cc + 3, off = c3 / nch;
                    if (cc == 0 && threadIdx.x < TR) rowoff[s2 * TR + threadIdx.x] = pol.row_fin(fu, ro);
                    ch.template store<FMT>(xs + ((bb + cc + 2) % 3) * CB);
                    const UnitDesc &tu = off == 0 ? cu : off == 1 ? nu : fu;
                    const int slot = off == 0 ? n % 3 : off == 1 ? s1 : s2;
                    ch.fetch(pol.src(tu), rowoff + slot * TR, pol.ld(), (c3 % nch) * KCH);
                    __syncthreads();
                }
            }
        }
        if (!nu.valid) break;
        cu = nu;
        nu = fu;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            cw[m] = nw[m];
            nw[m] = wrow(nu, m, cw[m]);
        }
    }
}

struct GuPol {
    const GemmArgs &a;
    MDEV int in_dim() const { return a.H; }
    MDEV int ld() const { return a.H; }
    MDEV UnitDesc desc(int n) const { return unit_desc(a.tiles, a.nyb, a.E, n, a.uwin); }
    MDEV const _Float16 *src(const UnitDesc &) const { return a.src; }
    MDEV const uint8_t *weights(const UnitDesc &u, int m) const {
        return u.sh ? (m ? a.sh_b : a.sh_a) : m ? a.wb + (size_t)u.e * a.stride_b : a.wa + (size_t)u.e * a.stride_a;
    }
    /* token row of tile row q in two steps (the pair load, then its use) */
    MDEV uint32_t row_raw(const UnitDesc &u, int q) const {
        if (!u.valid || q >= u.rows) return ~0u;
        return u.sh ? (uint32_t)(u.first + q) : a.pairs[u.first + q];
    }
    MDEV int row_fin(const UnitDesc &u, uint32_t r) const {
        return r == ~0u ? a.zrow : u.sh ? (int)r : (int)(r / (uint32_t)a.K);
    }
    template <int TBM>
    MDEV void epilogue(const UnitDesc &u, const f4v (&c)[2][TBM], int r, int tb) const {
        const GuEpi epi{u.sh ? a.act_sh : a.act, u.sh ? a.S : a.M, u.first, u.rows};
        epi.template operator()<TBM>(c, r, tb);
    }
};

struct DnPol {
    const GemmArgs &a;
    MDEV int in_dim() const { return a.M; }
    MDEV int ld() const { return a.M; }
    MDEV UnitDesc desc(int n) const { return unit_desc(a.tiles, a.nyb, a.E, n, a.uwin); }
    MDEV const _Float16 *src(const UnitDesc &u) const { return u.sh ? a.src_sh : a.src; }
    MDEV const uint8_t *weights(const UnitDesc &u, int) const { return u.sh ? a.sh_a : a.wa + (size_t)u.e * a.stride_a; }
    MDEV uint32_t row_raw(const UnitDesc &u, int q) const { return !u.valid || q >= u.rows ? ~0u : (uint32_t)(u.first + q); }
    MDEV int row_fin(const UnitDesc &u, uint32_t r) const { return r == ~0u ? (u.sh ? a.zrow_sh : a.zrow) : (int)r; }
    template <int TBM>
    MDEV void epilogue(const UnitDesc &u, const f4v (&c)[1][TBM], int r, int tb) const {
        const DnEpi epi{u.sh ? a.ysh : a.y, a.H, u.first, u.rows};
        epi.template operator()<TBM>(c, r, tb);
    }
};


/* The kernel arguments (and the grid size, an implicit argument), fetched
 * in one round of scalar loads at a kernel's entry.  Left alone, the
 * compiler fetches each where a branch first needs it, and every such
 * branch waits for its own round trip (two to four rounds ahead of a
 * block's first vector load). */
#define GEMM_PIN_ARGS(a, ...)                                                                                  \
    asm volatile("" ::"s"(a.wa), "s"(a.wb), "s"(a.stride_a), "s"(a.stride_b), "s"(a.sh_a), "s"(a.sh_b),      \
                 "s"(a.src), "s"(a.src_sh), "s"(a.tiles), "s"(a.pairs), "s"(a.kt), "s"(a.T), "s"(a.H),         \
                 "s"(a.M), "s"(a.S), "s"(a.K), "s"(a.E), "s"(a.zrow), "s"(a.zrow_sh), "s"(a.nyb), "s"(a.uwin), \
                 "s"(gridDim.x), __VA_ARGS__)

/* RF: routed gate/up format (Q4_K, row-major or tile-major); SF: the shared
 * expert's (the same, or Q8_0 row-major) */
template <int RF, int SF, int NST, int TBM>
DEV void k_gemm_gate_up_body(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[2 * Shape<TBM>::XR * BLD];
    __shared__ int rowoff[TBM * 16];
    int ti, yb;
    block_tile(a.nyb, ti, yb);
    uint32_t e, first, rows, base = 0;
    const bool sd = TBM == 2 && a.sd;
    if (sd) {
        if (!sd_locate(a, ti, yb, e, first, rows, base)) return;
    } else {
        const uint32_t nt = a.tiles[0];
        if ((uint32_t)ti >= nt) return;
        e = a.tiles[1 + 3 * ti];
        first = a.tiles[2 + 3 * ti];
        rows = a.tiles[3 + 3 * ti];
    }
    const bool sh = e == (uint32_t)a.E;
    if (yb * (Shape<TBM>::W * 16 * GU_RPW) >= (sh ? a.S : a.M)) return;
    /* the token rows, formed inside tile_run once its first weight loads
     * are issued */
    auto fill = [&]() {
        if (sd) {
            sd_rows(a, yb, e, first, rows, base, rowoff);
        } else {
            if (threadIdx.x < TBM * 16) { /* rows past the tile read the zero row */
                const uint32_t q = threadIdx.x;
                rowoff[threadIdx.x] = q >= rows ? a.zrow : sh ? (int)(first + q) : (int)(a.pairs[first + q] / (uint32_t)a.K);
            }
            lds_barrier();
        }
    };
    constexpr bool NT = TBM >= 5 || TBM == 1;
    /* a 32-row tile holding at most 16 rows runs the 16-row code: half the
     * matrix instructions and B-fragment reads, the same weight stream */
    if (sh) {
        const GuEpi epi{a.act_sh, a.S, (int)first, (int)rows};
        constexpr int D = SF == FQ8 || SF == FQ8T ? 2 : Shape<TBM>::DEPTH;
        if (TBM == 2 && rows <= 16)
            tile_run<SF, 2, GU_RPW, D, NST, 1, NT>(a.sh_a, a.sh_b, a.H, a.src, a.H, rowoff, (int)rows, yb, xs, epi, fill);
        else tile_run<SF, 2, GU_RPW, D, NST, TBM, NT>(a.sh_a, a.sh_b, a.H, a.src, a.H, rowoff, (int)rows, yb, xs, epi, fill);
    } else {
        const GuEpi epi{a.act, a.M, (int)first, (int)rows};
        const uint8_t *w0 = a.wa + (size_t)e * a.stride_a, *w1 = a.wb + (size_t)e * a.stride_b;
        if (TBM == 2 && rows <= 16)
            tile_run<RF, 2, GU_RPW, Shape<TBM>::DEPTH, NST, 1, NT>(w0, w1, a.H, a.src, a.H, rowoff, (int)rows, yb, xs, epi, fill);
        else tile_run<RF, 2, GU_RPW, Shape<TBM>::DEPTH, NST, TBM, NT>(w0, w1, a.H, a.src, a.H, rowoff, (int)rows, yb, xs, epi, fill);
    }
}

template <int RF, int SF, int NST, int TBM>
__global__ __launch_bounds__(Shape<TBM>::W * 64) void k_gemm_gate_up(GemmArgs a) {
    GEMM_PIN_ARGS(a, "s"(a.act), "s"(a.act_sh), "s"(a.sd), "s"(a.sd_g), "s"(a.nsh), "s"(a.dcnt), "s"(a.tmask),
                  "s"(a.idx), "s"(a.offsets), "s"(a.pos), "s"(a.pairs_out), "s"(a.tiles_out));
    KT_BEGIN(a.kt);
    k_gemm_gate_up_body<RF, SF, NST, TBM>(a);
    KT_END(a.kt);
}

template <int EFMT, int SFMT, int NST, int TBM>
__global__ __launch_bounds__(Shape<TBM>::W * 64) void k_gemm_down(GemmArgs a) {
    GEMM_PIN_ARGS(a, "s"(a.y), "s"(a.ysh));
    __shared__ __attribute__((aligned(16))) _Float16 xs[2 * Shape<TBM>::XR * BLD];
    __shared__ int rowoff[TBM * 16];
    int ti, yb;
    block_tile(a.nyb, ti, yb);
    const uint32_t nt = a.tiles[0];
    if ((uint32_t)ti >= nt) return;
    const uint32_t e = a.tiles[1 + 3 * ti], first = a.tiles[2 + 3 * ti], rows = a.tiles[3 + 3 * ti];
    const bool sh = e == (uint32_t)a.E;
    if (threadIdx.x < TBM * 16)
        rowoff[threadIdx.x] = threadIdx.x < rows ? (int)(first + threadIdx.x) : (sh ? a.zrow_sh : a.zrow);
    __syncthreads();
    if (sh) {
        const DnEpi epi{a.ysh, a.H, (int)first, (int)rows};
        tile_run<SFMT, 1, DN_RPW, Shape<TBM>::DEPTH, NST, TBM, (TBM >= 5 || TBM == 1)>(a.sh_a, nullptr, a.S, a.src_sh, a.S, rowoff, (int)rows, yb, xs, epi, [] {});
    } else {
        const DnEpi epi{a.y, a.H, (int)first, (int)rows};
        tile_run<EFMT, 1, DN_RPW, Shape<TBM>::DEPTH, NST, TBM, (TBM >= 5 || TBM == 1)>(a.wa + (size_t)e * a.stride_a, nullptr, a.M, a.src, a.M, rowoff, (int)rows, yb, xs, epi, [] {});
    }
}

/* Persistent big-tile kernels: one block per CU walks its units (tile_stream).
 * Shared expert in the routed format and of the routed width only. */
#ifndef GEMM_PERSIST
#define GEMM_PERSIST 1
#endif
/* small tiles: 0 = per-tile kernels, n = persistent with n blocks per CU
 * (measured: the down projection gains ~10 % at T = 512, gate/up nothing) */
#ifndef GEMM_PERSIST_SMALL
#define GEMM_PERSIST_SMALL 0
#endif
#ifndef GEMM_PERSIST_SMALL_DN
#define GEMM_PERSIST_SMALL_DN 2
#endif
template <int TBM, int GF>
DEV void k_gemm_gate_up_p_body(GemmArgs a) {
    static_assert(TBM >= 2, "persistent kernels take 32- and 80-row tiles");
    __shared__ __attribute__((aligned(16))) _Float16 xs[3 * Shape<TBM>::XR * BLD];
    __shared__ int rowoff[3 * TBM * 16];
    tile_stream<GF, 2, GU_RPW, (GF == FQ8 || GF == FQ8T ? 2 : Shape<TBM>::DEPTH), 16, TBM>(GuPol{a}, xs, rowoff);
}

template <int TBM, int GF>
__global__ __launch_bounds__(Shape<TBM>::W * 64) void k_gemm_gate_up_p(GemmArgs a) {
    GEMM_PIN_ARGS(a, "s"(a.act), "s"(a.act_sh));
    KT_BEGIN(a.kt);
    k_gemm_gate_up_p_body<TBM, GF>(a);
    KT_END(a.kt);
}

template <int EFMT, int TBM>
__global__ __launch_bounds__(Shape<TBM>::W * 64) void k_gemm_down_p(GemmArgs a) {
    GEMM_PIN_ARGS(a, "s"(a.y), "s"(a.ysh));
    /* the launchers send 16-row tile lists (T <= 16) to the per-tile kernels */
    static_assert(TBM >= 2, "persistent kernels take 32- and 80-row tiles");
    __shared__ __attribute__((aligned(16))) _Float16 xs[3 * Shape<TBM>::XR * BLD];
    __shared__ int rowoff[3 * TBM * 16];
    tile_stream<EFMT, 1, DN_RPW, Shape<TBM>::DEPTH, 4, TBM>(DnPol{a}, xs, rowoff);
}

/* Persistent grid: one block per CU, a multiple of the 8 XCDs.  The
 * environment variable OROME_GEMM_PERSIST_BLOCKS overrides it (tests use a
 * small grid to give every block many units); 0 selects the per-tile
 * kernels. */
static unsigned persist_blocks() {
    static int n[64];
    if (const char *env = getenv("OROME_GEMM_PERSIST_BLOCKS")) {
        const long v = strtol(env, nullptr, 10);
        return v <= 0 ? 0u : v < 8 ? 8u : (unsigned)(v / 8 * 8);
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!n[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 8) v = 256;
        n[dev] = v / 8 * 8;
    }
    return (unsigned)n[dev];
}

/* ------------------------------------------------------------ launch */
/* Waves per block of a tile size (16- and 32-row tiles share a shape). */
static_assert(Shape<GEMM_TILE_MIN / 16>::W == Shape<GEMM_TILE_SMALL / 16>::W, "tile shapes");
static int tile_waves(int tile_m) {
    return tile_m == GEMM_TILE_BIG ? Shape<GEMM_TILE_BIG / 16>::W : Shape<GEMM_TILE_SMALL / 16>::W;
}
/* Shapes and formats the launchers take (0) or decline (-2). */
static int gate_up_shape(const ExpertSide &ex, const SharedSide &sh, int H, int M, int tile_m) {
    const int W = tile_waves(tile_m);
    const int NB = W * 16 * GU_RPW;
    if ((H / KC * GU_RPW) % 4) return -2; /* every ring depth used divides the unit count */
    if (H % KCH || M % NB || (sh.gate && sh.S % NB) || (ex.gate_fmt != FQ4K && ex.gate_fmt != FQ4KT)) return -2;
    /* shared expert: the routed format, or Q8_0 (row-major, or tile-major
     * beside tile-major routed matrices) */
    if (sh.gate && sh.gate_fmt != ex.gate_fmt && sh.gate_fmt != FQ8 && !(sh.gate_fmt == FQ8T && ex.gate_fmt == FQ4KT))
        return -2;
    return 0;
}
static int down_shape(const ExpertSide &ex, const SharedSide &sh, int H, int M, int tile_m) {
    const int W = tile_waves(tile_m);
    const int NB = W * 16 * DN_RPW;
    if ((M / KC * DN_RPW) % 4 || (sh.gate && (sh.S / KC * DN_RPW) % 4)) return -2;
    /* all of a tile's activations stay resident: in_dim <= 2 chunks */
    if (H % NB || M % KCH || M > 2 * KCH || (sh.gate && (sh.S % KCH || sh.S > 2 * KCH))) return -2;
    const bool dtiled = ex.down_fmt == FQ4KT || ex.down_fmt == FQ5KT || ex.down_fmt == FQ6KT || ex.down_fmt == FQ8T;
    /* (a Q8_0 routed down only reaches here from the weight read-back debug
     * entry; the forward rejects it) */
    if (ex.down_fmt != FQ4K && ex.down_fmt != FQ5K && ex.down_fmt != FQ6K && ex.down_fmt != FQ8 && !dtiled) return -2;
    /* shared down: any supported format, tile-major beside a tile-major
     * routed down (the packer makes both) */
    const int sf = sh.gate ? sh.down_fmt : ex.down_fmt;
    if (dtiled ? sf != FQ4KT && sf != FQ5KT && sf != FQ6KT && sf != FQ8T
               : sf != FQ4K && sf != FQ5K && sf != FQ6K && sf != FQ8)
        return -2;
    return 0;
}
int gemm_small_tiles_ok(const ExpertSide &ex, const SharedSide &sh, int H, int M) {
    return !gate_up_shape(ex, sh, H, M, GEMM_TILE_SMALL) && !down_shape(ex, sh, H, M, GEMM_TILE_SMALL);
}

/* The shared expert's tiles end the list that holds most of the routed work
 * (the dispatch puts them there); how many of them this list has. */
static int shared_tiles_in(const SharedSide &sh, int T, int K, int E, int tile_m) {
    if (!sh.gate) return 0;
    if (tile_m == GEMM_TILE_MIN) return 1; /* small-batch list: T <= 16, one shared tile */
    const bool sh_small = (size_t)T * K <= (size_t)GEMM_TILE_SMALL * E;
    return (tile_m == GEMM_TILE_SMALL) == sh_small ? (T + tile_m - 1) / tile_m : 0;
}

#ifndef GEMM_SELF_DISPATCH
#define GEMM_SELF_DISPATCH 1
#endif
bool gemm_self_dispatch_ok(int T, int K, int E) {
    const long tk = (long)T * K;
    return GEMM_SELF_DISPATCH && !GEMM_PERSIST_SMALL && E <= 256 && T <= 1024 && tk <= (long)GEMM_TILE_SMALL * E;
}

int launch_gemm_gate_up(const ExpertSide &ex, const SharedSide &sh, const _Float16 *x16, int zrow, int T,
                        int H, int M, int K, int E, int tile_m, const uint32_t *tiles, int n_tiles_max,
                        const uint32_t *pairs, _Float16 *act, _Float16 *act_sh, hipStream_t s,
                        unsigned long long *kt, int kt_cap, const GemmSelfDispatch *sd) {
    if (gate_up_shape(ex, sh, H, M, tile_m)) return -2;
    if (sd && (tile_m != GEMM_TILE_SMALL || !gemm_self_dispatch_ok(T, K, E) || !sd->dcnt || sd->g < 1 || sd->g > 4 || !sd->tmask || !sd->idx || !sd->offsets || !sd->pairs || !sd->pos))
        return -2;
    if (tile_m != GEMM_TILE_SMALL && tile_m != GEMM_TILE_BIG && tile_m != GEMM_TILE_MIN) return -2;
    const int W = tile_waves(tile_m);
    const int NB = W * 16 * GU_RPW;
    const bool tiled = ex.gate_fmt == FQ4KT;
    GemmArgs a = {};
    a.wa = ex.gate; a.wb = ex.up; a.stride_a = ex.gate_stride; a.stride_b = ex.up_stride;
    a.sh_a = sh.gate; a.sh_b = sh.up;
    a.src = x16; a.T = T; a.H = H; a.M = M; a.S = sh.gate ? sh.S : 0; a.K = K; a.E = E;
    a.zrow = zrow; a.zrow_sh = zrow;
    a.tiles = tiles; a.pairs = pairs; a.act = act; a.act_sh = act_sh;
    a.nyb = (M > a.S ? M : a.S) / NB;
    if (sd) {
        a.sd = 1;
        a.nsh = shared_tiles_in(sh, T, K, E, tile_m);
        a.sd_g = sd->g;
        a.dcnt = sd->dcnt;
        a.tmask = sd->tmask;
        a.idx = sd->idx;
        a.offsets = sd->offsets;
        a.pos = sd->pos;
        a.pairs_out = sd->pairs;
        a.tiles_out = (uint32_t *)tiles;
    }
    const dim3 grid((unsigned)((n_tiles_max + 7) / 8 * 8 * a.nyb)), block(W * 64);
    const bool q8 = sh.gate && (sh.gate_fmt == FQ8 || sh.gate_fmt == FQ8T);
    const unsigned pb = !GEMM_PERSIST || tile_m == GEMM_TILE_MIN ? 0u
                        : tile_m == GEMM_TILE_BIG ? persist_blocks() : GEMM_PERSIST_SMALL * persist_blocks();
    a.kt = kt && (long)grid.x <= kt_cap ? kt : nullptr;
    if (pb && H == 2048 && (!sh.gate || sh.S == M)) {
        a.kt = kt && (long)pb <= kt_cap ? kt : nullptr;
#define GP_LAUNCH(GF, ARGS)                                                                                      \
    do {                                                                                                         \
        if (tile_m == GEMM_TILE_BIG) KLAUNCH((k_gemm_gate_up_p<GEMM_TILE_BIG / 16, GF>), dim3(pb), block, 0, s, ARGS); \
        else KLAUNCH((k_gemm_gate_up_p<GEMM_TILE_SMALL / 16, GF>), dim3(pb), block, 0, s, ARGS);          \
    } while (0)
        const int nsh = shared_tiles_in(sh, T, K, E, tile_m);
        if (nsh && q8) { /* Q8_0 shared expert: one walk over the routed tiles, one over the shared */
            GemmArgs ar = a, as = a;
            ar.uwin = -nsh;
            as.uwin = nsh;
            as.kt = nullptr;
            if (tiled) GP_LAUNCH(FQ4KT, ar);
            else GP_LAUNCH(FQ4K, ar);
            if (sh.gate_fmt == FQ8T) GP_LAUNCH(FQ8T, as);
            else GP_LAUNCH(FQ8, as);
        } else if (tiled) {
            GP_LAUNCH(FQ4KT, a);
        } else {
            GP_LAUNCH(FQ4K, a);
        }
#undef GP_LAUNCH
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    /* compile-time stage count for the common hidden size; other shapes
     * take the generic loop */
#define GU_LAUNCH(RF, SF, NS)                                                                    \
    do {                                                                                     \
        if (tile_m == GEMM_TILE_SMALL) KLAUNCH((k_gemm_gate_up<RF, SF, NS, GEMM_TILE_SMALL / 16>), grid, block, 0, s, a); \
        else if (tile_m == GEMM_TILE_MIN) KLAUNCH((k_gemm_gate_up<RF, SF, NS, GEMM_TILE_MIN / 16>), grid, block, 0, s, a); \
        else KLAUNCH((k_gemm_gate_up<RF, SF, NS, GEMM_TILE_BIG / 16>), grid, block, 0, s, a);              \
    } while (0)
    if (tiled) {
        if (sh.gate && sh.gate_fmt == FQ8T) {
            if (H == 2048) GU_LAUNCH(FQ4KT, FQ8T, 16);
            else GU_LAUNCH(FQ4KT, FQ8T, 0);
        } else if (q8) GU_LAUNCH(FQ4KT, FQ8, 0);
        else if (H == 2048) GU_LAUNCH(FQ4KT, FQ4KT, 16);
        else GU_LAUNCH(FQ4KT, FQ4KT, 0);
    } else if (q8) GU_LAUNCH(FQ4K, FQ8, 0);
    else if (H == 2048) GU_LAUNCH(FQ4K, FQ4K, 16);
    else GU_LAUNCH(FQ4K, FQ4K, 0);
#undef GU_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_gemm_down(const ExpertSide &ex, const SharedSide &sh, const _Float16 *act,
                     const _Float16 *act_sh, int zrow, int zrow_sh, int T, int H, int M, int K, int E, int tile_m,
                     const uint32_t *tiles, int n_tiles_max, float *y, float *ysh, hipStream_t s) {
    if (down_shape(ex, sh, H, M, tile_m)) return -2;
    const int W = tile_waves(tile_m);
    const int NB = W * 16 * DN_RPW;
    const int sf = sh.gate ? sh.down_fmt : ex.down_fmt;
    GemmArgs a = {};
    a.wa = ex.down; a.stride_a = ex.down_stride;
    a.sh_a = sh.gate ? sh.down : nullptr;
    a.src = act; a.src_sh = act_sh; a.T = T; a.H = H; a.M = M; a.S = sh.gate ? sh.S : 0; a.K = K; a.E = E;
    a.zrow = zrow; a.zrow_sh = zrow_sh;
    a.tiles = tiles; a.y = y; a.ysh = ysh;
    a.nyb = H / NB;
    const dim3 grid((unsigned)((n_tiles_max + 7) / 8 * 8 * a.nyb)), block(W * 64);
    if (tile_m != GEMM_TILE_SMALL && tile_m != GEMM_TILE_BIG && tile_m != GEMM_TILE_MIN) return -2;
    const unsigned pb = !GEMM_PERSIST || tile_m == GEMM_TILE_MIN ? 0u
                        : tile_m == GEMM_TILE_BIG ? persist_blocks() : GEMM_PERSIST_SMALL_DN * persist_blocks();
    const int nsh = shared_tiles_in(sh, T, K, E, tile_m);
    const bool mixed = nsh && sf != ex.down_fmt;
    if (pb && M == 512 && (!nsh || sh.S == M)) {
#define DP_LAUNCH(F, TB, ARGS)                                                                                        \
    do {                                                                                                              \
        if ((F) == FQ4K) KLAUNCH((k_gemm_down_p<FQ4K, TB>), dim3(pb), block, 0, s, ARGS);                    \
        else if ((F) == FQ4KT) KLAUNCH((k_gemm_down_p<FQ4KT, TB>), dim3(pb), block, 0, s, ARGS);             \
        else if ((F) == FQ6KT) KLAUNCH((k_gemm_down_p<FQ6KT, TB>), dim3(pb), block, 0, s, ARGS);             \
        else if ((F) == FQ8) KLAUNCH((k_gemm_down_p<FQ8, TB>), dim3(pb), block, 0, s, ARGS);                 \
        else if ((F) == FQ8T) KLAUNCH((k_gemm_down_p<FQ8T, TB>), dim3(pb), block, 0, s, ARGS);               \
        else if ((F) == FQ5KT) KLAUNCH((k_gemm_down_p<FQ5KT, TB>), dim3(pb), block, 0, s, ARGS);             \
        else if ((F) == FQ5K) KLAUNCH((k_gemm_down_p<FQ5K, TB>), dim3(pb), block, 0, s, ARGS);               \
        else KLAUNCH((k_gemm_down_p<FQ6K, TB>), dim3(pb), block, 0, s, ARGS);                                \
    } while (0)
#define DP_TILE(F, ARGS)                                                        \
    do {                                                                        \
        if (tile_m == GEMM_TILE_BIG) DP_LAUNCH(F, GEMM_TILE_BIG / 16, ARGS);     \
        else DP_LAUNCH(F, GEMM_TILE_SMALL / 16, ARGS);                           \
    } while (0)
        if (!mixed) {
            DP_TILE(ex.down_fmt, a);
        } else { /* routed and shared down differ in format: one walk each */
            GemmArgs ar = a, as = a;
            ar.uwin = -nsh;
            as.uwin = nsh;
            DP_TILE(ex.down_fmt, ar);
            DP_TILE(sf, as);
        }
#undef DP_TILE
#undef DP_LAUNCH
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    if (ex.down_fmt == FQ8 || ex.down_fmt == FQ8T) return -2; /* persistent kernels only */
    /* generic unit loop (a compile-time stage count spills here) */
#define DN_LAUNCH(EF, SF)                                                                    \
    do {                                                                                     \
        if (tile_m == GEMM_TILE_SMALL) KLAUNCH((k_gemm_down<EF, SF, 0, GEMM_TILE_SMALL / 16>), grid, block, 0, s, a); \
        else if (tile_m == GEMM_TILE_MIN) KLAUNCH((k_gemm_down<EF, SF, 0, GEMM_TILE_MIN / 16>), grid, block, 0, s, a); \
        else KLAUNCH((k_gemm_down<EF, SF, 0, GEMM_TILE_BIG / 16>), grid, block, 0, s, a);              \
    } while (0)
#define DN_TILED(EF)                                \
    do {                                            \
        if (sf == FQ4KT) DN_LAUNCH(EF, FQ4KT);      \
        else if (sf == FQ5KT) DN_LAUNCH(EF, FQ5KT); \
        else if (sf == FQ6KT) DN_LAUNCH(EF, FQ6KT); \
        else DN_LAUNCH(EF, FQ8T);                   \
    } while (0)
    if (ex.down_fmt == FQ4KT) {
        DN_TILED(FQ4KT);
    } else if (ex.down_fmt == FQ5KT) {
        DN_TILED(FQ5KT);
    } else if (ex.down_fmt == FQ6KT) {
        DN_TILED(FQ6KT);
    } else if (ex.down_fmt == FQ4K) {
        if (sf == FQ4K) DN_LAUNCH(FQ4K, FQ4K);
        else if (sf == FQ5K) DN_LAUNCH(FQ4K, FQ5K);
        else if (sf == FQ6K) DN_LAUNCH(FQ4K, FQ6K);
        else DN_LAUNCH(FQ4K, FQ8);
    } else if (ex.down_fmt == FQ5K) {
        if (sf == FQ4K) DN_LAUNCH(FQ5K, FQ4K);
        else if (sf == FQ5K) DN_LAUNCH(FQ5K, FQ5K);
        else if (sf == FQ6K) DN_LAUNCH(FQ5K, FQ6K);
        else DN_LAUNCH(FQ5K, FQ8);
    } else {
        if (sf == FQ4K) DN_LAUNCH(FQ6K, FQ4K);
        else if (sf == FQ5K) DN_LAUNCH(FQ6K, FQ5K);
        else if (sf == FQ6K) DN_LAUNCH(FQ6K, FQ6K);
        else DN_LAUNCH(FQ6K, FQ8);
    }
#undef DN_TILED
#undef DN_LAUNCH
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* ------------------------------------------------------------ repack */
/* Q4_K matrices [R rows][K/256 super-blocks of 144 B] (matrix e at src +
 * e * src_stride) into the tile-major layout of Span<FQ4KT>, densely (matrix
 * e at dst + e * R * row bytes): tile (row block rb, super-block sb) at
 * (rb * nsb + sb) * 2304, whose 16-byte piece o holds row o's header (o <
 * 16) or, for o = 16 + 64 jj + 16 kg + i, bytes 16 + 16 (kg + 4 jj) .. +15
 * of row i's super-block.  A byte permutation: dequantised values are
 * unchanged. */
__global__ __launch_bounds__(144) void k_pack_q4k(const uint8_t *src, uint8_t *dst, int R, int nsb, size_t src_stride) {
    const int tile = blockIdx.x, e = blockIdx.y, rb = tile / nsb, sb = tile - rb * nsb, o = threadIdx.x;
    const size_t rbytes = (size_t)nsb * 144;
    const uint8_t *t0 = src + (size_t)e * src_stride + (size_t)rb * 16 * rbytes + (size_t)sb * 144;
    int row, off;
    if (o < 16) {
        row = o;
        off = 0;
    } else {
        const int qo = o - 16, jj = qo >> 6, ln = qo & 63;
        row = ln & 15;
        off = 16 + 16 * ((ln >> 4) + 4 * jj);
    }
    const u4 v = ld_u4(t0 + (size_t)row * rbytes + off);
    *(u4 *)(dst + (size_t)e * R * rbytes + (size_t)tile * 2304 + (size_t)o * 16) = v;
}

size_t packed_q4k_bytes(int R, int K, int E) { return (size_t)E * R * (K / 256) * 144; }

int launch_pack_q4k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s) {
    if (R % 16 || K % 256 || E < 1 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (src_stride & 15)) return -2;
    const int nsb = K / 256;
    KLAUNCH(k_pack_q4k, dim3((unsigned)(R / 16 * nsb), (unsigned)E), dim3(144), 0, s, src, dst, R, nsb, src_stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Q5_K matrices [R rows][K/256 super-blocks of 176 B] into the tile-major
 * layout of Span<FQ5KT>: tile (rb, sb) at (rb * nsb + sb) * 2816, whose
 * 16-byte piece o holds row o's header (o < 16), for o = 16 + 64 jj + 16 kg +
 * i bytes 48 + 16 (kg + 4 jj) .. +15 of row i, and for o = 144 + 16 g + i
 * bytes 16 + 16 g .. +15 (qh) of row i.  A byte permutation. */
__global__ __launch_bounds__(176) void k_pack_q5k(const uint8_t *src, uint8_t *dst, int R, int nsb, size_t src_stride) {
    const int tile = blockIdx.x, e = blockIdx.y, rb = tile / nsb, sb = tile - rb * nsb, o = threadIdx.x;
    const size_t rbytes = (size_t)nsb * 176;
    const uint8_t *t0 = src + (size_t)e * src_stride + (size_t)rb * 16 * rbytes + (size_t)sb * 176;
    int row, off;
    if (o < 16) {
        row = o;
        off = 0;
    } else if (o < 144) {
        const int qo = o - 16, jj = qo >> 6, ln = qo & 63;
        row = ln & 15;
        off = 48 + 16 * ((ln >> 4) + 4 * jj);
    } else {
        const int x = o - 144;
        row = x & 15;
        off = 16 + 16 * (x >> 4);
    }
    const u4 v = ld_u4(t0 + (size_t)row * rbytes + off);
    *(u4 *)(dst + (size_t)e * R * rbytes + (size_t)tile * 2816 + (size_t)o * 16) = v;
}

size_t packed_q5k_bytes(int R, int K, int E) { return (size_t)E * R * (K / 256) * 176; }

int launch_pack_q5k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s) {
    if (R % 16 || K % 256 || E < 1 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15) || (src_stride & 15)) return -2;
    const int nsb = K / 256;
    KLAUNCH(k_pack_q5k, dim3((unsigned)(R / 16 * nsb), (unsigned)E), dim3(176), 0, s, src, dst, R, nsb, src_stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Q6_K matrices [R rows][K/256 super-blocks of 210 B] into the tile-major
 * layout of Span<FQ6KT> (a byte permutation; source blocks are only 2-byte
 * aligned, so the copy moves 16-bit words).  Output byte ob of tile (rb, sb):
 *   ob < 2048: half h = ob / 1024, lane (kg, i): row i, byte h 64 + 32 (kg & 1) + 16 (kg >> 1) + ob % 16
 *   ob < 3072: half h, group g = kg >> 1:  row i, byte 128 + h 32 + 16 g + ob % 16
 *   ob < 3328: row i = (ob - 3072) / 16,     byte 192 + ob % 16
 *   else:      row i = (ob - 3328) / 2,      byte 208 + ob % 2 */
__global__ __launch_bounds__(256) void k_pack_q6k(const uint8_t *src, uint8_t *dst, int R, int nsb, size_t src_stride) {
    const int tile = blockIdx.x, e = blockIdx.y, rb = tile / nsb, sb = tile - rb * nsb;
    const size_t rbytes = (size_t)nsb * 210;
    const uint8_t *t0 = src + (size_t)e * src_stride + (size_t)rb * 16 * rbytes + (size_t)sb * 210;
    uint8_t *d0 = dst + (size_t)e * R * rbytes + (size_t)tile * 3360;
    for (int w = threadIdx.x; w < 1680; w += 256) {
        const int ob = 2 * w;
        int row, byte;
        if (ob < 2048) {
            const int h = ob >> 10, ln = (ob & 1023) >> 4, kg = ln >> 4;
            row = ln & 15;
            byte = h * 64 + 32 * (kg & 1) + 16 * (kg >> 1) + (ob & 15);
        } else if (ob < 3072) {
            const int x = ob - 2048, h = x >> 9, idx = (x & 511) >> 4;
            row = idx & 15;
            byte = 128 + h * 32 + 16 * (idx >> 4) + (x & 15);
        } else if (ob < 3328) {
            const int x = ob - 3072;
            row = x >> 4;
            byte = 192 + (x & 15);
        } else {
            const int x = ob - 3328;
            row = x >> 1;
            byte = 208 + (x & 1);
        }
        *(uint16_t *)(d0 + ob) = *(const uint16_t *)(t0 + (size_t)row * rbytes + byte);
    }
}

size_t packed_q6k_bytes(int R, int K, int E) { return (size_t)E * R * (K / 256) * 210; }

/* Q8_0 matrices [R rows][K/32 blocks of 34 B] into the tile-major layout of
 * Span<FQ8T> (a byte permutation, moved in 16-bit words: source blocks are
 * 2-byte aligned).  Output byte ob of tile (rb, stage j):
 *   ob < 2048: lane ln = ob / 32 (kg = ln / 16, row i = ln % 16), step s = ob % 32 / 8:
 *              byte 2 + 8 kg + ob % 8 of row i's block 4j + s
 *   else:      row i = (ob - 2048) / 8, block 4j + (ob % 8) / 2: byte ob % 2 (the scale) */
__global__ __launch_bounds__(256) void k_pack_q8(const uint8_t *src, uint8_t *dst, int R, int nst, size_t src_stride) {
    const int tile = blockIdx.x, e = blockIdx.y, rb = tile / nst, j = tile - rb * nst;
    const size_t rbytes = (size_t)nst * 4 * 34;
    const uint8_t *t0 = src + (size_t)e * src_stride + (size_t)rb * 16 * rbytes + (size_t)j * 4 * 34;
    uint8_t *d0 = dst + (size_t)e * R * rbytes + (size_t)tile * 2176;
    for (int w = threadIdx.x; w < 1088; w += 256) {
        const int ob = 2 * w;
        int row, byte;
        if (ob < 2048) {
            const int ln = ob >> 5, st = (ob & 31) >> 3;
            row = ln & 15;
            byte = st * 34 + 2 + 8 * (ln >> 4) + (ob & 7);
        } else {
            const int x = ob - 2048;
            row = x >> 3;
            byte = ((x & 7) >> 1) * 34;
        }
        *(uint16_t *)(d0 + ob) = *(const uint16_t *)(t0 + (size_t)row * rbytes + byte);
    }
}

size_t packed_q8_bytes(int R, int K, int E) { return (size_t)E * R * (K / 32) * 34; }

int launch_pack_q8(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s) {
    if (R % 16 || K % 128 || E < 1 || ((uintptr_t)src & 1) || ((uintptr_t)dst & 15) || (src_stride & 1)) return -2;
    const int nst = K / 128;
    KLAUNCH(k_pack_q8, dim3((unsigned)(R / 16 * nst), (unsigned)E), dim3(256), 0, s, src, dst, R, nst, src_stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}


int launch_pack_q6k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s) {
    if (R % 16 || K % 256 || E < 1 || ((uintptr_t)src & 1) || ((uintptr_t)dst & 15) || (src_stride & 1)) return -2;
    const int nsb = K / 256;
    KLAUNCH(k_pack_q6k, dim3((unsigned)(R / 16 * nsb), (unsigned)E), dim3(256), 0, s, src, dst, R, nsb, src_stride);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
