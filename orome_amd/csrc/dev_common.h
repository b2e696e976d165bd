/*
 * dev_common.h -- gfx950 device helpers shared by the MoE kernels:
 * wave64 reductions, fp16 packing, and the Q4_K / Q6_K / Q8_0 block
 * decoders used by the GEMV (decode) and MFMA (prefill) kernels.
 *
 * Quant layouts (byte offsets inside one super-block / block):
 *   Q4_K 144 B / 256 w: d f16 @0, dmin f16 @2, 12 packed 6-bit scale/min
 *        bytes @4, 128 nibble bytes @16; weight (g*64 + l) is the low nibble
 *        and (g*64 + 32 + l) the high nibble of qs[g*32 + l].  Scale/min
 *        unpack follows inference/src/format.m:41-64 (reference layout).
 *   Q6_K 210 B / 256 w: ql @0 (128), qh @128 (64), int8 scales @192 (16),
 *        d f16 @208; inference/src/format.m:144-174.
 *   Q8_0 34 B / 32 w: d f16 @0, 32 int8 @2; inference/src/format.m:66-79.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

#define DEV static __device__ __forceinline__
#define MDEV __device__ __forceinline__ /* member functions */
/* Optional per-block start/end stamps of a kernel launch (s_memrealtime,
 * 100 MHz) into kt[2 b], kt[2 b + 1] for block b: the launch's duration is
 * max(end) - min(start), the quantity a kernel trace reports.  kt NULL:
 * nothing is written. */
#define KT_BEGIN(kt)                                                                   \
    do {                                                                               \
        if ((kt) && threadIdx.x == 0) (kt)[2 * blockIdx.x] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define KT_END(kt)                                                                     \
    do {                                                                               \
        if (kt) {                                                                      \
            __syncthreads();                                                           \
            if (threadIdx.x == 0) (kt)[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime(); \
        }                                                                              \
    } while (0)

DEV h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
DEV uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

DEV float f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
}

/* DPP lane exchange (compile-time control word). */
template <int CTRL>
DEV float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
DEV uint32_t dppu(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
#define DPP_XOR1 0xB1        /* quad_perm [1,0,3,2] */
#define DPP_XOR2 0x4E        /* quad_perm [2,3,0,1] */
#define DPP_HALF_MIRROR 0x141 /* lane i <-> 7-i within each 8 */
#define DPP_MIRROR 0x140     /* lane i <-> 15-i within each 16 */

/* Sum over each row of 16 lanes; every lane gets its row's total.  Lane 0 of
 * the row holds ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)) + ... exactly as an xor
 * butterfly 1,2,4,8 would leave it (adds are commutative, so the mirrored
 * partner yields the same bits). */
DEV float row_sum16(float v) {
    v = v + dppf<DPP_XOR1>(v);
    v = v + dppf<DPP_XOR2>(v);
    v = v + dppf<DPP_HALF_MIRROR>(v);
    v = v + dppf<DPP_MIRROR>(v);
    return v;
}

/* canonical per-lane layouts cover H <= 256 CANON_NI (f4 per lane per 256) */
#define CANON_NI 16
/* Canonical wave64 sum: the xor butterfly 1,2,4,8,16,32 as seen by lane 0,
 * i.e. rows r0..r3 of 16 lanes reduced as above, then (r0+r1)+(r2+r3).
 * Every lane returns the same value.  This order is part of the router/norm
 * bit-exact contract with the C oracle. */
DEV float wave_sum_canon(float v) {
    v = row_sum16(v);
    int b = __builtin_bit_cast(int, v);
    float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

/* Wave64 sum in no particular order (every lane gets the total). */
DEV float wave_sum_fast(float v) {
    v = row_sum16(v);
    int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

/* Sum over aligned groups of 16 lanes (a DPP row). */
template <int WIDTH>
DEV float group_sum(float v) {
    static_assert(WIDTH == 16, "row sums only");
    return row_sum16(v);
}

/* SiLU with the hardware reciprocal (1 ulp) instead of the IEEE divide
 * sequence: the result is rounded to fp16 right after, and g -> -inf still
 * gives -0 (rcp(inf) = 0) */
DEV float silu_f(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
DEV float sigmoid_f(float s) { return 1.0f / (1.0f + expf(-s)); }
/* act = half(silu(g) * u) as the reference stages it: the product rounded to
 * fp32, then to fp16 (the empty asm keeps the compiler from folding the
 * product into a mixed-precision FMA that rounds once, straight to fp16,
 * which differs in rare cases and would differ between kernels) */
DEV _Float16 glu_f16(float g, float u) {
    float v = silu_f(g) * u;
    asm volatile("" : "+v"(v));
    return (_Float16)v;
}

/* --------------------------------------------------------------- Q4_K */

/* 6-bit scale/min byte i (0..11) of the packed region, given its three dwords */
DEV uint32_t q4k_sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> ((i & 3) * 8)) & 0xFFu;
}

/* Scales/mins of sub-blocks 2g and 2g+1 (inference/src/format.m:41-64),
 * as integers. hdr = first 16 bytes of the super-block. */
DEV void q4k_scale_min(u4 hdr, int g, uint32_t &sl, uint32_t &sh, uint32_t &ml, uint32_t &mh) {
    uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
    if (g < 2) {
        int b = 2 * g;
        sl = q4k_sbyte(s0, s1, s2, b) & 63u;
        sh = q4k_sbyte(s0, s1, s2, b + 1) & 63u;
        ml = q4k_sbyte(s0, s1, s2, b + 4) & 63u;
        mh = q4k_sbyte(s0, s1, s2, b + 5) & 63u;
    } else {
        int b = 2 * (g - 2);
        uint32_t sp = q4k_sbyte(s0, s1, s2, 8 + g - 2), mp = q4k_sbyte(s0, s1, s2, 10 + g - 2);
        sl = (sp & 0xFu) | ((q4k_sbyte(s0, s1, s2, b) >> 6) << 4);
        sh = (sp >> 4) | ((q4k_sbyte(s0, s1, s2, b + 1) >> 6) << 4);
        ml = (mp & 0xFu) | ((q4k_sbyte(s0, s1, s2, b + 4) >> 6) << 4);
        mh = (mp >> 4) | ((q4k_sbyte(s0, s1, s2, b + 5) >> 6) << 4);
    }
}

/* Per-chunk affine terms for a Q4_K 16-byte quant chunk in group g:
 * weight = a * q - b (exact products; one rounding at the subtract). */
struct Q4Affine {
    float a_lo, a_hi, b_lo, b_hi;
};
DEV Q4Affine q4k_affine(u4 hdr, int g) {
    uint32_t sl, sh, ml, mh;
    q4k_scale_min(hdr, g, sl, sh, ml, mh);
    float d = f16_bits_to_f32(hdr.x), dm = f16_bits_to_f32(hdr.x >> 16);
    Q4Affine r;
    r.a_lo = d * (float)sl;
    r.a_hi = d * (float)sh;
    r.b_lo = dm * (float)ml;
    r.b_hi = dm * (float)mh;
    return r;
}

/* Exact fp16 pairs of 4-bit quants: for a dword of 4 quant bytes (positions
 * l..l+3), lo01 = (q_lo[l], q_lo[l+1]), lo23 = (q_lo[l+2], q_lo[l+3]) and
 * the same for the high nibbles.  0x64XX as fp16 is 1024 + XX. */
DEV void q4_nibbles_h2(uint32_t w, h2 &lo01, h2 &lo23, h2 &hi01, h2 &hi23) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    lo01 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x05010400u)) - bias;
    lo23 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x05030402u)) - bias;
    hi01 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x05010400u)) - bias;
    hi23 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x05030402u)) - bias;
}

/* Biased exact fp16 images of the eight 4-bit quants of a dword (bytes =
 * positions l..l+3), in the pair order (l, l+2), (l+1, l+3):
 * lo = 1024 + q_lo, hi = 1024 + 16 q_hi (the nibbles OR-ed under the 0x64
 * exponent byte; five instructions).  With S = sum of (image * x) over a
 * sub-block and X = sum of x, sum q_lo x = S_lo - 1024 X and
 * sum q_hi x = (S_hi - 1024 X) / 16. */
DEV void q4_bias_h2(uint32_t w, h2 &l02, h2 &l13, h2 &h02, h2 &h13) {
    const uint32_t p13 = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);
    l02 = as_h2((w & 0x000F000Fu) | 0x64006400u);
    l13 = as_h2(p13 & 0xFF0FFF0Fu);
    h02 = as_h2((w & 0x00F000F0u) | 0x64006400u);
    h13 = as_h2(p13 & 0xFFF0FFF0u);
}

/* --------------------------------------------------------------- Q5_K */

/* Five-bit quants of a Q5_K dword as biased exact fp16 pairs: w = 4 ql bytes
 * (positions l..l+3 of group g), h = the 4 qh bytes of the same positions;
 * low value = (w & 15) | bit 2g of h << 4, high value = (w >> 4) | bit 2g+1
 * of h << 4 (inference/src/format.m:110-141).  lo01 = (lo[l], lo[l+1]) + 1024
 * etc.: the values OR-ed under the 0x64 exponent byte. */
DEV void q5_bias_h2(uint32_t w, uint32_t h, int g, h2 &lo01, h2 &lo23, h2 &hi01, h2 &hi23) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * g)) & 0x01010101u) << 4);
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * g + 1)) & 0x01010101u) << 4);
    lo01 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x05010400u));
    lo23 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x05030402u));
    hi01 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x05010400u));
    hi23 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x05030402u));
}

/* --------------------------------------------------------------- Q6_K */

/* Six-bit quants minus 32 as exact fp16 pairs: inputs are 4 ql bytes
 * (nibble select by `shift` 0/4) and 4 qh bytes (2-bit field at qshift). */
DEV void q6_h2(uint32_t ql, uint32_t qh, int shift, int qshift, h2 &p01, h2 &p23) {
    uint32_t v = ((ql >> shift) & 0x0F0F0F0Fu) | (((qh >> qshift) & 0x03030303u) << 4);
    const h2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};  /* 1024 + 32 */
    p01 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x05010400u)) - bias;
    p23 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x05030402u)) - bias;
}

/* Signed int8 quants as exact fp16 pairs (flip the sign bit, bias 1152). */
DEV void q8_h2(uint32_t w, h2 &p01, h2 &p23) {
    uint32_t v = w ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    p01 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x05010400u)) - bias;
    p23 = as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x05030402u)) - bias;
}

/* Loads that only need 2-byte alignment (Q6_K and Q8_0 blocks are 210 and
 * 34 bytes long): aligned dword loads realigned with v_alignbyte.  They read
 * up to 4 bytes past the last byte asked for; uploads carry tail padding. */
typedef const __attribute__((address_space(1))) uint32_t *gp32;
DEV gp32 gptr32(const uint8_t *p) { return (gp32)(uintptr_t)p; }
DEV uint32_t ld_u32_a2(const uint8_t *p) {
    uintptr_t a = (uintptr_t)p;
    gp32 q = gptr32((const uint8_t *)(a & ~(uintptr_t)3));
    uint32_t s = (uint32_t)(a & 3);
    return __builtin_amdgcn_alignbyte(q[1], q[0], s);
}
DEV u2 ld_u32x2_a2(const uint8_t *p) {
    uintptr_t a = (uintptr_t)p;
    gp32 q = gptr32((const uint8_t *)(a & ~(uintptr_t)3));
    uint32_t s = (uint32_t)(a & 3);
    uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    return u2{__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s)};
}
DEV u4 ld_u32x4_a2(const uint8_t *p) {
    uintptr_t a = (uintptr_t)p;
    gp32 q = gptr32((const uint8_t *)(a & ~(uintptr_t)3));
    uint32_t s = (uint32_t)(a & 3);
    uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
    return u4{__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s),
              __builtin_amdgcn_alignbyte(w3, w2, s), __builtin_amdgcn_alignbyte(w4, w3, s)};
}
DEV u4 ld_u4(const uint8_t *p) {
    typedef const __attribute__((address_space(1))) u4 *gp4;
    return *(gp4)(uintptr_t)p;
}
/* Streaming load (`nt`): for expert weights that a forward reads once, so
 * that they do not push the activations and expert outputs the next kernels
 * read back out of the last-level cache */
DEV u4 ld_u4_nt(const uint8_t *p) {
    typedef __attribute__((address_space(1))) u4 *gp4;
    return __builtin_nontemporal_load((gp4)(uintptr_t)p);
}

/* Cross-block hand-off inside one kernel: data stored and loaded as
 * agent-scope atomics, published by an agent-scope release (the counter
 * increment that follows a workgroup barrier) and read after the matching
 * agent-scope acquire. */
DEV void st_coh(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV float ld_coh(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

/* Workgroup barrier ordering LDS only.  __syncthreads also makes the block's
 * global stores visible to the block, so it first waits for every store in
 * flight (a full memory round trip); blocks that exchange data through LDS
 * alone and whose global stores are read only by later kernels use this. */
DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* Inclusive scan of two words over the block (up to 16 waves), with both
 * totals: a DPP scan per wave, then one barrier for the wave sums (wsum:
 * LDS, 32 words).  Every thread of the block calls it. */
DEV void scan2_block(uint32_t &x, uint32_t &y, uint32_t *wsum, uint32_t &tx, uint32_t &ty) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    /* wave inclusive scan with DPP: shifts by 1, 2, 4, 8 inside each row of
     * 16 lanes (lanes shifted in from outside the row add 0), then lane 15
     * of each row into the next row, lane 31 into rows 2 and 3 */
#define SCAN_STEP(CTRL, ROWS)                                                            \
    do {                                                                                 \
        x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xF, false);   \
        y += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)y, CTRL, ROWS, 0xF, false);   \
    } while (0)
    SCAN_STEP(0x111, 0xF);
    SCAN_STEP(0x112, 0xF);
    SCAN_STEP(0x114, 0xF);
    SCAN_STEP(0x118, 0xF);
    SCAN_STEP(0x142, 0xA);
    SCAN_STEP(0x143, 0xC);
#undef SCAN_STEP
    const int nw = (int)(blockDim.x >> 6);
    if (lane == 63) {
        wsum[wv] = x;
        wsum[16 + wv] = y;
    }
    lds_barrier();
    tx = 0;
    ty = 0;
    for (int w = 0; w < nw; w++) {
        const uint32_t sx = wsum[w], sy = wsum[16 + w];
        if (w < wv) {
            x += sx;
            y += sy;
        }
        tx += sx;
        ty += sy;
    }
}

/* ------------------------------------------------------------ dots */
DEV float dot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
