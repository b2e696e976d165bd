/*
 * moe_gemm.hip -- prefill-path grouped expert GEMMs on the matrix cores.
 *
 * Work list: the dispatch kernel emits tiles (expert, first row, rows <= 32)
 * over the expert-sorted pair list; the shared expert is expert E over the
 * token order.  One block computes one tile x 64 output rows:
 *   gate/up  D[row][token] = W_{gate,up}[e][row] . x16[token]      (K = H)
 *   down     y[pos][row]   = W_down[e][row]    . act[pos]         (K = M)
 * with v_mfma_f32_16x16x32_f16 (A = 16 weight rows x 32 k, B = 32 k x 16
 * tokens, fp32 accumulate).  Each wave owns 16 weight rows (both gate and up
 * rows for the first GEMM) for all 32 tokens of the tile.
 *
 * Weights are dequantised straight into the A fragments: the exact fp32
 * value of format_decode_row_f32 (inference/src/format.m:81-174, products
 * exact), rounded once to fp16 (RNE).  A lane's 8 k-values per MFMA are two
 * runs of 4 consecutive k (k_a.., k_b..) chosen so that they come from one
 * quant dword; the B fragment reads the same k positions of the token rows
 * staged in LDS, so the contraction is the plain dot product.
 * Activations are fp16 as the reference stages them (half(x), half(act)).
 */
#include "dev_common.h"
#include "kernels.h"

enum { FQ4K = 0, FQ6K = 2, FQ8 = 3 };

typedef float f4v __attribute__((ext_vector_type(4)));

#define TM GEMM_TILE_M   /* tokens per tile (32) */
#define NB 64            /* weight rows per block */
#define KC 256           /* k per super-block step */
#define XS_LD (KC + 8)   /* padded LDS row (halves) */

DEV size_t gemm_row_bytes(int fmt, int n) {
    return fmt == FQ4K ? (size_t)(n / 256) * 144 : fmt == FQ6K ? (size_t)(n / 256) * 210 : (size_t)(n / 32) * 34;
}

/* Raw bytes of one 256-weight span of one row, as held by lane kg (0..3). */
struct SpanRaw {
    u4 a, b, c;      /* Q4_K: hdr, piece kg, piece kg+4 | Q6_K: ql 32B (a,b), qh 16B half (c) */
    u4 d;            /* Q6_K: other 16B of qh; scales in e */
    u4 e;            /* Q6_K: 16 scale bytes | Q8_0: d of the 8 blocks (packed) */
    uint32_t f;      /* Q6_K: d */
};

template <int FMT>
DEV SpanRaw span_load(const uint8_t *row, int sb, int kg) {
    SpanRaw r;
    if (FMT == FQ4K) {
        const uint8_t *p = row + (size_t)sb * 144;
        r.a = ld_u4(p);
        r.b = ld_u4(p + 16 + 16 * kg);
        r.c = ld_u4(p + 16 + 16 * (kg + 4));
    } else if (FMT == FQ6K) {
        const uint8_t *p = row + (size_t)sb * 210;
        const int h = kg >> 1;
        r.a = ld_u32x4_a2(p + 32 * kg);
        r.b = ld_u32x4_a2(p + 32 * kg + 16);
        r.c = ld_u32x4_a2(p + 128 + 32 * h);
        r.d = ld_u32x4_a2(p + 128 + 32 * h + 16);
        r.e = ld_u32x4_a2(p + 192);
        r.f = ld_u32_a2(p + 208);
    } else {
        /* Q8_0: 8 blocks of 34 B; lane kg takes quant bytes 8kg..8kg+7 of each */
        const uint8_t *p = row + (size_t)sb * 8 * 34;
        uint32_t q[16];
        uint32_t dd[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            u2 v = ld_u32x2_a2(p + s * 34 + 2 + 8 * kg);
            q[2 * s] = v.x;
            q[2 * s + 1] = v.y;
            dd[s] = ld_u32_a2(p + s * 34) & 0xFFFFu;
        }
        r.a = u4{q[0], q[1], q[2], q[3]};
        r.b = u4{q[4], q[5], q[6], q[7]};
        r.c = u4{q[8], q[9], q[10], q[11]};
        r.d = u4{q[12], q[13], q[14], q[15]};
        r.e = u4{dd[0] | (dd[1] << 16), dd[2] | (dd[3] << 16), dd[4] | (dd[5] << 16), dd[6] | (dd[7] << 16)};
    }
    return r;
}

DEV uint32_t u4_at(u4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

DEV h2 pk_f16(float a, float b) { return h2{(_Float16)a, (_Float16)b}; }

/* Step s (0..7) of a span: the lane's 8 weights as fp16 and the two k runs
 * (offsets inside the 256-wide span). */
template <int FMT>
DEV h8 span_step(const SpanRaw &r, int s, int kg, int &ka, int &kb) {
    float w[8];
    if (FMT == FQ4K) {
        const int p = kg + 4 * (s >> 2);
        const int g = p >> 1, l0 = (p & 1) * 16 + 4 * (s & 3);
        ka = g * 64 + l0;
        kb = ka + 32;
        Q4Affine af = q4k_affine(r.a, g);
        uint32_t q = u4_at((s >> 2) ? r.c : r.b, s & 3);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t byte = (q >> (8 * i)) & 0xFFu;
            w[i] = af.a_lo * (float)(byte & 0xFu) - af.b_lo;
            w[4 + i] = af.a_hi * (float)(byte >> 4) - af.b_hi;
        }
    } else if (FMT == FQ6K) {
        const int h = kg >> 1, odd = kg & 1, l = 4 * s;
        ka = h * 128 + (odd ? 32 : 0) + l;
        kb = ka + 64;
        uint32_t ql = u4_at(s < 4 ? r.a : r.b, s & 3);
        uint32_t qh = u4_at(l < 16 ? r.c : r.d, (l >> 2) & 3);
        const int sh_lo = odd ? 2 : 0, sh_hi = odd ? 6 : 4;
        const int is = l >> 4;
        const int grp_lo = odd ? 1 : 0, grp_hi = odd ? 3 : 2;
        const int sci_lo = h * 8 + is + 2 * grp_lo, sci_hi = h * 8 + is + 2 * grp_hi;
        float d = f16_bits_to_f32(r.f);
        float sc_lo = (float)(int8_t)((u4_at(r.e, sci_lo >> 2) >> (8 * (sci_lo & 3))) & 0xFF);
        float sc_hi = (float)(int8_t)((u4_at(r.e, sci_hi >> 2) >> (8 * (sci_hi & 3))) & 0xFF);
        float a_lo = d * sc_lo, a_hi = d * sc_hi;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t b = (ql >> (8 * i)) & 0xFFu, hb = (qh >> (8 * i)) & 0xFFu;
            int q1 = (int)((b & 0xFu) | (((hb >> sh_lo) & 3u) << 4)) - 32;
            int q2 = (int)((b >> 4) | (((hb >> sh_hi) & 3u) << 4)) - 32;
            w[i] = a_lo * (float)q1;
            w[4 + i] = a_hi * (float)q2;
        }
    } else {
        ka = s * 32 + 8 * kg;
        kb = ka + 4;
        uint32_t q0 = u4_at(s < 2 ? r.a : s < 4 ? r.b : s < 6 ? r.c : r.d, (2 * s) & 3);
        uint32_t q1 = u4_at(s < 2 ? r.a : s < 4 ? r.b : s < 6 ? r.c : r.d, (2 * s + 1) & 3);
        float d = f16_bits_to_f32(u4_at(r.e, s >> 1) >> (16 * (s & 1)));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w[i] = d * (float)(int8_t)((q0 >> (8 * i)) & 0xFF);
            w[4 + i] = d * (float)(int8_t)((q1 >> (8 * i)) & 0xFF);
        }
    }
    h8 o;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = (_Float16)w[i];
    return o;
}

DEV h8 lds_b_frag(const _Float16 *xs, int tok, int ka, int kb) {
    const _Float16 *p = xs + tok * XS_LD;
    h4 a = *(const h4 *)(p + ka);
    h4 b = *(const h4 *)(p + kb);
    return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

DEV f4v mfma(h8 a, h8 b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

/* stage rows (TM tokens) x KC halves of the B operand into LDS */
DEV void stage_tile(_Float16 *xs, const _Float16 *src, const int *rowoff, int ld, int k0) {
    /* 256 threads, TM*KC/8 = 1024 16-byte vectors */
    for (int v = threadIdx.x; v < TM * KC / 8; v += 256) {
        const int t = v / (KC / 8), c = (v % (KC / 8)) * 8;
        u4 val = u4{0, 0, 0, 0};
        if (rowoff[t] >= 0) val = ld_u4((const uint8_t *)(src + (size_t)rowoff[t] * ld + k0 + c));
        *(u4 *)(xs + t * XS_LD + c) = val;
    }
}

struct GemmArgs {
    const uint8_t *wa, *wb;   /* gate/up (wb NULL for down) of expert 0 */
    size_t stride_a, stride_b;
    int fmt;
    const uint8_t *sh_a, *sh_b;
    int sh_fmt;
    const _Float16 *src;      /* x16 [T][H] (gate/up) or act [pairs][M] (down) */
    const _Float16 *src_sh;   /* down: act_sh [T][S] */
    int T, H, M, S, K, E;
    const uint32_t *tiles, *pairs;
    _Float16 *act, *act_sh;   /* gate/up outputs */
    float *y, *ysh;           /* down outputs */
};

/* ---------------------------------------------------------- gate/up */
template <int FMT>
DEV void gu_tile(const GemmArgs &a, const uint8_t *wg, const uint8_t *wu, int nrows_out, int in_dim,
                 const int *rowoff, _Float16 *out, int out_ld, int first, int rows, _Float16 *xs) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kg = lane >> 4, i = lane & 15;
    const int r0 = blockIdx.y * NB + wv * 16;
    const size_t rb = gemm_row_bytes(FMT, in_dim);
    const uint8_t *rg = wg + (size_t)(r0 + i) * rb, *ru = wu + (size_t)(r0 + i) * rb;
    f4v cg[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}}, cu[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    const int nsb = in_dim / 256;
    SpanRaw ng = span_load<FMT>(rg, 0, kg), nu = span_load<FMT>(ru, 0, kg);
    for (int sb = 0; sb < nsb; sb++) {
        SpanRaw g = ng, u = nu;
        __syncthreads();
        stage_tile(xs, a.src, rowoff, a.H, sb * KC);
        if (sb + 1 < nsb) {
            ng = span_load<FMT>(rg, sb + 1, kg);
            nu = span_load<FMT>(ru, sb + 1, kg);
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 8; s++) {
            int ka, kb;
            h8 ag = span_step<FMT>(g, s, kg, ka, kb);
            h8 au = span_step<FMT>(u, s, kg, ka, kb);
#pragma unroll
            for (int tb = 0; tb < 2; tb++) {
                h8 b = lds_b_frag(xs, tb * 16 + i, ka, kb);
                cg[tb] = mfma(ag, b, cg[tb]);
                cu[tb] = mfma(au, b, cu[tb]);
            }
        }
    }
    (void)nrows_out;
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
        const int tok = tb * 16 + i;
        if (tok >= rows) continue;
        h4 v;
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = (_Float16)(silu_f(cg[tb][q]) * cu[tb][q]);
        *(h4 *)(out + (size_t)(first + tok) * out_ld + r0 + 4 * kg) = v;
    }
}

__global__ __launch_bounds__(256) void k_gemm_gate_up(GemmArgs a) {
    __shared__ _Float16 xs[TM * XS_LD];
    __shared__ int rowoff[TM];
    const uint32_t nt = a.tiles[0];
    if (blockIdx.x >= nt) return;
    const uint32_t e = a.tiles[1 + 3 * blockIdx.x], first = a.tiles[2 + 3 * blockIdx.x],
                   rows = a.tiles[3 + 3 * blockIdx.x];
    const bool sh = e == (uint32_t)a.E;
    const int nout = sh ? a.S : a.M;
    if (blockIdx.y * NB >= (unsigned)nout) return;
    if (threadIdx.x < TM) {
        int t = -1;
        if (threadIdx.x < rows)
            t = sh ? (int)(first + threadIdx.x) : (int)(a.pairs[first + threadIdx.x] / (uint32_t)a.K);
        rowoff[threadIdx.x] = t;
    }
    if (sh) {
        if (a.sh_fmt == FQ8) gu_tile<FQ8>(a, a.sh_a, a.sh_b, a.S, a.H, rowoff, a.act_sh, a.S, first, rows, xs);
        else gu_tile<FQ4K>(a, a.sh_a, a.sh_b, a.S, a.H, rowoff, a.act_sh, a.S, first, rows, xs);
    } else {
        gu_tile<FQ4K>(a, a.wa + (size_t)e * a.stride_a, a.wb + (size_t)e * a.stride_b, a.M, a.H, rowoff,
                      a.act, a.M, first, rows, xs);
    }
}

/* ------------------------------------------------------------- down */
template <int FMT>
DEV void down_tile(const uint8_t *w, int in_dim, const _Float16 *src, int ld, const int *rowoff,
                   float *out, int out_ld, int first, int rows, _Float16 *xs) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kg = lane >> 4, i = lane & 15;
    const int r0 = blockIdx.y * NB + wv * 16;
    const size_t rb = gemm_row_bytes(FMT, in_dim);
    const uint8_t *rw = w + (size_t)(r0 + i) * rb;
    f4v c[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    const int nsb = in_dim / 256;
    SpanRaw nx = span_load<FMT>(rw, 0, kg);
    for (int sb = 0; sb < nsb; sb++) {
        SpanRaw r = nx;
        __syncthreads();
        stage_tile(xs, src, rowoff, ld, sb * KC);
        if (sb + 1 < nsb) nx = span_load<FMT>(rw, sb + 1, kg);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 8; s++) {
            int ka, kb;
            h8 aw = span_step<FMT>(r, s, kg, ka, kb);
#pragma unroll
            for (int tb = 0; tb < 2; tb++) c[tb] = mfma(aw, lds_b_frag(xs, tb * 16 + i, ka, kb), c[tb]);
        }
    }
#pragma unroll
    for (int tb = 0; tb < 2; tb++) {
        const int tok = tb * 16 + i;
        if (tok >= rows) continue;
        *(f4v *)(out + (size_t)(first + tok) * out_ld + r0 + 4 * kg) = c[tb];
    }
}

__global__ __launch_bounds__(256) void k_gemm_down(GemmArgs a) {
    __shared__ _Float16 xs[TM * XS_LD];
    __shared__ int rowoff[TM];
    const uint32_t nt = a.tiles[0];
    if (blockIdx.x >= nt) return;
    const uint32_t e = a.tiles[1 + 3 * blockIdx.x], first = a.tiles[2 + 3 * blockIdx.x],
                   rows = a.tiles[3 + 3 * blockIdx.x];
    const bool sh = e == (uint32_t)a.E;
    if (threadIdx.x < TM) rowoff[threadIdx.x] = threadIdx.x < rows ? (int)(first + threadIdx.x) : -1;
    if (sh) {
        if (a.sh_fmt == FQ8) down_tile<FQ8>(a.sh_a, a.S, a.src_sh, a.S, rowoff, a.ysh, a.H, first, rows, xs);
        else if (a.sh_fmt == FQ6K) down_tile<FQ6K>(a.sh_a, a.S, a.src_sh, a.S, rowoff, a.ysh, a.H, first, rows, xs);
        else down_tile<FQ4K>(a.sh_a, a.S, a.src_sh, a.S, rowoff, a.ysh, a.H, first, rows, xs);
    } else {
        const uint8_t *w = a.wa + (size_t)e * a.stride_a;
        if (a.fmt == FQ6K) down_tile<FQ6K>(w, a.M, a.src, a.M, rowoff, a.y, a.H, first, rows, xs);
        else down_tile<FQ4K>(w, a.M, a.src, a.M, rowoff, a.y, a.H, first, rows, xs);
    }
}

/* ------------------------------------------------------------ launch */
int launch_gemm_gate_up(const ExpertSide &ex, const SharedSide &sh, const _Float16 *x16, int T, int H,
                        int M, int K, int E, const uint32_t *tiles, int n_tiles_max,
                        const uint32_t *pairs, _Float16 *act, _Float16 *act_sh, hipStream_t s) {
    if (H % 256 || M % NB || (sh.gate && sh.S % NB) || ex.gate_fmt != FQ4K) return -2;
    if (sh.gate && sh.gate_fmt != FQ4K && sh.gate_fmt != FQ8) return -2;
    GemmArgs a = {};
    a.wa = ex.gate; a.wb = ex.up; a.stride_a = ex.gate_stride; a.stride_b = ex.up_stride; a.fmt = FQ4K;
    a.sh_a = sh.gate; a.sh_b = sh.up; a.sh_fmt = sh.gate_fmt;
    a.src = x16; a.T = T; a.H = H; a.M = M; a.S = sh.gate ? sh.S : 0; a.K = K; a.E = E;
    a.tiles = tiles; a.pairs = pairs; a.act = act; a.act_sh = act_sh;
    const int nby = (M > a.S ? M : a.S) / NB;
    hipLaunchKernelGGL(k_gemm_gate_up, dim3(n_tiles_max, nby), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

int launch_gemm_down(const ExpertSide &ex, const SharedSide &sh, const _Float16 *act,
                     const _Float16 *act_sh, int T, int H, int M, int K, int E, const uint32_t *tiles,
                     int n_tiles_max, float *y, float *ysh, hipStream_t s) {
    if (H % NB || M % 256 || (sh.gate && sh.S % 256)) return -2;
    if (ex.down_fmt != FQ4K && ex.down_fmt != FQ6K) return -2;
    if (sh.gate && sh.down_fmt != FQ4K && sh.down_fmt != FQ6K && sh.down_fmt != FQ8) return -2;
    GemmArgs a = {};
    a.wa = ex.down; a.stride_a = ex.down_stride; a.fmt = ex.down_fmt;
    a.sh_a = sh.gate ? sh.down : nullptr; a.sh_fmt = sh.down_fmt;
    a.src = act; a.src_sh = act_sh; a.T = T; a.H = H; a.M = M; a.S = sh.gate ? sh.S : 0; a.K = K; a.E = E;
    a.tiles = tiles; a.y = y; a.ysh = ysh;
    hipLaunchKernelGGL(k_gemm_down, dim3(n_tiles_max, H / NB), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
