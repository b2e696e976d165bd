/* kernels.h -- launch interface between the C-ABI host code and the kernels. */
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

/* Kernel launches of the library.  While the host's stage timing brackets a
 * stage, g_launch_ev holds that stage's event pair: the stage's kernels are
 * launched with hipExtLaunchKernel, the first one recording `start` when it
 * begins and each one recording `stop` when it ends, so the pair spans
 * exactly the stage's kernels (the dispatches' own begin/end times, not
 * separate marker packets).  Otherwise a plain launch. */
struct LaunchEvents {
    hipEvent_t start, stop;
};
extern thread_local LaunchEvents g_launch_ev;
#define KLAUNCH(K, G, B, SH, S, ...)                                                                     \
    do {                                                                                                 \
        if (g_launch_ev.stop) {                                                                          \
            hipExtLaunchKernelGGL(K, G, B, SH, S, g_launch_ev.start, g_launch_ev.stop, 0, __VA_ARGS__);  \
            g_launch_ev.start = nullptr;                                                                 \
        } else {                                                                                         \
            hipLaunchKernelGGL(K, G, B, SH, S, __VA_ARGS__);                                             \
        }                                                                                                \
    } while (0)

/* Compact list of the experts a call touches, written by the routing kernels:
 *   list[0]            n_active
 *   list[1 + u]        expert id of active slot u (ascending), u < n_active
 *   list[1 + E + u]    first sorted position of slot u; entry n_active = T*K */
#define OROME_MAXK 16

#define ACT_N(list) ((list)[0])
#define ACT_E(list, u) ((list)[1 + (u)])
#define ACT_OFF(list, E, u) ((list)[1 + (E) + (u)])

struct RouteArgs {
    const float *W;      /* [E][H] */
    const float *wsg;    /* [H] or NULL */
    const float *bias;   /* [E] or NULL */
    const float *x;      /* [T][H] */
    int T, E, H, K;
    float *logits;       /* [T][E+1] */
    _Float16 *x16;       /* large-batch router: also writes x as fp16, (0,2,1,3) per 4-group (or NULL) */
    const _Float16 *x16in; /* two-pass router: x already staged so (the previous layer's combine), read
                              in place of x by the approximation pass; NULL: x */
    int32_t *idx;        /* [T][K] */
    float *w;            /* [T][K] */
    float *sgl;          /* [T] shared-gate logit */
    uint32_t *offsets;   /* [E+1] */
    uint32_t *pairs;     /* [T*K] sorted pair ids */
    uint32_t *pos;       /* [T*K] sorted position of pair p */
    uint32_t *list;      /* active list, 2E+2 entries */
    uint32_t *counter;   /* one zeroed word, returned to zero by the kernel */
    /* fused RMSNorm (small-batch router only): when norm_h is set, x is
     * RMSNorm(norm_h) * bf16(norm_w) computed in the router kernel, which
     * also writes it to xnorm for the later kernels */
    const float *norm_h, *norm_w;
    float norm_eps;
    float *xnorm;
    /* two-pass large-batch router (launch_route_approx + launch_topk_exact):
     * W16[e] = fp16(W[e] * 2^s_e), wscale[e] = 2^-s_e, wnorm[e] >= ||W[e]||_2
     * (from launch_pack_router); eps_c1/eps_c2 from route_eps_coeffs */
    const _Float16 *W16;
    const float *wscale, *wnorm;
    float eps_c1, eps_c2;
    /* the approximation pass writes unscaled partial sums part[q][t][e]
     * over 8 k-slices q ([8][T][E]); the exact top-k sums them, q
     * ascending, and applies wscale */
    float *part;
    /* small-batch dispatch feeding the grouped GEMMs: also write the small
     * tile list (one tile per active expert, then the shared expert's) */
    uint32_t *tiles_s;
    int has_shared;
    /* exact top-k above the one-block dispatch's size: also adds each
     * selected (token, expert) to dcnt[token / 256][expert], the counts the
     * three-launch dispatch would otherwise count (launch_dispatch(counted));
     * the approximation pass clears them first.  NULL: not counted */
    uint32_t *dcnt;
    /* exact top-k: sets byte tmask[e * TMASK_LD(T) + t] to 1 for each
     * selection (t, e): the token marks the self-dispatching gate/up reads
     * (plain byte stores; the approximation pass clears them first).  NULL:
     * not set */
    uint8_t *tmask;
};

struct ExpertSide {
    const uint8_t *gate, *up, *down;  /* device addresses of expert 0 */
    size_t gate_stride, up_stride, down_stride;
    int gate_fmt, down_fmt;           /* gate and up share a format */
};

struct SharedSide {
    const uint8_t *gate, *up, *down;  /* NULL gate: no shared expert */
    int gate_fmt, down_fmt;
    int S;
};

/* fold_topk: the router's last block also runs the top-k and dispatch of
 * launch_topk_dispatch_small (when route_small_folds(a)) */
int launch_route_small(const RouteArgs &a, hipStream_t s, int fold_topk = 0);
int route_small_folds(const RouteArgs &a);
int launch_route_logits(const RouteArgs &a, hipStream_t s);
int launch_topk(const RouteArgs &a, hipStream_t s);
int launch_route_approx(const RouteArgs &a, hipStream_t s);
/* whether the small-tile grouped GEMMs take these shapes and formats */
int gemm_small_tiles_ok(const ExpertSide &ex, const SharedSide &sh, int H, int M);
int launch_topk_exact(const RouteArgs &a, hipStream_t s);
int launch_pack_router(const float *W, int E, int H, _Float16 *W16, float *wscale, float *wnorm, hipStream_t s);
void route_eps_coeffs(int H, float *c1, float *c2);
int dispatch_blocks(int T); /* rows of the dispatch count scratch ([rows][E] words) */
int launch_dispatch(const RouteArgs &a, uint32_t *tiles_s, uint32_t *tiles_b, int has_shared, uint32_t *cnt,
                    hipStream_t s, int counted = 0);
/* the dispatch runs in three launches (count, scan, scatter) for these
 * shapes, one block otherwise */
bool dispatch_three_launches(const RouteArgs &a);

/* decode gate/up; with route_in_block the top-k + dispatch of the call is
 * folded in (every block selects; block 0 publishes the routing outputs in
 * `ra`), otherwise it reads the routing written by launch_topk_dispatch_small */
/* act_by_slot (only where the one-token kernel runs, gemv_gate_up1_path):
 * act row k holds the expert of selection slot k instead of its sorted
 * position, for launch_gemv_down_combine1 with the same flag */
int launch_gemv_gate_up(const ExpertSide &ex, const SharedSide &sh, const RouteArgs &ra, int route_in_block,
                        const float *x, int T, int H, int M, int K, int E, _Float16 *act, _Float16 *act_sh,
                        hipStream_t s, unsigned long long *kt = nullptr, int kt_cap = 0, int act_by_slot = 0);
/* the decode gate/up takes its one-token kernel (routing folded in) */
bool gemv_gate_up1_path(int route_in_block, int T, int H, const SharedSide &sh);
int launch_topk_dispatch_small(const RouteArgs &a, hipStream_t s);

int launch_gemv_down(const ExpertSide &ex, const SharedSide &sh, const _Float16 *act,
                     const _Float16 *act_sh, int T, int H, int M, int K, int E, const uint32_t *list,
                     float *y, float *ysh, hipStream_t s);

/* T = 1: down of all K routed slots and the shared slot, combined into h_out
 * (K <= 8, M = S = 512); returns -2 when the shape is not covered */
int launch_gemv_down_combine1(const ExpertSide &ex, const SharedSide &sh, const RouteArgs &ra,
                              const _Float16 *act, const _Float16 *act_sh, int H, int M, int K,
                              const float *h_in, float *h_out, float *res, hipStream_t s,
                              const float *next_router = nullptr, int act_by_slot = 0);
int launch_delay(uint32_t usec, hipStream_t s);
int launch_rmsnorm(const float *h, const float *w, int T, int H, float eps, float *x, hipStream_t s);
int launch_dequant(int fmt, const uint8_t *src, uint32_t rows, uint32_t n, float *out32,
                   _Float16 *out16, hipStream_t s);

/* prefill (MFMA) path; x16 is written (0,2,1,3) within each 4-group */
int launch_to_f16(const float *x, int T, int H, _Float16 *x16, hipStream_t s);
/* x16, act and act_sh rows are stored (0,2,1,3) within each 4-group; zrow /
 * zrow_sh name an all-zero row of the activation source(s) */
/* self-dispatch of the small-tile gate/up: the exact top-k's counts, token
 * marks and selections, and the dispatch outputs the gate/up writes in place
 * of the dispatch kernel (offsets, pairs, pos and the tile list `tiles`) */
/* row pitch (bytes) of the token marks: T rounded up to 64 */
#define TMASK_LD(T) (((T) + 63) / 64 * 64)
struct GemmSelfDispatch {
    const uint32_t *dcnt;  /* [g][E] expert counts per 256-token block */
    int g;
    const uint8_t *tmask;  /* [E][TMASK_LD(T)] token marks per expert */
    const int32_t *idx;    /* [T][K] */
    uint32_t *offsets, *pairs, *pos;
};
/* whether the small-tile gate/up can dispatch itself at these shapes */
bool gemm_self_dispatch_ok(int T, int K, int E);
int launch_gemm_gate_up(const ExpertSide &ex, const SharedSide &sh, const _Float16 *x16, int zrow, int T,
                        int H, int M, int K, int E, int tile_m, const uint32_t *tiles, int n_tiles_max,
                        const uint32_t *pairs, _Float16 *act, _Float16 *act_sh, hipStream_t s, unsigned long long *kt = nullptr,
                        int kt_cap = 0, const GemmSelfDispatch *sd = nullptr);
int launch_gemm_down(const ExpertSide &ex, const SharedSide &sh, const _Float16 *act,
                     const _Float16 *act_sh, int zrow, int zrow_sh, int T, int H, int M, int K, int E, int tile_m,
                     const uint32_t *tiles, int n_tiles_max, float *y, float *ysh,
                     hipStream_t s);
/* tile-major repack of Q4_K expert matrices for the grouped GEMMs (format
 * id 4 in ExpertSide / SharedSide) */
enum { GEMM_FMT_Q4K_TILED = 4, GEMM_FMT_Q6K_TILED = 5, GEMM_FMT_Q8_TILED = 6, GEMM_FMT_Q5K_TILED = 7 };
size_t packed_q4k_bytes(int R, int K, int E);
int launch_pack_q4k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s);
size_t packed_q6k_bytes(int R, int K, int E);
int launch_pack_q6k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s);
size_t packed_q8_bytes(int R, int K, int E);
size_t packed_q5k_bytes(int R, int K, int E);
int launch_pack_q5k(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s);
int launch_pack_q8(const uint8_t *src, uint8_t *dst, int R, int K, int E, size_t src_stride, hipStream_t s);
/* prefill combine of one token per wave that also writes the next layer's
 * RMSNorm of h_out into xnorm (nw: its weight, or NULL for ones) */
int launch_combine_norm(const float *y, const float *ysh, const uint32_t *pos, const float *w, const float *sgl,
                        int has_shared, const float *h_in, float *h_out, float *res, float *ssq, int T, int H, int K,
                        const float *nw, float eps, float *xnorm, _Float16 *x16, hipStream_t s);
/* combine; res (a copy of h_out) and ssq (the [T][H/256] canonical Sigma h^2
 * parts) may be NULL */
int launch_combine(const float *y, const float *ysh, const uint32_t *pos, const float *w,
                   const float *sgl, int has_shared, const float *h_in, float *h_out, float *res, float *ssq,
                   int T, int H, int K, hipStream_t s);
/* ssq[t][b] = canonical sum of h[t][256 b .. 256 b + 255]^2 */
int launch_sumsq_parts(const float *h, int T, int H, float *ssq, hipStream_t s);
/* ggml -> reference Q4_K scale packing of n blocks in place */
int launch_q4k_ggml_to_ref(uint8_t *blocks, size_t n, hipStream_t s);
/* zero fill by a kernel (bytes a multiple of 4) */
int launch_zero(void *p, size_t bytes, hipStream_t s);
int launch_fill_u32(void *p, uint32_t v, size_t words, hipStream_t s);

/* tile list for the grouped GEMM: tiles[0] = count, then (expert, first, rows)
 * triples; expert == E denotes the shared expert over all T tokens */
/* two tile lists per call: experts with <= GEMM_TILE_SMALL rows (one small
 * tile each) and the rest in tiles of GEMM_TILE_BIG rows; while T*K <=
 * GEMM_TILE_SMALL*E every expert is cut into small tiles and the shared
 * expert joins the small list (the big list is empty).  Capacities: small
 * 2E + T/SMALL + 1, big T*K/BIG + E + T/BIG + 1. */
#define GEMM_TILE_SMALL 32
/* 16-row tiles for lists whose experts hold at most 16 rows (the small-batch
 * path: T <= 16); per-tile kernels only */
#define GEMM_TILE_MIN 16
#ifndef GEMM_TILE_BIG
#define GEMM_TILE_BIG 80
#endif
