/*
 * host.hip -- C ABI: context, device memory, and the MoE forward driver.
 *
 * Replaces the reference's Metal context (inference/src/metal.m:41-256) and
 * the encoding of the MoE stages (inference/src/engine.m:158-340, routing at
 * 656-685).  All work of one call is queued on the context's stream in
 * order; there are no host synchronisations inside a forward.
 */
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "kernels.h"
#include "orome_internal.h"
#include "orome_moe.h"

static thread_local char g_err[512];

extern "C" int orome_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "[hip] %s\n", g_err);
    return code;
}

extern "C" const char *orome_last_error(void) { return g_err; }
extern "C" const char *orome_version(void) { return "orome-mi355x 0.1 (gfx950)"; }

#define HIP_OK(expr, code)                                                                  \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return orome_fail(code, "%s failed: %s", #expr, hipGetErrorString(e_));         \
    } while (0)

enum { ST_NORM, ST_ROUTE, ST_TOPK, ST_DISPATCH, ST_STAGE, ST_GATE_UP, ST_DOWN, ST_COMBINE, N_STAGES };

struct orome_hip_ctx {
    int device;
    hipStream_t stream;
    hipStream_t side;        /* second stream: the big-tile GEMM list runs beside the small one */
    hipEvent_t fork, join;
    OromeHipModelConfig cfg;
    int tmax, kmax, path;
    /* scratch */
    float *logits, *w, *sgl, *y, *ysh, *xnorm;
    int32_t *idx;
    uint32_t *offsets, *pairs, *pos, *list, *counter, *tiles, *tiles_b, *dcount;
    uint8_t *tmask;
    _Float16 *x16, *act, *act_sh;
    void *arena;
    size_t arena_bytes;
    int last_T, last_K;
    hipStream_t last_stream; /* stream of the most recent forward (debug outputs wait for it) */
    /* per-stage kernel timing (eager launches only) */
    int timing, tcap;
    hipEvent_t *ev;          /* [N_STAGES][tcap][2] */
    int tcount[N_STAGES];
    /* tile-major copies of registered layers' Q4_K expert matrices */
    struct Pack *packs;
    int npacks, pcap;
    /* per-block stamps of the gate/up launches (orome_hip_kernel_timing) */
    unsigned long long *kt;
    int kt_blocks;
    int inject; /* orome_hip_debug_inject_failure: fail the next forward after its router launch */
};

/* One registered layer: keyed by the routed gate and shared gate device
 * addresses; the copies' addresses (NULL where a matrix was not repacked). */
struct Pack {
    const uint8_t *key, *sh_key;
    void *mem;
    const uint8_t *gate, *up, *down, *sgate, *sup, *sdown;
    size_t gate_stride, down_stride;
    int sgate_fmt;           /* GEMM_FMT_Q4K_TILED or GEMM_FMT_Q8_TILED */
    int down_fmt, sdown_fmt; /* GEMM_FMT_Q{4,5,6}K_TILED (or, shared, GEMM_FMT_Q8_TILED) */
    /* router copy for the two-pass large-batch router (r16 NULL: none) */
    const float *rkey;
    _Float16 *r16;
    float *rscale, *rnorm;
};

/* Carves the scratch buffers of a context sized for c->tmax tokens, K up to
 * c->kmax and c->cfg's shapes out of `base` (NULL: only sizes); returns the
 * bytes needed.  Each part starts on a 256-byte boundary. */
static size_t scratch_layout(orome_hip_ctx *c, uint8_t *base) {
    const OromeHipModelConfig *cfg = &c->cfg;
    const size_t T = (size_t)c->tmax, E = (size_t)cfg->num_experts, K = (size_t)c->kmax,
                 H = (size_t)cfg->hidden_dim, M = (size_t)cfg->moe_intermediate,
                 S = (size_t)(cfg->shared_intermediate > 0 ? cfg->shared_intermediate : 0);
    const size_t ntile_s = 2 * E + T / GEMM_TILE_SMALL + 2, ntile_b = (T * K) / GEMM_TILE_BIG + E + T / GEMM_TILE_BIG + 2;
    struct { void **p; size_t bytes; } parts[] = {
        {(void **)&c->logits, T * (E + 1) * 4}, {(void **)&c->idx, T * K * 4},
        {(void **)&c->w, T * K * 4},           {(void **)&c->sgl, T * 4},
        {(void **)&c->offsets, (E + 1) * 4},    {(void **)&c->pairs, T * K * 4},
        {(void **)&c->pos, T * K * 4},          {(void **)&c->list, (2 * E + 2) * 4},
        {(void **)&c->counter, 256},            {(void **)&c->tiles, (1 + 3 * ntile_s) * 4},
        {(void **)&c->tiles_b, (1 + 3 * ntile_b) * 4},
        {(void **)&c->dcount, (size_t)dispatch_blocks((int)T) * E * 4},
        {(void **)&c->tmask, (size_t)TMASK_LD(T) * E},
        /* one extra all-zero row each (index tmax, tmax*kmax, tmax) */
        {(void **)&c->x16, (T + 1) * H * 2},    {(void **)&c->act, (T * K + 1) * M * 2},
        {(void **)&c->act_sh, (T + 1) * (S ? S : 1) * 2}, {(void **)&c->y, T * K * H * 4},
        {(void **)&c->ysh, T * H * 4},          {(void **)&c->xnorm, T * H * 4},
    };
    size_t off = 0;
    for (auto &p : parts) {
        if (base) *p.p = base + off;
        off += (p.bytes + 255) / 256 * 256;
    }
    return off;
}

static int set_dev(orome_hip_ctx *c) {
    HIP_OK(hipSetDevice(c->device), OROME_EHIP);
    return OROME_OK;
}

extern "C" orome_hip_ctx *orome_hip_create(const OromeHipModelConfig *cfg, int max_tokens, int device) {
    if (!cfg || max_tokens < 1 || cfg->hidden_dim <= 0 || cfg->num_experts <= 0 ||
        cfg->moe_intermediate <= 0) {
        orome_fail(OROME_EINVAL, "orome_hip_create: invalid config or max_tokens");
        return NULL;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        orome_fail(OROME_EHIP, "orome_hip_create: no HIP device %d (count %d)", device, ndev);
        return NULL;
    }
    orome_hip_ctx *c = (orome_hip_ctx *)calloc(1, sizeof *c);
    c->device = device;
    c->cfg = *cfg;
    c->tmax = max_tokens;
    c->kmax = OROME_MAX_ACTIVE;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        orome_fail(OROME_EHIP, "orome_hip_create: stream creation failed");
        free(c);
        return NULL;
    }
    if (hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->join, hipEventDisableTiming) != hipSuccess) {
        orome_fail(OROME_EHIP, "orome_hip_create: side stream creation failed");
        (void)hipStreamDestroy(c->stream);
        free(c);
        return NULL;
    }
    const size_t total = scratch_layout(c, NULL);
    if (hipMalloc(&c->arena, total) != hipSuccess) {
        orome_fail(OROME_ENOMEM, "orome_hip_create: scratch arena of %zu bytes", total);
        (void)hipStreamDestroy(c->side);
        (void)hipStreamDestroy(c->stream);
        free(c);
        return NULL;
    }
    c->arena_bytes = total;
    scratch_layout(c, (uint8_t *)c->arena);
    /* the zero rows past x16, act and act_sh must read as zeros; nothing
     * writes them, so this is the only clear needed */
    if (hipMemset(c->arena, 0, total) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        orome_fail(OROME_EHIP, "orome_hip_create: scratch clear failed");
        (void)hipFree(c->arena);
        (void)hipStreamDestroy(c->side);
        (void)hipStreamDestroy(c->stream);
        free(c);
        return NULL;
    }
    return c;
}

static void free_timing(orome_hip_ctx *c) {
    if (!c->ev) return;
    for (int i = 0; i < N_STAGES * c->tcap * 2; i++) (void)hipEventDestroy(c->ev[i]);
    free(c->ev);
    c->ev = NULL;
    c->timing = 0;
}

extern "C" int orome_hip_unpack_all(orome_hip_ctx *c);

extern "C" void orome_hip_destroy(orome_hip_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    (void)hipStreamSynchronize(c->side);
    (void)orome_hip_unpack_all(c);
    free_timing(c);
    (void)hipFree(c->arena);
    (void)hipEventDestroy(c->fork);
    (void)hipEventDestroy(c->join);
    (void)hipStreamDestroy(c->side);
    (void)hipStreamDestroy(c->stream);
    free(c);
}

extern "C" int orome_hip_sync(orome_hip_ctx *c) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_hip_sync: NULL ctx");
    HIP_OK(hipStreamSynchronize(c->stream), OROME_EHIP);
    return OROME_OK;
}

extern "C" void *orome_hip_get_stream(orome_hip_ctx *c) { return c ? (void *)c->stream : NULL; }

extern "C" int orome_hip_set_path(orome_hip_ctx *c, int path) {
    if (!c || path < OROME_PATH_AUTO || path > OROME_PATH_MFMA)
        return orome_fail(OROME_EINVAL, "orome_hip_set_path: bad argument");
    c->path = path;
    return OROME_OK;
}

extern "C" int orome_hip_kernel_timing(orome_hip_ctx *c, unsigned long long *stamps, int blocks) {
    if (!c || (stamps && blocks < 2)) return orome_fail(OROME_EINVAL, "orome_hip_kernel_timing: bad argument");
    c->kt = stamps;
    c->kt_blocks = stamps ? blocks : 0;
    return OROME_OK;
}

extern "C" void *orome_hip_malloc(orome_hip_ctx *c, size_t bytes) {
    if (!c) { orome_fail(OROME_EINVAL, "orome_hip_malloc: NULL ctx"); return NULL; }
    if (set_dev(c)) return NULL;
    void *p = NULL;
    /* 256 bytes of tail padding: the 2-byte-aligned block loads of the Q6_K /
     * Q8_0 kernels may touch up to 4 bytes past a tensor's last block */
    if (hipMalloc(&p, bytes + 256) != hipSuccess) {
        orome_fail(OROME_ENOMEM, "hipMalloc(%zu) failed", bytes);
        return NULL;
    }
    return p;
}

extern "C" int orome_hip_free(orome_hip_ctx *c, void *p) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_hip_free: NULL ctx");
    if (set_dev(c)) return OROME_EHIP;
    HIP_OK(hipFree(p), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_htod(orome_hip_ctx *c, void *dst, const void *src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return orome_fail(OROME_EINVAL, "orome_hip_htod: bad argument");
    if (set_dev(c)) return OROME_EHIP;
    HIP_OK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), OROME_EHIP);
    HIP_OK(hipStreamSynchronize(c->stream), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_dtoh(orome_hip_ctx *c, void *dst, const void *src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return orome_fail(OROME_EINVAL, "orome_hip_dtoh: bad argument");
    if (set_dev(c)) return OROME_EHIP;
    HIP_OK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), OROME_EHIP);
    HIP_OK(hipStreamSynchronize(c->stream), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_q4k_ggml_to_reference(orome_hip_ctx *c, void *blocks, size_t nblocks) {
    if (!c || !blocks) return orome_fail(OROME_EINVAL, "q4k relayout: NULL argument");
    if (set_dev(c)) return OROME_EHIP;
    const int rc = launch_q4k_ggml_to_ref((uint8_t *)blocks, nblocks, c->stream);
    if (rc) return orome_fail(rc == -1 ? OROME_EINVAL : OROME_EHIP, "q4k relayout: launch failed (%d)", rc);
    HIP_OK(hipStreamSynchronize(c->stream), OROME_EHIP);
    return OROME_OK;
}

/* --------------------------------------------------------------- forward */

static const uint8_t *dev_addr(const void *buffer, size_t offset) {
    return buffer ? (const uint8_t *)buffer + offset : NULL;
}

static int kfmt(OromeHipQuantFormat f) {
    switch (f) {
        case OROME_QFMT_GGUF_Q4_K: return 0;
        case OROME_QFMT_GGUF_Q5_K: return 1;
        case OROME_QFMT_GGUF_Q6_K: return 2;
        case OROME_QFMT_GGUF_Q8_0: return 3;
        default: return -1;
    }
}

/* ------------------------------------------------- tile-major repacking */

/* The grouped GEMMs' view of a layer: registered layers read their
 * tile-major copies (each matrix that was repacked). */
static const Pack *find_pack(const orome_hip_ctx *c, const uint8_t *gate, const uint8_t *sh_gate);
static void apply_pack(const orome_hip_ctx *c, int S, ExpertSide &exm, SharedSide &shm) {
    const Pack *pk = find_pack(c, exm.gate, shm.gate);
    if (!pk) return;
    exm.gate = pk->gate;
    exm.up = pk->up;
    exm.gate_stride = exm.up_stride = pk->gate_stride;
    exm.gate_fmt = GEMM_FMT_Q4K_TILED;
    if (S && pk->sgate) {
        shm.gate = pk->sgate;
        shm.up = pk->sup;
        shm.gate_fmt = pk->sgate_fmt;
    }
    if (pk->down) {
        exm.down = pk->down;
        exm.down_stride = pk->down_stride;
        exm.down_fmt = pk->down_fmt;
    }
    if (S && pk->sdown) {
        shm.down = pk->sdown;
        shm.down_fmt = pk->sdown_fmt;
    }
}

/* OROME_ROUTE_EXACT=1 keeps the one-pass canonical router on registered
 * layers too (the two routers select identically; this is for comparing them). */
static bool route_exact_only() {
    const char *v = getenv("OROME_ROUTE_EXACT");
    return v && v[0] == '1';
}

static const Pack *find_pack(const orome_hip_ctx *c, const uint8_t *gate, const uint8_t *sh_gate) {
    for (int k = 0; k < c->npacks; k++)
        if (c->packs[k].key == gate && c->packs[k].sh_key == sh_gate) return &c->packs[k];
    return NULL;
}

extern "C" int orome_hip_pack_layer(orome_hip_ctx *c, const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *elr,
                                    const OromeHipLayerTensorCache *lt) {
    if (!c || !cfg || !elr || !lt || !elr->buffer) return orome_fail(OROME_EINVAL, "orome_hip_pack_layer: NULL argument");
    const int H = cfg->hidden_dim, E = cfg->num_experts, M = cfg->moe_intermediate;
    if (H != c->cfg.hidden_dim || E != c->cfg.num_experts || M != c->cfg.moe_intermediate)
        return orome_fail(OROME_EINVAL, "orome_hip_pack_layer: config differs from the context's");
    if (elr->gate.format != OROME_QFMT_GGUF_Q4_K || elr->up.format != OROME_QFMT_GGUF_Q4_K || H % 256 || M % 256)
        return orome_fail(OROME_EUNSUPPORTED, "orome_hip_pack_layer: routed gate/up must be Q4_K, H and M multiples of 256");
    const int S = lt->shared_gate.buffer ? (int)lt->shared_gate.out_dim : 0;
    if (S % 256) return orome_fail(OROME_EUNSUPPORTED, "orome_hip_pack_layer: shared intermediate %d not a multiple of 256", S);
    /* Every matrix the tile-major spans can hold is repacked: routed gate/up
     * (Q4_K), the shared gate/up when Q4_K or Q8_0 (the reference's 35B
     * layout has a Q8_0 shared expert), the routed down when Q4_K, Q5_K or
     * Q6_K, and then the shared down when Q4_K, Q5_K, Q6_K or Q8_0. */
    auto tileable = [](OromeHipQuantFormat f) {
        return f == OROME_QFMT_GGUF_Q4_K || f == OROME_QFMT_GGUF_Q5_K || f == OROME_QFMT_GGUF_Q6_K;
    };
    /* bytes, packer and tile-major format id of a down projection */
    auto dn_bytes = [](OromeHipQuantFormat f, int R, int K, int n) {
        return f == OROME_QFMT_GGUF_Q6_K ? packed_q6k_bytes(R, K, n)
               : f == OROME_QFMT_GGUF_Q5_K ? packed_q5k_bytes(R, K, n)
               : f == OROME_QFMT_GGUF_Q8_0 ? packed_q8_bytes(R, K, n)
                                           : packed_q4k_bytes(R, K, n);
    };
    auto dn_pack = [](OromeHipQuantFormat f) {
        return f == OROME_QFMT_GGUF_Q6_K ? launch_pack_q6k
               : f == OROME_QFMT_GGUF_Q5_K ? launch_pack_q5k
               : f == OROME_QFMT_GGUF_Q8_0 ? launch_pack_q8
                                           : launch_pack_q4k;
    };
    auto dn_fmt = [](OromeHipQuantFormat f) {
        return f == OROME_QFMT_GGUF_Q6_K ? (int)GEMM_FMT_Q6K_TILED
               : f == OROME_QFMT_GGUF_Q5_K ? (int)GEMM_FMT_Q5K_TILED
               : f == OROME_QFMT_GGUF_Q8_0 ? (int)GEMM_FMT_Q8_TILED
                                           : (int)GEMM_FMT_Q4K_TILED;
    };
    const OromeHipQuantFormat sgf = S ? lt->shared_gate.format : OROME_QFMT_F32;
    const bool sh_q8 = S && sgf == OROME_QFMT_GGUF_Q8_0 && lt->shared_up.format == OROME_QFMT_GGUF_Q8_0;
    const bool sh_gu = sh_q8 || (S && sgf == OROME_QFMT_GGUF_Q4_K && lt->shared_up.format == OROME_QFMT_GGUF_Q4_K);
    const bool dn = tileable(elr->down.format);
    const bool sdn_q8 = S && lt->shared_down.format == OROME_QFMT_GGUF_Q8_0;
    const bool sdn_t = S && dn && (tileable(lt->shared_down.format) || sdn_q8);
    const size_t gu = packed_q4k_bytes(M, H, E),
                 dnb = !dn ? 0 : dn_bytes(elr->down.format, H, M, E),
                 sgu = !sh_gu ? 0 : sh_q8 ? packed_q8_bytes(S, H, 1) : packed_q4k_bytes(S, H, 1),
                 sdn = !sdn_t ? 0 : dn_bytes(lt->shared_down.format, H, S, 1);
    if (set_dev(c)) return OROME_EHIP;
    const uint8_t *gate = dev_addr(elr->buffer, elr->gate.offset), *sh_gate = S ? dev_addr(lt->shared_gate.buffer, lt->shared_gate.offset) : NULL;
    if (c->npacks == c->pcap) {
        const int cap = c->pcap ? 2 * c->pcap : 64;
        Pack *np = (Pack *)realloc(c->packs, (size_t)cap * sizeof(Pack));
        if (!np) return orome_fail(OROME_ENOMEM, "orome_hip_pack_layer: registry");
        c->packs = np;
        c->pcap = cap;
    }
    Pack pk = {};
    pk.key = gate;
    pk.sh_key = sh_gate;
    /* router copy (fp32 router, whatever the shared expert's format): fp16
     * rows, scales, norms */
    const bool rt = lt->routing_gate.buffer && lt->routing_gate.format == OROME_QFMT_F32 && H % 128 == 0;
    const size_t rb16 = rt ? ((size_t)E * H * 2 + 255) / 256 * 256 : 0, rbf = rt ? ((size_t)E * 4 + 255) / 256 * 256 : 0;
    const size_t body = (2 * gu + dnb + 2 * sgu + sdn + 255) / 256 * 256;
    HIP_OK(hipMalloc(&pk.mem, body + rb16 + 2 * rbf), OROME_ENOMEM);
    uint8_t *m = (uint8_t *)pk.mem;
    int rc = 0;
    if (rt) {
        pk.rkey = (const float *)dev_addr(lt->routing_gate.buffer, lt->routing_gate.offset);
        pk.r16 = (_Float16 *)(m + body);
        pk.rscale = (float *)(m + body + rb16);
        pk.rnorm = (float *)(m + body + rb16 + rbf);
        rc |= launch_pack_router(pk.rkey, E, H, pk.r16, pk.rscale, pk.rnorm, c->stream);
    }
    pk.gate = m;
    rc |= launch_pack_q4k(gate, m, M, H, E, elr->gate.expert_stride, c->stream);
    m += gu;
    pk.up = m;
    rc |= launch_pack_q4k(dev_addr(elr->buffer, elr->up.offset), m, M, H, E, elr->up.expert_stride, c->stream);
    m += gu;
    pk.gate_stride = gu / E;
    if (dn) {
        pk.down = m;
        pk.down_fmt = dn_fmt(elr->down.format);
        rc |= dn_pack(elr->down.format)(dev_addr(elr->buffer, elr->down.offset), m, H, M, E, elr->down.expert_stride,
                                        c->stream);
        m += dnb;
        pk.down_stride = dnb / E;
    }
    if (sh_gu) {
        auto packf = sh_q8 ? launch_pack_q8 : launch_pack_q4k;
        pk.sgate_fmt = sh_q8 ? GEMM_FMT_Q8_TILED : GEMM_FMT_Q4K_TILED;
        pk.sgate = m;
        rc |= packf(sh_gate, m, S, H, 1, 0, c->stream);
        m += sgu;
        pk.sup = m;
        rc |= packf(dev_addr(lt->shared_up.buffer, lt->shared_up.offset), m, S, H, 1, 0, c->stream);
        m += sgu;
    }
    if (sdn_t) {
        pk.sdown = m;
        pk.sdown_fmt = dn_fmt(lt->shared_down.format);
        rc |= dn_pack(lt->shared_down.format)(dev_addr(lt->shared_down.buffer, lt->shared_down.offset), m, H, S, 1, 0,
                                              c->stream);
    }
    if (rc || hipStreamSynchronize(c->stream) != hipSuccess) {
        (void)hipFree(pk.mem);
        return orome_fail(OROME_EHIP, "orome_hip_pack_layer: repack failed (%d)", rc);
    }
    for (int k = 0; k < c->npacks; k++) /* re-registration replaces */
        if (c->packs[k].key == gate && c->packs[k].sh_key == sh_gate) {
            (void)hipFree(c->packs[k].mem);
            c->packs[k] = pk;
            return OROME_OK;
        }
    c->packs[c->npacks++] = pk;
    return OROME_OK;
}

extern "C" int orome_hip_unpack_all(orome_hip_ctx *c) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_hip_unpack_all: NULL ctx");
    if (c->npacks) {
        if (set_dev(c)) return OROME_EHIP;
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamSynchronize(c->side);
        for (int k = 0; k < c->npacks; k++) (void)hipFree(c->packs[k].mem);
    }
    free(c->packs);
    c->packs = NULL;
    c->npacks = c->pcap = 0;
    return OROME_OK;
}

static int launch_rc(int rc, const char *what) {
    if (rc == 0) return OROME_OK;
    if (rc == -2) return orome_fail(OROME_EUNSUPPORTED, "%s: shape or format not supported", what);
    if (rc == -1) return orome_fail(OROME_EINVAL, "%s: invalid argument", what);
    return orome_fail(OROME_EHIP, "%s: launch failed: %s", what, hipGetErrorString(hipGetLastError()));
}

#define LAUNCH(call, what)                  \
    do {                                    \
        int rc_ = launch_rc((call), (what)); \
        if (rc_) return rc_;                \
    } while (0)

/* launch with optional per-stage timing: the stage's kernels carry the
 * stage's event pair (KLAUNCH) */
thread_local LaunchEvents g_launch_ev = {nullptr, nullptr};
#define TLAUNCH(c, st, call, what)                                                         \
    do {                                                                                   \
        hipEvent_t *ev_ = NULL;                                                            \
        if ((c)->timing) {                                                                 \
            ev_ = &(c)->ev[((st) * (c)->tcap + (c)->tcount[st] % (c)->tcap) * 2];          \
            g_launch_ev = LaunchEvents{ev_[0], ev_[1]};                                    \
        }                                                                                  \
        const int trc_ = launch_rc((call), (what));                                        \
        g_launch_ev = LaunchEvents{nullptr, nullptr};                                      \
        if (trc_) return trc_;                                                             \
        if (ev_) (c)->tcount[st]++;                                                        \
    } while (0)

/* State that kernels carry from one forward to the next: the folded small-
 * batch router's arrival counter, which its last block returns to zero.  A
 * forward that stops between launches (an error on the host) may leave it
 * torn; this fill kernel (no memset node, so graph capture may record it)
 * puts it back.  The top-k counts are cleared by every forward that uses
 * them, before use. */
static int reset_state(orome_hip_ctx *c, hipStream_t s) {
    return launch_rc(launch_zero(c->counter, 256, s), "scratch state reset");
}

/* The MoE block on x (or, with norm_h, on RMSNorm(norm_h) * bf16(norm_w),
 * which the small-batch router computes itself and the large-batch path
 * computes in a separate kernel first). */
/* Outputs beside h_out: the residual copy and the Sigma h^2 parts (either
 * may be NULL). */
struct FwdOut {
    float *res, *ssq;
    const float *next_router = nullptr; /* the next layer's router rows (a stack forward), touched early */
};

static int forward_impl(orome_hip_ctx *c, const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *elr,
                        const OromeHipLayerTensorCache *lt, const float *x, const float *h_in, float *h_out, int T,
                        int K, const float *norm_h, const float *norm_w, hipStream_t s, FwdOut fo,
                        const float *next_norm_w = NULL, int fuse_next_norm = 0, int pre_normed = 0) {
    if (!c || !cfg || !elr || !lt || !(x || norm_h) || !h_out)
        return orome_fail(OROME_EINVAL, "orome_moe_forward: NULL argument");
    const int H = cfg->hidden_dim, E = cfg->num_experts, M = cfg->moe_intermediate;
    if (H != c->cfg.hidden_dim || E != c->cfg.num_experts || M != c->cfg.moe_intermediate ||
        cfg->shared_intermediate > c->cfg.shared_intermediate)
        return orome_fail(OROME_EINVAL, "orome_moe_forward: config differs from the context's");
    if (T < 1 || T > c->tmax) return orome_fail(OROME_EINVAL, "orome_moe_forward: T=%d outside 1..%d", T, c->tmax);
    if (K < 1 || K > OROME_MAX_ACTIVE || K > E)
        return orome_fail(OROME_EINVAL, "orome_moe_forward: K=%d outside 1..min(%d, E)", K, OROME_MAX_ACTIVE);
    if (H % 256 || M % 256) return orome_fail(OROME_EUNSUPPORTED, "orome_moe_forward: H and M must be multiples of 256");
    if (!elr->buffer || elr->gate.format != OROME_QFMT_GGUF_Q4_K || elr->up.format != OROME_QFMT_GGUF_Q4_K)
        return orome_fail(OROME_EUNSUPPORTED, "orome_moe_forward: routed gate/up must be Q4_K");
    if (kfmt(elr->down.format) < 0 || kfmt(elr->down.format) > 2)
        return orome_fail(OROME_EUNSUPPORTED, "orome_moe_forward: routed down must be Q4_K, Q5_K or Q6_K");
    if (!lt->routing_gate.buffer || lt->routing_gate.format != OROME_QFMT_F32)
        return orome_fail(OROME_EUNSUPPORTED, "orome_moe_forward: router must be F32");
    const int S = lt->shared_gate.buffer ? (int)lt->shared_gate.out_dim : 0;
    SharedSide sh = {NULL, NULL, NULL, 0, 0, 0};
    if (S) {
        if (S > c->cfg.shared_intermediate)
            return orome_fail(OROME_EINVAL, "orome_moe_forward: shared expert larger than the context's");
        if (!lt->shared_up.buffer || !lt->shared_down.buffer ||
            lt->shared_gate.format != lt->shared_up.format || kfmt(lt->shared_gate.format) == 1 ||
            kfmt(lt->shared_gate.format) == 2 || kfmt(lt->shared_gate.format) < 0 || kfmt(lt->shared_down.format) < 0)
            return orome_fail(OROME_EUNSUPPORTED, "orome_moe_forward: shared expert formats");
        sh.gate = dev_addr(lt->shared_gate.buffer, lt->shared_gate.offset);
        sh.up = dev_addr(lt->shared_up.buffer, lt->shared_up.offset);
        sh.down = dev_addr(lt->shared_down.buffer, lt->shared_down.offset);
        sh.gate_fmt = kfmt(lt->shared_gate.format);
        sh.down_fmt = kfmt(lt->shared_down.format);
        sh.S = S;
    }
    ExpertSide ex;
    ex.gate = dev_addr(elr->buffer, elr->gate.offset);
    ex.up = dev_addr(elr->buffer, elr->up.offset);
    ex.down = dev_addr(elr->buffer, elr->down.offset);
    ex.gate_stride = elr->gate.expert_stride;
    ex.up_stride = elr->up.expert_stride;
    ex.down_stride = elr->down.expert_stride;
    ex.gate_fmt = 0;
    ex.down_fmt = kfmt(elr->down.format);
    if (set_dev(c)) return OROME_EHIP;

    RouteArgs a;
    memset(&a, 0, sizeof a);
    a.W = (const float *)dev_addr(lt->routing_gate.buffer, lt->routing_gate.offset);
    a.wsg = lt->shared_expert_gate.buffer && lt->shared_expert_gate.format == OROME_QFMT_F32
                ? (const float *)dev_addr(lt->shared_expert_gate.buffer, lt->shared_expert_gate.offset)
                : NULL;
    a.bias = lt->routing_bias.buffer ? (const float *)dev_addr(lt->routing_bias.buffer, lt->routing_bias.offset) : NULL;
    a.x = x;
    a.T = T; a.E = E; a.H = H; a.K = K;
    a.logits = c->logits; a.idx = c->idx; a.w = c->w; a.sgl = c->sgl;
    a.offsets = c->offsets; a.pairs = c->pairs; a.pos = c->pos; a.list = c->list;
    a.counter = c->counter;
    a.norm_h = NULL; a.norm_w = NULL; a.norm_eps = cfg->rms_norm_eps; a.xnorm = c->xnorm;
    a.x16 = NULL; a.x16in = NULL;
    a.W16 = NULL; a.wscale = NULL; a.wnorm = NULL; a.eps_c1 = a.eps_c2 = 0.0f;
    a.tiles_s = NULL; a.has_shared = 0; a.dcnt = NULL;

    int path = c->path;
    /* AUTO: GEMV kernels up to 2 tokens (routing folded into gate/up), the
     * small-batch routing with the small-tile grouped GEMMs for 3..16, the
     * large-batch routing and grouped GEMMs above */
    ExpertSide hx = ex;
    SharedSide hs = sh;
    apply_pack(c, S, hx, hs);
    /* (from 3 tokens: the separate top-k + dispatch kernel, which writes the
     * small-tile list, runs only there -- 1..2 tokens fold the routing into
     * the GEMV gate/up; up to 16: one 32-row small tile per expert, and
     * T K <= 256 for the small-batch dispatch) */
    /* (the small-batch router takes H <= 4096; wider layers take the MFMA
     * path under AUTO) */
    const bool small_router = H <= 4096;
    const bool hybrid = path == OROME_PATH_AUTO && T >= 3 && T <= 16 && T * K <= 256 && small_router &&
                        gemm_small_tiles_ok(hx, hs, H, M);
    /* (the GEMV down kernels take in_dim multiples of 512) */
    const bool gemv_shapes = M % 512 == 0 && (!S || S % 512 == 0);
    if (path == OROME_PATH_AUTO)
        path = (T <= 8 && small_router && gemv_shapes) || hybrid ? OROME_PATH_GEMV : OROME_PATH_MFMA;
    c->last_stream = s;
    if (norm_h) {
        if (path == OROME_PATH_GEMV) { /* the router kernel normalises and writes xnorm */
            a.norm_h = norm_h;
            a.norm_w = norm_w;
        } else if (!pre_normed) { /* else the previous layer's combine wrote xnorm */
            TLAUNCH(c, ST_NORM, launch_rmsnorm(norm_h, norm_w, T, H, cfg->rms_norm_eps, c->xnorm, s), "rmsnorm");
        }
        x = c->xnorm;
        a.x = x;
    }
    if (path == OROME_PATH_GEMV) {
        if (T > 8 && !hybrid) return orome_fail(OROME_EUNSUPPORTED, "GEMV path handles T <= 8 (T=%d)", T);
        if (hybrid) { /* the router stages x16 and the dispatch writes the small-tile list */
            a.x16 = c->x16;
            a.tiles_s = c->tiles;
            a.has_shared = S ? 1 : 0;
        }
        /* one or two tokens: every gate/up block selects the experts itself
         * (saves a launch); larger batches route once, in the router
         * kernel's last block where the shapes allow, else in a kernel of
         * its own */
        const int fold = T <= 2, rfold = !fold && route_small_folds(a);
        TLAUNCH(c, ST_ROUTE, launch_route_small(a, s, rfold), rfold ? "router logits + top-k + dispatch" : "router logits");
        if (c->inject) { /* test hook: a torn hand-off counter, then an error */
            c->inject = 0;
            LAUNCH(launch_fill_u32(c->counter, 1u, 1, s), "injected failure");
            return orome_fail(OROME_EHIP, "orome_moe_forward: injected failure after the router launch");
        }
        if (!fold && !rfold) TLAUNCH(c, ST_TOPK, launch_topk_dispatch_small(a, s), "top-k + dispatch");
        if (hybrid) {
            /* every expert holds at most 16 rows: the grouped GEMMs alone
             * (gate/up on 16-row tiles; down keeps the persistent 32-row
             * kernel, faster here), then the combine */
            /* tiles: the active experts (at most T K), then the shared expert's */
            const int ns_max = (T * K < E ? T * K : E) + (S ? 1 : 0);
            TLAUNCH(c, ST_GATE_UP,
                    launch_gemm_gate_up(hx, hs, c->x16, c->tmax, T, H, M, K, E, GEMM_TILE_MIN, c->tiles, ns_max,
                                        c->pairs, c->act, c->act_sh, s, c->kt, c->kt_blocks),
                    "grouped gate/up (small tiles)");
            TLAUNCH(c, ST_DOWN,
                    launch_gemm_down(hx, hs, c->act, c->act_sh, c->tmax * c->kmax, c->tmax, T, H, M, K, E,
                                     GEMM_TILE_SMALL, c->tiles, ns_max, c->y, c->ysh, s),
                    "grouped down (small tiles)");
            TLAUNCH(c, ST_COMBINE, launch_combine(c->y, c->ysh, c->pos, c->w, c->sgl, S ? 1 : 0, h_in, h_out, fo.res, fo.ssq, T, H, K, s),
                    "combine");
            c->last_T = T;
            c->last_K = K;
            return OROME_OK;
        }
        /* one token: down and combine in one kernel when the shape allows;
         * after the one-token gate/up the act rows are in slot order, so
         * that kernel requests them without waiting for the routing */
        const bool dc1 = T == 1 && K <= 8 && M == 512 && (!S || S == 512);
        const int by_slot = dc1 && gemv_gate_up1_path(fold, T, H, sh) ? 1 : 0;
        TLAUNCH(c, ST_GATE_UP,
                launch_gemv_gate_up(ex, sh, a, fold, x, T, H, M, K, E, c->act, c->act_sh, s, c->kt, c->kt_blocks, by_slot),
                "gemv gate/up");
        if (dc1) {
            TLAUNCH(c, ST_DOWN,
                    launch_gemv_down_combine1(ex, sh, a, c->act, c->act_sh, H, M, K, h_in, h_out, fo.res, s, fo.next_router, by_slot),
                    "gemv down + combine");
            if (fo.ssq) TLAUNCH(c, ST_COMBINE, launch_sumsq_parts(h_out, T, H, fo.ssq, s), "sum-of-squares parts");
        } else {
            TLAUNCH(c, ST_DOWN, launch_gemv_down(ex, sh, c->act, c->act_sh, T, H, M, K, E, c->list, c->y, c->ysh, s),
                    "gemv down");
            TLAUNCH(c, ST_COMBINE,
                    launch_combine(c->y, c->ysh, c->pos, c->w, c->sgl, S ? 1 : 0, h_in, h_out, fo.res, fo.ssq, T, H, K, s),
                    "combine");
        }
    } else {
        /* the router writes the fp16 copy of x the GEMMs read, unless the
         * previous layer's combine + RMSNorm already wrote it (a stack) */
        a.x16 = pre_normed ? NULL : c->x16;
        const Pack *rpk = find_pack(c, ex.gate, sh.gate);
        bool self_dispatch = false; /* the small-tile gate/up forms the dispatch itself */
        /* the two-pass router's partial sums (8 T E floats) borrow the down
         * projection's output rows, which are written only after the top-k
         * has read them */
        if (rpk && rpk->r16 && rpk->rkey == a.W && H <= 4096 && K <= 64 && (size_t)8 * E <= (size_t)c->kmax * H &&
            !route_exact_only()) {
            /* registered layer: approximate logits on the matrix cores, then
             * the canonical logits of the experts that can win */
            a.W16 = rpk->r16;
            if (pre_normed) a.x16in = c->x16;
            a.wscale = rpk->rscale;
            a.wnorm = rpk->rnorm;
            a.part = c->y;
            route_eps_coeffs(H, &a.eps_c1, &a.eps_c2);
            /* where the dispatch takes more than one launch, the top-k counts
             * for it, and where the small-tile gate/up dispatches itself, it
             * marks each expert's tokens (into counts or masks the
             * approximation pass clears) */
            self_dispatch = gemm_self_dispatch_ok(T, K, E);
            if (dispatch_three_launches(a) || self_dispatch) a.dcnt = c->dcount;
            if (self_dispatch) a.tmask = c->tmask;
            TLAUNCH(c, ST_ROUTE, launch_route_approx(a, s), "router logits (matrix cores) + fp16 staging");
            a.x16 = NULL;
            TLAUNCH(c, ST_TOPK, launch_topk_exact(a, s), "top-k with canonical recomputation");
        } else {
            TLAUNCH(c, ST_ROUTE, launch_route_logits(a, s), "router logits + fp16 staging");
            a.x16 = NULL;
            TLAUNCH(c, ST_TOPK, launch_topk(a, s), "top-k");
        }
        if (!self_dispatch)
            TLAUNCH(c, ST_DISPATCH, launch_dispatch(a, c->tiles, c->tiles_b, S ? 1 : 0, c->dcount, s, a.dcnt ? 1 : 0), "dispatch");
        const GemmSelfDispatch sdargs = {c->dcount, dispatch_blocks(T), c->tmask, c->idx, c->offsets, c->pairs, c->pos};
        /* one launch per tile list (grid sized for the most tiles it can hold) */
        /* small batches (T K <= 32 E): every expert in 32-row tiles, the
         * shared expert too, and no big-tile list */
        const bool sh_small = (long)T * K <= (long)GEMM_TILE_SMALL * E;
        const int ns_max = E + (sh_small ? (T * K) / GEMM_TILE_SMALL : 0) +
                           (S && sh_small ? (T + GEMM_TILE_SMALL - 1) / GEMM_TILE_SMALL : 0),
                  nb_max = (T * K) / GEMM_TILE_BIG + E + (S && !sh_small ? (T + GEMM_TILE_BIG - 1) / GEMM_TILE_BIG : 0);
        /* registered layers: the grouped GEMMs read the tile-major copies */
        ExpertSide exm = ex;
        SharedSide shm = sh;
        apply_pack(c, S, exm, shm);
        auto gate_up = [&](int tm, hipStream_t st) {
            return tm == GEMM_TILE_SMALL
                       ? launch_gemm_gate_up(exm, shm, c->x16, c->tmax, T, H, M, K, E, tm, c->tiles, ns_max, c->pairs, c->act,
                                             c->act_sh, st, c->kt ? c->kt + 2 * (c->kt_blocks / 2) : nullptr, c->kt_blocks / 2,
                                             self_dispatch ? &sdargs : nullptr)
                       : launch_gemm_gate_up(exm, shm, c->x16, c->tmax, T, H, M, K, E, tm, c->tiles_b, nb_max, c->pairs, c->act,
                                             c->act_sh, st, c->kt, c->kt_blocks / 2);
        };
        auto down = [&](int tm, hipStream_t st) {
            return tm == GEMM_TILE_SMALL
                       ? launch_gemm_down(exm, shm, c->act, c->act_sh, c->tmax * c->kmax, c->tmax, T, H, M, K, E, tm, c->tiles, ns_max, c->y,
                                          c->ysh, st)
                       : launch_gemm_down(exm, shm, c->act, c->act_sh, c->tmax * c->kmax, c->tmax, T, H, M, K, E, tm, c->tiles_b, nb_max, c->y,
                                          c->ysh, st);
        };
        if (sh_small) { /* one list */
            TLAUNCH(c, ST_GATE_UP, gate_up(GEMM_TILE_SMALL, s), "grouped gate/up");
            TLAUNCH(c, ST_DOWN, down(GEMM_TILE_SMALL, s), "grouped down");
        } else if (c->timing || !c->side) { /* per-stage timing (or no side stream): both lists in order on one stream */
            TLAUNCH(c, ST_GATE_UP, (gate_up(GEMM_TILE_SMALL, s) ? -3 : gate_up(GEMM_TILE_BIG, s)), "grouped gate/up");
            TLAUNCH(c, ST_DOWN, (down(GEMM_TILE_SMALL, s) ? -3 : down(GEMM_TILE_BIG, s)), "grouped down");
        } else {
            /* the lists touch disjoint rows of act and y: the big-tile list
             * runs on the side stream, overlapping the small one's tail */
            HIP_OK(hipEventRecord(c->fork, s), OROME_EHIP);
            HIP_OK(hipStreamWaitEvent(c->side, c->fork, 0), OROME_EHIP);
            LAUNCH(gate_up(GEMM_TILE_BIG, c->side), "grouped gate/up (big tiles)");
            LAUNCH(down(GEMM_TILE_BIG, c->side), "grouped down (big tiles)");
            LAUNCH(gate_up(GEMM_TILE_SMALL, s), "grouped gate/up (small tiles)");
            LAUNCH(down(GEMM_TILE_SMALL, s), "grouped down (small tiles)");
            HIP_OK(hipEventRecord(c->join, c->side), OROME_EHIP);
            HIP_OK(hipStreamWaitEvent(s, c->join, 0), OROME_EHIP);
        }
        if (fuse_next_norm) /* also the next layer's RMSNorm of h_out into xnorm */
            TLAUNCH(c, ST_COMBINE,
                    launch_combine_norm(c->y, c->ysh, c->pos, c->w, c->sgl, S ? 1 : 0, h_in, h_out, fo.res, fo.ssq, T, H, K, next_norm_w,
                                        cfg->rms_norm_eps, c->xnorm, c->x16, s),
                    "combine + next RMSNorm");
        else
            TLAUNCH(c, ST_COMBINE, launch_combine(c->y, c->ysh, c->pos, c->w, c->sgl, S ? 1 : 0, h_in, h_out, fo.res, fo.ssq, T, H, K, s),
                    "combine");
    }
    c->last_T = T;
    c->last_K = K;
    return OROME_OK;
}

static hipStream_t call_stream(const orome_hip_ctx *c, void *stream) {
    return stream ? (hipStream_t)stream : c->stream;
}

extern "C" int orome_moe_forward(orome_hip_ctx *c, const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *elr,
                                 const OromeHipLayerTensorCache *lt, const float *x, const float *h_in, float *h_out,
                                 float *residual_out, float *sumsq_parts, int T, int K, void *stream) {
    if (!c || !x) return orome_fail(OROME_EINVAL, "orome_moe_forward: NULL argument");
    const int rc = forward_impl(c, cfg, elr, lt, x, h_in, h_out, T, K, NULL, NULL, call_stream(c, stream),
                                FwdOut{residual_out, sumsq_parts});
    if (rc) (void)reset_state(c, call_stream(c, stream));
    return rc;
}

extern "C" int orome_moe_layer_forward(orome_hip_ctx *c, const OromeHipModelConfig *cfg,
                                       const OromeHipExpertLayerRef *elr, const OromeHipLayerTensorCache *lt,
                                       float *h, int T, int K, void *stream) {
    if (!c || !cfg || !lt || !h) return orome_fail(OROME_EINVAL, "orome_moe_layer_forward: NULL argument");
    if (T < 1 || T > c->tmax) return orome_fail(OROME_EINVAL, "orome_moe_layer_forward: T=%d", T);
    if (set_dev(c)) return OROME_EHIP;
    const float *nw = lt->post_norm.buffer && lt->post_norm.format == OROME_QFMT_F32
                          ? (const float *)dev_addr(lt->post_norm.buffer, lt->post_norm.offset)
                          : NULL;
    const int rc = forward_impl(c, cfg, elr, lt, NULL, h, h, T, K, h, nw, call_stream(c, stream), FwdOut{NULL, NULL});
    if (rc) (void)reset_state(c, call_stream(c, stream));
    return rc;
}

extern "C" int orome_moe_stack_forward(orome_hip_ctx *c, const OromeHipModelConfig *cfg,
                                       const OromeHipExpertLayerRef *elrs, const OromeHipLayerTensorCache *lts,
                                       int n_layers, float *h, int T, int K, void *stream) {
    if (!elrs || !lts || n_layers < 0) return orome_fail(OROME_EINVAL, "orome_moe_stack_forward: bad arguments");
    if (!c || !cfg || !h) return orome_fail(OROME_EINVAL, "orome_moe_stack_forward: NULL argument");
    if (T < 1 || T > c->tmax) return orome_fail(OROME_EINVAL, "orome_moe_stack_forward: T=%d", T);
    if (set_dev(c)) return OROME_EHIP;
    /* on the MFMA path each layer's combine also computes the next layer's
     * RMSNorm (same bits as the separate norm kernel), which then is skipped */
    /* (AUTO takes the small-batch routing, with the norm in the router, up
     * to 16 tokens) */
    const int path = c->path == OROME_PATH_AUTO ? (T <= 16 ? OROME_PATH_GEMV : OROME_PATH_MFMA) : c->path;
    const bool fuse = path == OROME_PATH_MFMA && cfg->hidden_dim % 512 == 0 && cfg->hidden_dim <= 4096;
    auto norm_w = [&](int l) -> const float * {
        return lts[l].post_norm.buffer && lts[l].post_norm.format == OROME_QFMT_F32
                   ? (const float *)dev_addr(lts[l].post_norm.buffer, lts[l].post_norm.offset)
                   : NULL;
    };
    const hipStream_t s = call_stream(c, stream);
    for (int l = 0; l < n_layers; l++) {
        if (!lts[l].routing_gate.buffer) return orome_fail(OROME_EINVAL, "orome_moe_stack_forward: layer %d", l);
        const bool next = fuse && l + 1 < n_layers;
        FwdOut fo{NULL, NULL};
        /* (only a router the next layer's forward will accept: F32, and
         * [E][H] where the reference gives its shape) */
        const OromeHipTensorRef *nr = l + 1 < n_layers ? &lts[l + 1].routing_gate : NULL;
        if (nr && nr->buffer && nr->format == OROME_QFMT_F32 && (!nr->out_dim || (int)nr->out_dim >= cfg->num_experts) &&
            (!nr->in_dim || (int)nr->in_dim == cfg->hidden_dim))
            fo.next_router = (const float *)dev_addr(lts[l + 1].routing_gate.buffer, lts[l + 1].routing_gate.offset);
        int rc = forward_impl(c, cfg, &elrs[l], &lts[l], NULL, h, h, T, K, h, norm_w(l), s, fo,
                              next ? norm_w(l + 1) : NULL, next ? 1 : 0, fuse && l > 0 ? 1 : 0);
        if (rc) {
            (void)reset_state(c, s);
            return rc;
        }
    }
    return OROME_OK;
}

extern "C" int orome_moe_debug_outputs(orome_hip_ctx *c, float *logits, int32_t *idx, float *w,
                                       uint32_t *offsets, uint32_t *pairs) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_moe_debug_outputs: NULL ctx");
    if (!c->last_T) return orome_fail(OROME_EINVAL, "orome_moe_debug_outputs: no forward yet");
    const size_t T = (size_t)c->last_T, K = (size_t)c->last_K, E = (size_t)c->cfg.num_experts;
    if (set_dev(c)) return OROME_EHIP;
    if (c->last_stream) HIP_OK(hipStreamSynchronize(c->last_stream), OROME_EHIP);
    int rc = 0;
    if (!rc && logits) rc = orome_hip_dtoh(c, logits, c->logits, T * (E + 1) * 4);
    if (!rc && idx) rc = orome_hip_dtoh(c, idx, c->idx, T * K * 4);
    if (!rc && w) rc = orome_hip_dtoh(c, w, c->w, T * K * 4);
    if (!rc && offsets) rc = orome_hip_dtoh(c, offsets, c->offsets, (E + 1) * 4);
    if (!rc && pairs) rc = orome_hip_dtoh(c, pairs, c->pairs, T * K * 4);
    if (!rc) rc = orome_hip_sync(c);
    return rc;
}

extern "C" int orome_moe_topk(orome_hip_ctx *c, const float *logits, const float *bias, int T, int E,
                              int K, int32_t *idx, float *w) {
    if (!c || !logits || !idx || !w) return orome_fail(OROME_EINVAL, "orome_moe_topk: NULL argument");
    if (T < 1 || T > c->tmax || E < 1 || E > 1024 || K < 1 || K > OROME_MAX_ACTIVE || K > E)
        return orome_fail(OROME_EINVAL, "orome_moe_topk: bad shape T=%d E=%d K=%d", T, E, K);
    if (set_dev(c)) return OROME_EHIP;
    RouteArgs a;
    memset(&a, 0, sizeof a);
    a.bias = bias; a.T = T; a.E = E; a.K = K;
    a.logits = (float *)logits; a.idx = idx; a.w = w; a.sgl = c->sgl;
    LAUNCH(launch_topk(a, c->stream), "top-k");
    return OROME_OK;
}

extern "C" int orome_dequant_rows(orome_hip_ctx *c, OromeHipQuantFormat fmt, const void *src, uint32_t rows,
                                  uint32_t in_dim, float *out) {
    if (!c || !src || !out) return orome_fail(OROME_EINVAL, "orome_dequant_rows: NULL argument");
    if (set_dev(c)) return OROME_EHIP;
    LAUNCH(launch_dequant(kfmt(fmt), (const uint8_t *)src, rows, in_dim, out, NULL, c->stream), "dequant");
    return OROME_OK;
}

extern "C" int orome_dequant_rows_f16(orome_hip_ctx *c, OromeHipQuantFormat fmt, const void *src,
                                      uint32_t rows, uint32_t in_dim, uint16_t *out) {
    if (!c || !src || !out) return orome_fail(OROME_EINVAL, "orome_dequant_rows_f16: NULL argument");
    if (set_dev(c)) return OROME_EHIP;
    LAUNCH(launch_dequant(kfmt(fmt), (const uint8_t *)src, rows, in_dim, NULL, (_Float16 *)out, c->stream),
           "dequant f16");
    return OROME_OK;
}

/* one-hot activation rows for orome_debug_mfma_weights: row j is e_j in the
 * (0,2,1,3)-per-4-group storage order of the GEMM sources */
__global__ void k_one_hot_f16(_Float16 *act, int n, int ld) {
    const int j = blockIdx.x;
    for (int i = threadIdx.x; i < ld; i += blockDim.x) act[(size_t)j * ld + i] = (_Float16)0.0f;
    __syncthreads();
    if (threadIdx.x == 0 && j < n) {
        const int perm[4] = {0, 2, 1, 3};
        act[(size_t)j * ld + (j & ~3) + perm[j & 3]] = (_Float16)1.0f;
    }
}

extern "C" int orome_debug_mfma_weights(orome_hip_ctx *c, OromeHipQuantFormat fmt, int tiled, const void *w,
                                        uint32_t rows, uint32_t in_dim, float *out) {
    if (!c || !w || !out) return orome_fail(OROME_EINVAL, "orome_debug_mfma_weights: NULL argument");
    const int H = c->cfg.hidden_dim, M = c->cfg.moe_intermediate;
    const int f = kfmt(fmt);
    if ((int)rows != H || (int)in_dim != M || f < 0 || (tiled && f != 0 && f != 1 && f != 2 && f != 3))
        return orome_fail(OROME_EINVAL, "orome_debug_mfma_weights: a %ux%u %s matrix does not fit", rows, in_dim,
                          tiled ? "tile-major" : "row-major");
    if ((size_t)M > (size_t)c->tmax * c->kmax)
        return orome_fail(OROME_EINVAL, "orome_debug_mfma_weights: context too small for %d one-hot rows", M);
    if (set_dev(c)) return OROME_EHIP;
    hipStream_t s = c->stream;
    void *packed = NULL;
    ExpertSide ex = {};
    ex.down = (const uint8_t *)w;
    ex.down_fmt = f;
    ex.gate_fmt = 0;
    if (tiled) {
        const size_t nb = f == 0 ? packed_q4k_bytes(H, M, 1) : f == 1 ? packed_q5k_bytes(H, M, 1)
                          : f == 2 ? packed_q6k_bytes(H, M, 1) : packed_q8_bytes(H, M, 1);
        HIP_OK(hipMalloc(&packed, nb), OROME_ENOMEM);
        const int rc = (f == 0 ? launch_pack_q4k : f == 1 ? launch_pack_q5k : f == 2 ? launch_pack_q6k : launch_pack_q8)(
            (const uint8_t *)w, (uint8_t *)packed, H, M, 1, 0, s);
        if (rc) {
            (void)hipFree(packed);
            return launch_rc(rc, "orome_debug_mfma_weights: repack");
        }
        ex.down = (const uint8_t *)packed;
        ex.down_fmt = f == 0 ? GEMM_FMT_Q4K_TILED : f == 1 ? GEMM_FMT_Q5K_TILED : f == 2 ? GEMM_FMT_Q6K_TILED : GEMM_FMT_Q8_TILED;
    }
    SharedSide sh = {NULL, NULL, NULL, 0, 0, 0};
    /* M one-hot rows as the pairs of expert 0, in 32-row tiles */
    KLAUNCH(k_one_hot_f16, dim3((unsigned)M), dim3(256), 0, s, c->act, M, M);
    const int ntile = (M + GEMM_TILE_SMALL - 1) / GEMM_TILE_SMALL;
    uint32_t *hl = (uint32_t *)calloc(1 + 3 * (size_t)ntile, 4);
    hl[0] = (uint32_t)ntile;
    for (int t = 0; t < ntile; t++) {
        hl[1 + 3 * t] = 0;
        hl[2 + 3 * t] = (uint32_t)(t * GEMM_TILE_SMALL);
        hl[3 + 3 * t] = (uint32_t)(M - t * GEMM_TILE_SMALL < GEMM_TILE_SMALL ? M - t * GEMM_TILE_SMALL : GEMM_TILE_SMALL);
    }
    hipError_t e = hipMemcpyAsync(c->tiles, hl, (1 + 3 * (size_t)ntile) * 4, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? 0 : -3;
    if (!rc) e = hipStreamSynchronize(s);
    free(hl);
    if (!rc && e == hipSuccess)
        rc = launch_gemm_down(ex, sh, c->act, c->act_sh, c->tmax * c->kmax, c->tmax, M, H, M, 1, 1, GEMM_TILE_SMALL,
                              c->tiles, ntile, c->y, c->ysh, s);
    if (!rc) e = hipMemcpyAsync(out, c->y, (size_t)M * H * 4, hipMemcpyDeviceToDevice, s);
    if (!rc && e == hipSuccess) e = hipStreamSynchronize(s);
    if (packed) (void)hipFree(packed);
    if (rc) return launch_rc(rc, "orome_debug_mfma_weights: grouped down GEMM");
    if (e != hipSuccess) return orome_fail(OROME_EHIP, "orome_debug_mfma_weights: %s", hipGetErrorString(e));
    return OROME_OK;
}

extern "C" int orome_hip_debug_inject_failure(orome_hip_ctx *c) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_hip_debug_inject_failure: NULL ctx");
    c->inject = 1;
    return OROME_OK;
}

/* ------------------------------------------------------- graphs, timing */

extern "C" int orome_hip_capture_begin(orome_hip_ctx *c) {
    if (!c) return orome_fail(OROME_EINVAL, "orome_hip_capture_begin: NULL ctx");
    if (c->timing) return orome_fail(OROME_EINVAL, "stage timing must be off while capturing");
    if (set_dev(c)) return OROME_EHIP;
    /* the graph starts from a clean counter whatever ran before */
    if (reset_state(c, c->stream)) return OROME_EHIP;
    HIP_OK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_capture_end(orome_hip_ctx *c, void **exec) {
    if (!c || !exec) return orome_fail(OROME_EINVAL, "orome_hip_capture_end: NULL argument");
    hipGraph_t g = NULL;
    HIP_OK(hipStreamEndCapture(c->stream, &g), OROME_EHIP);
    hipGraphExec_t ge = NULL;
    hipError_t e = hipGraphInstantiate(&ge, g, NULL, NULL, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return orome_fail(OROME_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *exec = (void *)ge;
    return OROME_OK;
}

extern "C" int orome_hip_graph_launch(orome_hip_ctx *c, void *exec) {
    if (!c || !exec) return orome_fail(OROME_EINVAL, "orome_hip_graph_launch: NULL argument");
    HIP_OK(hipGraphLaunch((hipGraphExec_t)exec, c->stream), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_graph_destroy(void *exec) {
    if (exec) HIP_OK(hipGraphExecDestroy((hipGraphExec_t)exec), OROME_EHIP);
    return OROME_OK;
}

extern "C" int orome_hip_stage_timing(orome_hip_ctx *c, int capacity) {
    if (!c || capacity < 0) return orome_fail(OROME_EINVAL, "orome_hip_stage_timing: bad argument");
    if (set_dev(c)) return OROME_EHIP;
    (void)hipStreamSynchronize(c->stream);
    free_timing(c);
    memset(c->tcount, 0, sizeof c->tcount);
    if (!capacity) return OROME_OK;
    c->ev = (hipEvent_t *)calloc((size_t)N_STAGES * capacity * 2, sizeof(hipEvent_t));
    for (int i = 0; i < N_STAGES * capacity * 2; i++)
        HIP_OK(hipEventCreate(&c->ev[i]), OROME_EHIP);
    c->tcap = capacity;
    c->timing = 1;
    return OROME_OK;
}

extern "C" int orome_hip_stage_times(orome_hip_ctx *c, float *total_ms, int *counts, int n) {
    if (!c || !total_ms || !counts || n < 1) return orome_fail(OROME_EINVAL, "orome_hip_stage_times: bad argument");
    HIP_OK(hipStreamSynchronize(c->stream), OROME_EHIP);
    for (int st = 0; st < n; st++) {
        total_ms[st] = 0.0f;
        counts[st] = 0;
        if (st >= N_STAGES || !c->timing) continue;
        int k = c->tcount[st] < c->tcap ? c->tcount[st] : c->tcap;
        for (int i = 0; i < k; i++) {
            float ms = 0.0f;
            HIP_OK(hipEventElapsedTime(&ms, c->ev[(st * c->tcap + i) * 2], c->ev[(st * c->tcap + i) * 2 + 1]),
                   OROME_EHIP);
            total_ms[st] += ms;
        }
        counts[st] = k;
    }
    return OROME_OK;
}

extern "C" int orome_hip_stream_delay(orome_hip_ctx *c, uint32_t usec) {
    if (!c || usec > 10000000u) return orome_fail(OROME_EINVAL, "orome_hip_stream_delay: bad argument");
    if (set_dev(c)) return OROME_EHIP;
    LAUNCH(launch_delay(usec, c->stream), "delay");
    return OROME_OK;
}

/* ------------------------------------------- forward without allocation */

/* The scratch of orome_moe_forward_noalloc: one copy per GPU, held until the
 * process ends.  Host code must not use this name as a device address (it is
 * the host-side stand-in of the symbol); each device's address comes from
 * hipGetSymbolAddress on that device, kept in g_na_ptr. */
static __device__ __align__(256) uint8_t scratch[OROME_NOALLOC_SCRATCH_BYTES];

#define NA_MAX_DEVICES 64
static std::mutex g_na_lock;
static uint8_t *g_na_ptr[NA_MAX_DEVICES];
/* shapes of the layout the device's scratch was last cleared for */
static int g_na_key[NA_MAX_DEVICES][4];

extern "C" int orome_moe_forward_noalloc(const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *elr,
                                         const OromeHipLayerTensorCache *lt, const float *x, const float *h_in,
                                         float *h_out, float *residual_out, float *sumsq_parts, int T, int K,
                                         void *stream) {
    if (!cfg || !elr || !lt || !x || !h_out) return orome_fail(OROME_EINVAL, "orome_moe_forward_noalloc: NULL argument");
    if (T < 1 || T > OROME_NOALLOC_MAX_TOKENS)
        return orome_fail(OROME_EINVAL, "orome_moe_forward_noalloc: T=%d outside 1..%d", T, OROME_NOALLOC_MAX_TOKENS);
    if (cfg->hidden_dim <= 0 || cfg->num_experts <= 0 || cfg->moe_intermediate <= 0 || cfg->shared_intermediate < 0)
        return orome_fail(OROME_EINVAL, "orome_moe_forward_noalloc: invalid config");
    int dev = 0;
    HIP_OK(hipGetDevice(&dev), OROME_EHIP);
    if (dev < 0 || dev >= NA_MAX_DEVICES) return orome_fail(OROME_EINVAL, "orome_moe_forward_noalloc: device %d", dev);
    /* a context on the stack: no streams, events or packs of its own */
    orome_hip_ctx c = {};
    c.device = dev;
    c.stream = stream ? (hipStream_t)stream : 0;
    c.cfg = *cfg;
    c.tmax = OROME_NOALLOC_MAX_TOKENS;
    c.kmax = OROME_MAX_ACTIVE;
    c.path = OROME_PATH_AUTO;
    const size_t need = scratch_layout(&c, NULL);
    if (need > sizeof(scratch))
        return orome_fail(OROME_EINVAL, "orome_moe_forward_noalloc: shapes need %zu bytes of scratch, the maximum is %zu",
                          need, sizeof(scratch));
    const int key[4] = {cfg->hidden_dim, cfg->num_experts, cfg->moe_intermediate, cfg->shared_intermediate};
    uint8_t *base;
    bool clear = false;
    {
        std::lock_guard<std::mutex> g(g_na_lock);
        if (!g_na_ptr[dev]) {
            void *p = NULL;
            HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), OROME_EHIP);
            g_na_ptr[dev] = (uint8_t *)p;
        }
        base = g_na_ptr[dev];
        /* the zero rows of the layout sit at shape-dependent offsets: clear
         * the scratch whenever the shapes change (and on the first call) */
        clear = memcmp(g_na_key[dev], key, sizeof key) != 0;
    }
    /* the key is recorded only once the clear is queued, and forgotten when
     * a call fails, so the next call clears the array (zero rows and the
     * router's arrival counter) again */
    auto forget = [&]() {
        std::lock_guard<std::mutex> g(g_na_lock);
        memset(g_na_key[dev], 0, sizeof g_na_key[dev]);
    };
    if (clear) {
        const int rc = launch_rc(launch_zero(base, need, c.stream), "orome_moe_forward_noalloc: scratch clear");
        if (rc) {
            forget();
            return rc;
        }
        std::lock_guard<std::mutex> g(g_na_lock);
        memcpy(g_na_key[dev], key, sizeof key);
    }
    scratch_layout(&c, base);
    const int rc = forward_impl(&c, cfg, elr, lt, x, h_in, h_out, T, K, NULL, NULL, c.stream, FwdOut{residual_out, sumsq_parts});
    if (rc) forget();
    return rc;
}
