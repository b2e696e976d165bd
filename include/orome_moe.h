/*
 * orome_moe.h -- C ABI of the MI355X (gfx950) MoE feed-forward library.
 *
 * Drop-in boundary for Orome's MoE hot path.  The types carry the fields of
 * the C subset of the reference's interfaces (inference/include/orome.h) with
 * the Metal handles replaced by HIP device pointers; the functions replace the
 * reference's GGUF loader, weight-format layer, GPU context and the MoE
 * encoder (encode_experts_gguf).  Every declaration names the reference
 * interface it replaces as path:line relative to the reference repository.
 *
 * Every exported type, enumerator and function carries an OromeHip / OROME_ /
 * orome_ prefix, so this header and the reference's orome.h can be included in
 * one translation unit and both libraries linked into one engine: the
 * reference's ModelConfig, TensorRef, GGUFFile, gguf_open, ... keep their own
 * layouts and symbols, and the engine copies the MoE fields across once at
 * load time.  Enumerator values equal the reference's (QuantFormat, FFNType).
 *
 * Conventions
 *   - Return codes: OROME_OK (0) or a negative OROME_E* code; a message is
 *     printed to stderr with the tag "[hip]" and kept for orome_last_error().
 *     The reference returns NULL/false and prints "[tag] ..."
 *     (inference/src/metal.m:44-56, inference/src/gguf.m:274-308).
 *   - All device pointers are HBM addresses from this library's allocator
 *     (or any hipMalloc'd memory on the context's device).
 *   - A context owns one HIP stream; forward calls are asynchronous on it (or
 *     on a stream the caller passes) and orome_hip_sync() waits.  A context is not thread-safe (the reference is
 *     single-threaded too: inference/src/metal.m:51).
 */
#ifndef OROME_MOE_H
#define OROME_MOE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

/* inference/include/orome.h:29 -- upper bound on active experts per token
 * (the same definition, so both headers may be included together). */
#ifndef OROME_MAX_ACTIVE
#define OROME_MAX_ACTIVE 16
#endif

enum {
    OROME_OK = 0,
    OROME_EINVAL = -1,      /* bad argument or shape */
    OROME_EUNSUPPORTED = -2,/* format / shape not handled by a kernel */
    OROME_EHIP = -3,        /* HIP runtime error */
    OROME_ENOMEM = -4,      /* allocation failed */
    OROME_ENOTFOUND = -5,   /* missing tensor or file */
    OROME_EFORMAT = -6,     /* malformed GGUF */
};

/* inference/include/orome.h:40-43 */
typedef enum { OROME_FFN_MOE, OROME_FFN_DENSE } OromeHipFFNType;

/* MoE-path subset of the reference's ModelConfig (inference/include/orome.h:49-98);
 * field names and meanings are the reference's. */
typedef struct {
    char name[64];
    int hidden_dim;           /* H, e.g. 2048 */
    int num_layers;
    float rms_norm_eps;       /* e.g. 1e-6 */
    OromeHipFFNType ffn_type;
    int num_experts;          /* E, e.g. 256 */
    int num_experts_per_tok;  /* K, e.g. 8 */
    int moe_intermediate;     /* M, e.g. 512 */
    int shared_intermediate;  /* S, e.g. 512; 0 = no shared expert */
} OromeHipModelConfig;

/* inference/include/orome.h:227-235 (same values, same order). */
typedef enum {
    OROME_QFMT_GGUF_Q4_K,
    OROME_QFMT_GGUF_Q5_K,
    OROME_QFMT_GGUF_Q6_K,
    OROME_QFMT_GGUF_Q8_0,
    OROME_QFMT_F16,
    OROME_QFMT_BF16,
    OROME_QFMT_F32,
} OromeHipQuantFormat;

/* inference/include/orome.h:239-246.  `buffer` is the device base of the
 * uploaded GGUF data (it was an id<MTLBuffer>); `offset` is the same GGUF byte
 * offset (data_offset + tensor offset, relative to the file start).  The
 * reference's `pipeline` is dropped: `format` selects the kernel. */
typedef struct {
    void *buffer;
    size_t offset;
    OromeHipQuantFormat format;
    uint32_t out_dim;
    uint32_t in_dim;
} OromeHipTensorRef;

/* inference/include/orome.h:249-254 */
typedef struct {
    size_t offset;
    size_t expert_stride;
    OromeHipQuantFormat format;
} OromeHipExpertProjRef;

/* inference/include/orome.h:256-259 */
typedef struct {
    void *buffer;
    OromeHipExpertProjRef gate, up, down;
} OromeHipExpertLayerRef;

/* MoE subset of the reference's LayerTensorCache (inference/include/orome.h:264-279), plus
 * `routing_bias`: an optional fp32 [E] bias added to the router logits
 * before top-k (synthetic skewed-routing workloads; a zeroed ref = none). */
typedef struct {
    OromeHipTensorRef post_norm;           /* F32 [H]; truncated to bf16 when applied */
    OromeHipTensorRef routing_gate;        /* F32 [E x H] */
    OromeHipTensorRef shared_gate;         /* Q4_K/Q8_0 [S x H] */
    OromeHipTensorRef shared_up;           /* Q4_K/Q8_0 [S x H] */
    OromeHipTensorRef shared_down;         /* Q4_K/Q6_K/Q8_0 [H x S] */
    OromeHipTensorRef shared_expert_gate;  /* F32 [1 x H] */
    OromeHipTensorRef routing_bias;        /* F32 [E] or empty */
} OromeHipLayerTensorCache;

/* ------------------------------------------------------------------ GGUF */

/* inference/include/orome.h:415-421 */
typedef struct OromeHipGGUFTensorInfo {
    char *name;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;    /* ggml type id */
    uint64_t offset;  /* relative to the data section */
} OromeHipGGUFTensorInfo;

/* MoE subset of the reference's GGUFFile (inference/include/orome.h:423-437). */
typedef struct OromeHipGGUFFile {
    int fd;                 /* -1 for an in-memory image */
    void *mmap_base;        /* start of the image */
    size_t file_size;
    size_t data_offset;     /* absolute offset of the tensor data section */
    OromeHipGGUFTensorInfo *tensors;
    uint64_t num_tensors;
    uint32_t alignment;
    char arch[32];
    OromeHipFFNType ffn_type;
    int num_layers, hidden_dim, num_experts, num_experts_per_tok, moe_intermediate;
    float rms_norm_eps;
    void *index;            /* private name index */
    bool owns_map;
    int q4k_layout;         /* OROME_Q4K_LAYOUT_* the file declares (REFERENCE if silent) */
} OromeHipGGUFFile;

/* Q4_K scale/min packing of a file's Q4_K tensors.  The reference decodes
 * sub-blocks 4..7 from scale bytes 8..11 as: scales 4,5 = the low/high
 * nibbles of byte 8, scales 6,7 of byte 9, mins 4,5 of byte 10, mins 6,7 of
 * byte 11 (inference/src/format.m:41-64).  ggml/llama.cpp files pack byte
 * 8 + j as scale 4+j (low nibble) | min 4+j (high nibble)
 * (get_scale_min_k4; the reference's own llama-style kernel,
 * inference/src/shaders.metal:1575-1578).  The high 2-bit parts agree.  A
 * file declares ggml packing with the string metadata key
 * OROME_Q4K_LAYOUT_KEY = "ggml" (or "reference"); the kernels decode the
 * reference packing only, and a ggml-packed file has bytes 8..11 of every
 * Q4_K block permuted into it once, on the device, at upload. */
#define OROME_Q4K_LAYOUT_KEY "orome.q4_k.scale_layout"
enum { OROME_Q4K_LAYOUT_FILE = 0, OROME_Q4K_LAYOUT_REFERENCE = 1, OROME_Q4K_LAYOUT_GGML = 2 };

/* inference/src/gguf.m:273-518 (mmap + parse; v2/v3; alignment rule 511-512) */
OromeHipGGUFFile *orome_hip_gguf_open(const char *path);
/* Same parser over an image already in host memory (not copied; must outlive
 * the OromeHipGGUFFile).  No counterpart in the reference (it only maps files). */
OromeHipGGUFFile *orome_hip_gguf_open_memory(const void *data, size_t size);
/* inference/src/gguf.m:520-531 */
void orome_hip_gguf_close(OromeHipGGUFFile *gf);
/* inference/src/gguf.m:533-537 */
OromeHipGGUFTensorInfo *orome_hip_gguf_find_tensor(OromeHipGGUFFile *gf, const char *name);
/* inference/src/gguf.m:540-550 */
size_t orome_hip_gguf_tensor_size(const OromeHipGGUFTensorInfo *ti);
/* inference/src/gguf.m:552-575 */
const char *orome_hip_ggml_type_name(uint32_t type);
/* inference/src/format.m:326-337.  Unknown types are an error here
 * (OROME_EUNSUPPORTED) instead of the reference's silent Q4_K fallback. */
int orome_hip_format_from_ggml_type(uint32_t ggml_type, OromeHipQuantFormat *out);
/* The MoE fields of ModelConfig read from GGUF metadata and tensor shapes
 * (inference/src/main.m:443-633, shared_intermediate at 576-588). */
int orome_hip_model_config_from_gguf(const OromeHipGGUFFile *gf, OromeHipModelConfig *cfg);

/* ---------------------------------------------------------- HIP context */

/* Replaces MetalCtx + metal_setup/metal_free (inference/include/orome.h:125-221,
 * inference/src/metal.m:41-256, 321-328): binds a device, creates the stream,
 * and sizes the scratch arena for up to `max_tokens` tokens per call. */
typedef struct orome_hip_ctx orome_hip_ctx;
orome_hip_ctx *orome_hip_create(const OromeHipModelConfig *cfg, int max_tokens, int device);
void orome_hip_destroy(orome_hip_ctx *ctx);
int orome_hip_sync(orome_hip_ctx *ctx);
void *orome_hip_get_stream(orome_hip_ctx *ctx);   /* hipStream_t */
const char *orome_last_error(void);

/* Kernel path for orome_moe_forward.  AUTO: the GEMV kernels for 1-2 tokens
 * (routing folded into gate/up), the small-batch routing with the small-tile
 * grouped MFMA GEMMs for 3..16 tokens (T K <= 256; where those GEMMs do not
 * take the shapes, the GEMV kernels up to 8 tokens and the MFMA path above),
 * the large-batch routing and grouped GEMMs above 16.
 * GEMV and MFMA force one kernel family for every T (GEMV: T <= 8). */
enum { OROME_PATH_AUTO = 0, OROME_PATH_GEMV = 1, OROME_PATH_MFMA = 2 };
int orome_hip_set_path(orome_hip_ctx *ctx, int path);

/* Tile-major copies of a layer's expert matrices for the MFMA path.  No
 * counterpart in the reference (its kernels read the GGUF blocks in place):
 * registering a layer declares its weights immutable while registered and
 * repacks, into one allocation on the context's device (the same bytes as the
 * originals), the routed gate/up (Q4_K), the routed down when Q4_K, Q5_K or
 * Q6_K, the shared gate/up when Q4_K or Q8_0 (the reference's 35B layout has
 * a Q8_0 shared expert), and, beside a repacked routed down, the shared down
 * (Q4_K, Q5_K, Q6_K or Q8_0).  orome_moe_forward then feeds the grouped GEMMs
 * from the copies, so each wave's weight loads are contiguous 1-2 KB runs.
 * Outputs are bit-identical with and without.  Layers are keyed by the routed
 * gate and shared gate addresses; registering again replaces the copy.  With
 * an F32 router (any shared-expert format) the copy also holds the router as
 * fp16 rows (one power-of-two scale each) and row-norm bounds: above 16
 * tokens under AUTO (at any T on the forced MFMA path) a registered layer is
 * routed in two passes (approximate logits on the matrix cores, then the
 * canonical fp32 logits of the experts that can win), which selects exactly
 * the experts, order and weights of the one-pass router; the debug logits
 * output then holds the canonical values for those candidates and the
 * approximation (within its proven bound) elsewhere.  OROME_ROUTE_EXACT=1 in
 * the environment keeps the one-pass router.  Fails with OROME_EUNSUPPORTED
 * (nothing registered) when the routed gate/up is not Q4_K or a dimension is
 * not a multiple of 256.
 * orome_hip_unpack_all frees every copy (orome_hip_destroy calls it). */
int orome_hip_pack_layer(orome_hip_ctx *ctx, const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *layer,
                         const OromeHipLayerTensorCache *lt);
int orome_hip_unpack_all(orome_hip_ctx *ctx);

/* Launch timing of the gate/up stage for measurement tools (no counterpart in
 * the reference): with `stamps` set (device memory of 2 * blocks 64-bit words,
 * or NULL to stop), each gate/up kernel block b writes its start and end time
 * (s_memrealtime, 100 MHz) to stamps[2 b] and stamps[2 b + 1]; on the MFMA
 * path the big-tile launch uses blocks [0, blocks/2) and the small-tile one
 * [blocks/2, blocks).  A launch whose grid does not fit writes nothing.  The
 * launch's duration is max(end) - min(start) over the blocks written. */
int orome_hip_kernel_timing(orome_hip_ctx *ctx, unsigned long long *stamps, int blocks);

/* Device memory plumbing on the context's device. */
void *orome_hip_malloc(orome_hip_ctx *ctx, size_t bytes);
int orome_hip_free(orome_hip_ctx *ctx, void *p);
int orome_hip_htod(orome_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int orome_hip_dtoh(orome_hip_ctx *ctx, void *dst, const void *src, size_t bytes);

/* -------------------------------------------------- weight format layer */

/* inference/include/orome.h:262-265 (FormatProvider).  model_buf is the HBM
 * copy of the GGUF image from data_offset on; device addresses are
 * model_buf + (gguf offset - data_offset). */
typedef struct {
    OromeHipGGUFFile *gguf;
    void *model_buf;      /* device base, already shifted so that
                             model_buf + gguf_offset addresses the tensor */
    void *alloc_base;     /* the allocation itself */
    size_t model_bytes;
    orome_hip_ctx *ctx;
} OromeHipFormatProvider;

/* inference/src/format.m:343-363: the reference wraps the mmap without a copy
 * (unified memory); here the data section is copied unchanged into one HBM
 * allocation, so the same GGUF bytes feed the kernels. */
OromeHipFormatProvider *orome_hip_format_provider_open_gguf(OromeHipGGUFFile *gf, orome_hip_ctx *ctx);
/* The same with the Q4_K packing given by the caller (OROME_Q4K_LAYOUT_*;
 * FILE = what the file declares, as orome_hip_format_provider_open_gguf
 * does).  No counterpart in the reference, which has one packing. */
OromeHipFormatProvider *orome_hip_format_provider_open_gguf_layout(OromeHipGGUFFile *gf, orome_hip_ctx *ctx,
                                                                   int q4k_layout);
/* inference/src/format.m:365-369 */
void orome_hip_format_provider_close(OromeHipFormatProvider *fp);
/* inference/src/format.m:374-409.  A missing tensor leaves a zeroed ref. */
OromeHipExpertLayerRef orome_hip_format_resolve_expert_layer(OromeHipFormatProvider *fp, int layer_idx,
                                           uint32_t num_experts);
/* MoE part of build_tensor_cache_gguf (inference/src/format.m:458-590,
 * MoE refs 495-509).  Returns cfg->num_layers entries; free with
 * orome_hip_free_tensor_cache(). */
OromeHipLayerTensorCache *orome_hip_build_tensor_cache_gguf(OromeHipFormatProvider *fp, const OromeHipModelConfig *cfg);
void orome_hip_free_tensor_cache(OromeHipLayerTensorCache *cache);

/* ------------------------------------------------------------ MoE block */

/* One MoE feed-forward block for T tokens.
 * Replaces the routing matvec (inference/src/engine.m:656-685) plus
 * encode_experts_gguf (inference/src/engine.m:158-340) with its final
 * moe_combine_copy_sq_k8 (inference/src/shaders.metal:1079-1135):
 *   logits = [W_r x ; w_sg x]   (fp32, fixed reduction order)
 *   idx, w = top-K of logits (+routing_bias), renormalised softmax
 *   h_out  = (h_in + sum_k w_k E_idx_k(x)) + sigmoid(w_sg x) * S(x)
 * x_dev: fp32 [T x H] normalised input.  h_in_dev: fp32 [T x H] residual or
 * NULL (zero).  h_out_dev may alias h_in_dev.  K <= OROME_MAX_ACTIVE.
 * The combine's other two outputs, as the reference's kernel writes them:
 *   residual_out_dev  fp32 [T x H] copy of h_out (NULL: not written);
 *   sumsq_parts_dev   fp32 [T x H/256]: part b of token t is the sum of
 *                     h_out[t][j]^2 over j in [256 b, 256 b + 256), summed
 *                     in the canonical order of the router's dots (lane L of
 *                     a wave64 owns j = 256 b + 4 L + c, fma over c from
 *                     zero, then the contiguous balanced tree over lanes);
 *                     the next RMSNorm adds the parts (NULL: not written).
 * stream: a hipStream_t on the context's device, or NULL for the context's
 * own stream; the call is asynchronous on it. */
int orome_moe_forward(orome_hip_ctx *ctx, const OromeHipModelConfig *cfg,
                      const OromeHipExpertLayerRef *elr, const OromeHipLayerTensorCache *lt,
                      const float *x_dev, const float *h_in_dev, float *h_out_dev,
                      float *residual_out_dev, float *sumsq_parts_dev, int T, int K, void *stream);

/* RMSNorm (post_norm, bf16-truncated weights) then the MoE block with the
 * residual add, in place on h_dev [T x H]: h = h + MoE(RMSNorm(h)).
 * The reference fuses the same norm into the previous combine
 * (inference/src/shaders.metal:90-149, 1079-1135; inference/src/engine.m:627-653).
 * stream as for orome_moe_forward. */
int orome_moe_layer_forward(orome_hip_ctx *ctx, const OromeHipModelConfig *cfg,
                            const OromeHipExpertLayerRef *elr, const OromeHipLayerTensorCache *lt,
                            float *h_dev, int T, int K, void *stream);

/* n_layers consecutive orome_moe_layer_forward calls (the per-layer loop of
 * engine_step restricted to the FFN blocks, inference/src/engine.m:481-694).
 * stream as for orome_moe_forward. */
int orome_moe_stack_forward(orome_hip_ctx *ctx, const OromeHipModelConfig *cfg,
                            const OromeHipExpertLayerRef *elrs, const OromeHipLayerTensorCache *lts,
                            int n_layers, float *h_dev, int T, int K, void *stream);

/* No counterpart in the reference: orome_moe_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  It needs no context and calls no
 * hipMalloc/hipFree or other allocating routine: its scratch is one static
 * device array of OROME_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends.  The device is the calling thread's current one; `stream` (NULL: the
 * null stream) must belong to it.  Same arguments, semantics and results as
 * orome_moe_forward with the default (AUTO) kernel path and unregistered
 * layers, for T <= OROME_NOALLOC_MAX_TOKENS; shapes whose scratch layout
 * exceeds the array, and larger T, are rejected with OROME_EINVAL.  All calls
 * on one GPU share that GPU's array and it keeps the last call's contents:
 * calls that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller.  The array is cleared (by a fill kernel on
 * `stream`) on the first call, whenever the shapes (H, E, M, S) differ from
 * the previous call's, and after a call that failed; its zero rows sit at
 * shape-dependent offsets.  So a HIP graph that captured a call stays valid
 * only while no call with other shapes runs on that GPU between its
 * replays. */
#define OROME_NOALLOC_MAX_TOKENS 16
#define OROME_NOALLOC_SCRATCH_BYTES (8u << 20)
int orome_moe_forward_noalloc(const OromeHipModelConfig *cfg, const OromeHipExpertLayerRef *elr,
                              const OromeHipLayerTensorCache *lt, const float *x_dev,
                              const float *h_in_dev, float *h_out_dev, float *residual_out_dev,
                              float *sumsq_parts_dev, int T, int K, void *stream);

/* Parity hooks: copy the intermediates of the most recent forward to host
 * memory (synchronises the stream that forward ran on).  Any pointer may be NULL.
 *   logits  [T x (E+1)]  router logits, slot E = shared-gate logit
 *   idx     [T x K]      expert indices, descending logit per token
 *   w       [T x K]      renormalised weights
 *   offsets [E+1]        dispatch run starts, pairs[offsets[e]..offsets[e+1])
 *   pairs   [T x K]      expert-sorted pair ids p = t*K + k (stable in p) */
int orome_moe_debug_outputs(orome_hip_ctx *ctx, float *logits, int32_t *idx, float *w,
                            uint32_t *offsets, uint32_t *pairs);

/* Top-k routing alone on given logits [T x (E+1)] (device), for teacher-forced
 * parity of the selection (restates inference/src/shaders.metal:1141-1234).
 * Outputs are device pointers; bias_dev may be NULL. */
int orome_moe_topk(orome_hip_ctx *ctx, const float *logits_dev, const float *bias_dev, int T,
                   int E, int K, int32_t *idx_dev, float *w_dev);

/* Scalar dequant of `rows` rows of `in_dim` weights to fp32 on the GPU
 * (format_decode_row_f32, inference/src/format.m:176-218; bit-exact). */
int orome_dequant_rows(orome_hip_ctx *ctx, OromeHipQuantFormat fmt, const void *src_dev, uint32_t rows,
                       uint32_t in_dim, float *out_dev);

/* fp16(dequant(w)) rounded to nearest even, [rows x in_dim] (the scalar
 * dequant above, then one rounding).  For Q8_0 and for Q6_K with
 * |q sc| <= 2048 these are the MFMA path's weights; Q4_K and Q5_K there
 * round d sc q - fp16(dmin m) once, which can differ by one ulp
 * (orome_debug_mfma_weights returns the MFMA path's own values). */
int orome_dequant_rows_f16(orome_hip_ctx *ctx, OromeHipQuantFormat fmt, const void *src_dev,
                           uint32_t rows, uint32_t in_dim, uint16_t *out_dev);

/* The fp16 weights the grouped GEMMs feed to the matrix cores, read back
 * through the real down-projection GEMM: one matrix [rows x in_dim]
 * (rows = the context's hidden size, in_dim = its expert intermediate size)
 * of `fmt` (Q4_K, Q5_K, Q6_K, Q8_0) is multiplied by in_dim one-hot fp16
 * activation rows, so out_dev[j][r] = the fp16 weight (r, j) the matrix cores
 * used, exactly (products with 1, sums of zeros).  tiled: repack it first
 * (any of the four) as orome_hip_pack_layer does and read the tile-major copy.
 * out_dev: fp32 [in_dim x rows].  For tests; not thread-safe with forward
 * calls on the context (it uses the context's scratch).  No counterpart in
 * the reference. */
int orome_debug_mfma_weights(orome_hip_ctx *ctx, OromeHipQuantFormat fmt, int tiled, const void *w_dev,
                             uint32_t rows, uint32_t in_dim, float *out_dev);

/* Test hook for the error path: the next forward call on the context that
 * takes the small-batch routing (1..16 tokens) fails right after its router
 * launch, having first set the router's arrival counter to a torn value (as
 * a forward interrupted between launches could leave it).  Every forward
 * entry point that fails returns the kernel-carried state to its initial
 * value before it returns, so the following call computes normally.  No
 * counterpart in the reference. */
int orome_hip_debug_inject_failure(orome_hip_ctx *ctx);

/* ------------------------------------------------- graphs and timing */

/* Capture the work queued on the context stream into a HIP graph and replay
 * it.  Counterpart of the reference's one command buffer per token, encoded
 * once and committed (inference/src/engine.m:453-454, 1048-1050); a graph
 * removes per-kernel launch cost from decode.  Forward calls made between
 * begin and end are recorded, not executed.  No memset nodes are recorded:
 * the forward path clears nothing with hipMemset.  capture_begin first
 * resets the scratch state kernels carry between forwards (a fill kernel
 * queued before the capture starts). */
int orome_hip_capture_begin(orome_hip_ctx *ctx);
int orome_hip_capture_end(orome_hip_ctx *ctx, void **graph_exec);
int orome_hip_graph_launch(orome_hip_ctx *ctx, void *graph_exec);
int orome_hip_graph_destroy(void *graph_exec);

/* Per-stage kernel timing of eager (not captured) forward calls with HIP
 * events on the launches themselves (hipExtLaunchKernel: the first kernel of
 * a stage records the start event when it begins, each records the stop
 * event when it ends, so a pair spans the stage's kernels as a kernel trace
 * does); `capacity` samples are kept per stage (0 turns timing off).  While
 * timing is on, the two tile lists of the MFMA path run one after the other
 * on the context stream.  Replaces the reference's CPU-side [profile]
 * timers (inference/src/engine.m:687-693, 1063-1068), which measured
 * encode time rather than GPU time.  Stages: 0 norm, 1 router, 2 top-k,
 * 3 dispatch, 4 fp16 staging, 5 gate/up, 6 down, 7 combine. */
#define OROME_N_STAGES 8
int orome_hip_stage_timing(orome_hip_ctx *ctx, int capacity);
/* Queue a bounded GPU busy-wait of `usec` microseconds (<= 10 s) on the
 * context stream, so that work queued behind it runs back to back and event
 * pairs bracket kernels rather than host launch gaps.  No counterpart in the
 * reference. */
int orome_hip_stream_delay(orome_hip_ctx *ctx, uint32_t usec);
/* total milliseconds and sample counts per stage since timing was enabled */
int orome_hip_stage_times(orome_hip_ctx *ctx, float *total_ms, int *counts, int n);

/* Library version string. */
const char *orome_version(void);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif /* OROME_MOE_H */
