/*
 * format.c -- weight-format layer: GGUF tensors -> HBM-resident TensorRefs.
 *
 * Mirrors the reference's OromeHipFormatProvider / tensor cache
 * (inference/src/format.m:326-409, 458-590) for the MoE block.  The reference
 * wraps the whole GGUF mmap as one Metal buffer without copying (unified
 * memory, format.m:343-363); MI355X memory is discrete, so the data section
 * is copied once, byte for byte, into one HBM allocation and every ref keeps
 * the GGUF byte offset it had in the file.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "orome_internal.h"
#include "orome_moe.h"

OromeHipFormatProvider *orome_hip_format_provider_open_gguf_layout(OromeHipGGUFFile *gf, orome_hip_ctx *ctx,
                                                                   int q4k_layout) {
    if (!gf || !ctx || q4k_layout < OROME_Q4K_LAYOUT_FILE || q4k_layout > OROME_Q4K_LAYOUT_GGML) {
        orome_fail(OROME_EINVAL, "orome_hip_format_provider_open_gguf: bad argument");
        return NULL;
    }
    const int layout = q4k_layout == OROME_Q4K_LAYOUT_FILE ? gf->q4k_layout : q4k_layout;
    size_t bytes = gf->file_size - gf->data_offset;
    void *dev = orome_hip_malloc(ctx, bytes ? bytes : 1);
    if (!dev) return NULL;
    if (bytes && orome_hip_htod(ctx, dev, (const uint8_t *)gf->mmap_base + gf->data_offset, bytes)) {
        orome_hip_free(ctx, dev);
        return NULL;
    }
    /* ggml-packed Q4_K tensors: bytes 8..11 of each block's scales into the
     * reference packing the kernels decode (a byte permutation, once) */
    for (uint64_t i = 0; layout == OROME_Q4K_LAYOUT_GGML && i < gf->num_tensors; i++) {
        const OromeHipGGUFTensorInfo *ti = &gf->tensors[i];
        if (ti->type != 12) continue; /* ggml type id of Q4_K */
        const size_t nb = orome_hip_gguf_tensor_size(ti) / 144;
        if (nb && orome_hip_q4k_ggml_to_reference(ctx, (uint8_t *)dev + ti->offset, nb)) {
            orome_hip_free(ctx, dev);
            return NULL;
        }
    }
    OromeHipFormatProvider *fp = calloc(1, sizeof *fp);
    fp->gguf = gf;
    fp->alloc_base = dev;
    /* model_buf + (data_offset + tensor offset) == device address of the tensor */
    fp->model_buf = (uint8_t *)dev - gf->data_offset;
    fp->model_bytes = bytes;
    fp->ctx = ctx;
    return fp;
}

OromeHipFormatProvider *orome_hip_format_provider_open_gguf(OromeHipGGUFFile *gf, orome_hip_ctx *ctx) {
    return orome_hip_format_provider_open_gguf_layout(gf, ctx, OROME_Q4K_LAYOUT_FILE);
}

void orome_hip_format_provider_close(OromeHipFormatProvider *fp) {
    if (!fp) return;
    if (fp->alloc_base) orome_hip_free(fp->ctx, fp->alloc_base);
    free(fp);
}

static int proj(OromeHipFormatProvider *fp, const char *name, uint32_t E, OromeHipExpertProjRef *out) {
    OromeHipGGUFTensorInfo *ti = orome_hip_gguf_find_tensor(fp->gguf, name);
    if (!ti) return OROME_ENOTFOUND;
    OromeHipQuantFormat f;
    int rc = orome_hip_format_from_ggml_type(ti->type, &f);
    if (rc) return rc;
    out->offset = fp->gguf->data_offset + ti->offset;
    out->format = f;
    out->expert_stride = orome_hip_gguf_tensor_size(ti) / E;
    return OROME_OK;
}

OromeHipExpertLayerRef orome_hip_format_resolve_expert_layer(OromeHipFormatProvider *fp, int layer, uint32_t E) {
    OromeHipExpertLayerRef r;
    memset(&r, 0, sizeof r);
    if (!fp || !E) return r;
    r.buffer = fp->model_buf;
    char nm[128];
    snprintf(nm, sizeof nm, "blk.%d.ffn_gate_exps.weight", layer);
    proj(fp, nm, E, &r.gate);
    snprintf(nm, sizeof nm, "blk.%d.ffn_up_exps.weight", layer);
    proj(fp, nm, E, &r.up);
    snprintf(nm, sizeof nm, "blk.%d.ffn_down_exps.weight", layer);
    proj(fp, nm, E, &r.down);
    return r;
}

/* gguf_ref (inference/src/format.m:416-427) */
static OromeHipTensorRef ref(OromeHipFormatProvider *fp, const char *name, uint32_t out_dim, uint32_t in_dim) {
    OromeHipTensorRef t;
    memset(&t, 0, sizeof t);
    OromeHipGGUFTensorInfo *ti = orome_hip_gguf_find_tensor(fp->gguf, name);
    if (!ti) return t;
    OromeHipQuantFormat f;
    if (orome_hip_format_from_ggml_type(ti->type, &f)) return t;
    t.buffer = fp->model_buf;
    t.offset = fp->gguf->data_offset + ti->offset;
    t.format = f;
    t.out_dim = out_dim;
    t.in_dim = in_dim;
    return t;
}

OromeHipLayerTensorCache *orome_hip_build_tensor_cache_gguf(OromeHipFormatProvider *fp, const OromeHipModelConfig *cfg) {
    if (!fp || !cfg || cfg->num_layers <= 0) {
        orome_fail(OROME_EINVAL, "orome_hip_build_tensor_cache_gguf: bad arguments");
        return NULL;
    }
    OromeHipLayerTensorCache *c = calloc((size_t)cfg->num_layers, sizeof *c);
    uint32_t H = (uint32_t)cfg->hidden_dim, E = (uint32_t)cfg->num_experts;
    uint32_t S = (uint32_t)(cfg->shared_intermediate > 0 ? cfg->shared_intermediate : 0);
    char nm[128];
    for (int i = 0; i < cfg->num_layers; i++) {
        OromeHipLayerTensorCache *l = &c[i];
        snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", i);
        l->post_norm = ref(fp, nm, 1, H);
        if (!l->post_norm.buffer) {
            snprintf(nm, sizeof nm, "blk.%d.post_attention_norm.weight", i);
            l->post_norm = ref(fp, nm, 1, H);
        }
        snprintf(nm, sizeof nm, "blk.%d.ffn_gate_inp.weight", i);
        l->routing_gate = ref(fp, nm, E, H);
        snprintf(nm, sizeof nm, "blk.%d.exp_probs_b.bias", i);
        l->routing_bias = ref(fp, nm, 1, E);
        if (S) {
            snprintf(nm, sizeof nm, "blk.%d.ffn_gate_shexp.weight", i);
            l->shared_gate = ref(fp, nm, S, H);
            snprintf(nm, sizeof nm, "blk.%d.ffn_up_shexp.weight", i);
            l->shared_up = ref(fp, nm, S, H);
            snprintf(nm, sizeof nm, "blk.%d.ffn_down_shexp.weight", i);
            l->shared_down = ref(fp, nm, H, S);
            snprintf(nm, sizeof nm, "blk.%d.ffn_gate_inp_shexp.weight", i);
            l->shared_expert_gate = ref(fp, nm, 1, H);
        }
    }
    return c;
}

void orome_hip_free_tensor_cache(OromeHipLayerTensorCache *c) { free(c); }
