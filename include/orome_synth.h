/*
 * orome_synth.h -- seeded synthetic MoE models and inputs in GGUF form.
 *
 * No counterpart in the reference (which loads real model files through
 * gguf_open, inference/src/gguf.m:273).  These entry points build a GGUF v3
 * image in host memory, with the tensor names and layouts of a Qwen3.5 MoE
 * file (inference/src/format.m:374-409, 495-509), filled from a seeded
 * generator, so that benchmarks and parity tests feed the GGUF loader, the
 * HBM upload and the kernels exactly as a real file would.
 *
 * Generator: SplitMix64-seeded xoshiro256** per (layer, tensor, expert)
 * stream; normals by Box-Muller in double precision.
 *   F32 norm weights   1.0
 *   router W_r [E x H] N(0, 0.02^2); shared-gate vector [H] N(0, 0.02^2)
 *   Q4_K  d = fp16(|N|*2e-3), dmin = fp16(|N|*1e-3), 12 scale bytes and
 *         128 quant bytes uniform
 *         centered: mins equal the scales and dmin = fp16(7.5*d), so a
 *         weight is d*sc*q - fp16(7.5 d)*sc, about zero-mean (stacked layers
 *         with residuals stay finite under fp16 activation staging)
 *   Q5_K  d = fp16(|N|*1e-3), dmin = fp16(|N|*1e-3), 12 scale bytes, 32 qh
 *         and 128 ql bytes uniform
 *   Q6_K  ql/qh bytes uniform, 16 int8 scales uniform in [-64, 63],
 *         d = fp16(|N|*2e-3)
 *   Q8_0  d = fp16(|N|*4e-3), 32 int8 quants uniform in [-127, 127]
 *   Zipf bias (optional, blk.N.exp_probs_b.bias, F32 [E]):
 *         bias[e] = ln p(pi(e)), p(r) = r^-s / sum_r r^-s over ranks 1..E,
 *         pi a seeded permutation.
 */
#ifndef OROME_SYNTH_H
#define OROME_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

typedef struct {
    int num_layers;
    int hidden_dim;
    int num_experts;
    int num_experts_per_tok;
    int moe_intermediate;
    int shared_intermediate;      /* 0: no shared expert tensors */
    uint32_t gate_type;           /* ggml type ids: 12 Q4_K, 13 Q5_K, 14 Q6_K, 8 Q8_0 */
    uint32_t up_type;
    uint32_t down_type;
    uint32_t shared_gate_type;    /* gate and up of the shared expert */
    uint32_t shared_down_type;
    int q6k_down_every;           /* >0: layers l with l % n == n-1 use Q6_K expert down */
    int zipf_bias;                /* nonzero: add blk.N.exp_probs_b.bias */
    float zipf_s;
    float rms_norm_eps;
    uint64_t seed;
    int centered;                 /* nonzero: zero-mean Q4_K rows (see above) */
    int q4k_ggml_layout;          /* nonzero: the same Q4_K values, written in the ggml scale
                                     packing, and the file declares it (orome_moe.h,
                                     OROME_Q4K_LAYOUT_KEY) */
} orome_synth_spec;

/* Size in bytes of the GGUF image for `spec` (0 if the spec is invalid). */
size_t orome_synth_gguf_size(const orome_synth_spec *spec);
/* Writes the image into dst[0..size); returns 0 or a negative OROME_E* code.
 * Uses all host threads (OpenMP). */
int orome_synth_gguf_write(const orome_synth_spec *spec, void *dst, size_t size);
/* n fp32 samples of N(0, std^2) from stream (seed, stream). */
int orome_synth_normal(uint64_t seed, uint64_t stream, float std, float *out, size_t n);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
