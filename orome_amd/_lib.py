"""ctypes binding of liborome_moe.so (the C ABI declared in include/orome_moe.h
and include/orome_synth.h).

The library is built in-tree by ``python orome_amd/build.py``.  Importing
this module without the built library raises immediately: there is no
fallback implementation of any kernel.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# OROME_LIB names another build of the same library (e.g. an instrumented one)
LIB_PATH = os.environ.get("OROME_LIB") or os.path.join(HERE, "liborome_moe.so")

# OromeHipQuantFormat: the values of QuantFormat (inference/include/orome.h:227-235)
QFMT_GGUF_Q4_K, QFMT_GGUF_Q5_K, QFMT_GGUF_Q6_K, QFMT_GGUF_Q8_0, QFMT_F16, QFMT_BF16, QFMT_F32 = range(7)
FFN_MOE, FFN_DENSE = 0, 1
OROME_PATH_AUTO, OROME_PATH_GEMV, OROME_PATH_MFMA = 0, 1, 2
OROME_Q4K_LAYOUT_FILE, OROME_Q4K_LAYOUT_REFERENCE, OROME_Q4K_LAYOUT_GGML = 0, 1, 2
OROME_MAX_ACTIVE = 16
STAGES = ["norm", "router", "topk", "dispatch", "stage_f16", "gate_up", "down", "combine"]
ERRORS = {0: "OK", -1: "EINVAL", -2: "EUNSUPPORTED", -3: "EHIP", -4: "ENOMEM", -5: "ENOTFOUND",
          -6: "EFORMAT"}
GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, GGML_F32 = 12, 14, 8, 0


class ModelConfig(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("hidden_dim", C.c_int), ("num_layers", C.c_int),
                ("rms_norm_eps", C.c_float), ("ffn_type", C.c_int), ("num_experts", C.c_int),
                ("num_experts_per_tok", C.c_int), ("moe_intermediate", C.c_int),
                ("shared_intermediate", C.c_int)]


class TensorRef(C.Structure):
    _fields_ = [("buffer", C.c_void_p), ("offset", C.c_size_t), ("format", C.c_int),
                ("out_dim", C.c_uint32), ("in_dim", C.c_uint32)]


class ExpertProjRef(C.Structure):
    _fields_ = [("offset", C.c_size_t), ("expert_stride", C.c_size_t), ("format", C.c_int)]


class ExpertLayerRef(C.Structure):
    _fields_ = [("buffer", C.c_void_p), ("gate", ExpertProjRef), ("up", ExpertProjRef),
                ("down", ExpertProjRef)]


class LayerTensorCache(C.Structure):
    _fields_ = [(n, TensorRef) for n in ("post_norm", "routing_gate", "shared_gate", "shared_up",
                                          "shared_down", "shared_expert_gate", "routing_bias")]


class GGUFTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("type", C.c_uint32), ("offset", C.c_uint64)]


class GGUFFile(C.Structure):
    _fields_ = [("fd", C.c_int), ("mmap_base", C.c_void_p), ("file_size", C.c_size_t),
                ("data_offset", C.c_size_t), ("tensors", C.POINTER(GGUFTensorInfo)),
                ("num_tensors", C.c_uint64), ("alignment", C.c_uint32), ("arch", C.c_char * 32),
                ("ffn_type", C.c_int), ("num_layers", C.c_int), ("hidden_dim", C.c_int),
                ("num_experts", C.c_int), ("num_experts_per_tok", C.c_int),
                ("moe_intermediate", C.c_int), ("rms_norm_eps", C.c_float), ("index", C.c_void_p),
                ("owns_map", C.c_bool), ("q4k_layout", C.c_int)]


class FormatProvider(C.Structure):
    _fields_ = [("gguf", C.POINTER(GGUFFile)), ("model_buf", C.c_void_p),
                ("alloc_base", C.c_void_p), ("model_bytes", C.c_size_t), ("ctx", C.c_void_p)]


class SynthSpec(C.Structure):
    _fields_ = [("num_layers", C.c_int), ("hidden_dim", C.c_int), ("num_experts", C.c_int),
                ("num_experts_per_tok", C.c_int), ("moe_intermediate", C.c_int),
                ("shared_intermediate", C.c_int), ("gate_type", C.c_uint32),
                ("up_type", C.c_uint32), ("down_type", C.c_uint32),
                ("shared_gate_type", C.c_uint32), ("shared_down_type", C.c_uint32),
                ("q6k_down_every", C.c_int), ("zipf_bias", C.c_int), ("zipf_s", C.c_float),
                ("rms_norm_eps", C.c_float), ("seed", C.c_uint64), ("centered", C.c_int),
                ("q4k_ggml_layout", C.c_int)]


VP, I, U32, SZ, F32P = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t, C.POINTER(C.c_float)
P = C.POINTER

# name -> (restype, argtypes); every symbol declared in include/*.h
SIGNATURES = {
    "orome_hip_gguf_open": (P(GGUFFile), [C.c_char_p]),
    "orome_hip_gguf_open_memory": (P(GGUFFile), [VP, SZ]),
    "orome_hip_gguf_close": (None, [P(GGUFFile)]),
    "orome_hip_gguf_find_tensor": (P(GGUFTensorInfo), [P(GGUFFile), C.c_char_p]),
    "orome_hip_gguf_tensor_size": (SZ, [P(GGUFTensorInfo)]),
    "orome_hip_ggml_type_name": (C.c_char_p, [U32]),
    "orome_hip_format_from_ggml_type": (I, [U32, P(C.c_int)]),
    "orome_hip_model_config_from_gguf": (I, [P(GGUFFile), P(ModelConfig)]),
    "orome_hip_create": (VP, [P(ModelConfig), I, I]),
    "orome_hip_destroy": (None, [VP]),
    "orome_hip_sync": (I, [VP]),
    "orome_hip_get_stream": (VP, [VP]),
    "orome_last_error": (C.c_char_p, []),
    "orome_hip_set_path": (I, [VP, I]),
    "orome_hip_malloc": (VP, [VP, SZ]),
    "orome_hip_free": (I, [VP, VP]),
    "orome_hip_htod": (I, [VP, VP, VP, SZ]),
    "orome_hip_dtoh": (I, [VP, VP, VP, SZ]),
    "orome_hip_pack_layer": (I, [VP, P(ModelConfig), P(ExpertLayerRef), P(LayerTensorCache)]),
    "orome_hip_unpack_all": (I, [VP]),
    "orome_hip_kernel_timing": (I, [VP, VP, I]),
    "orome_hip_format_provider_open_gguf": (P(FormatProvider), [P(GGUFFile), VP]),
    "orome_hip_format_provider_open_gguf_layout": (P(FormatProvider), [P(GGUFFile), VP, I]),
    "orome_hip_format_provider_close": (None, [P(FormatProvider)]),
    "orome_hip_format_resolve_expert_layer": (ExpertLayerRef, [P(FormatProvider), I, U32]),
    "orome_hip_build_tensor_cache_gguf": (P(LayerTensorCache), [P(FormatProvider), P(ModelConfig)]),
    "orome_hip_free_tensor_cache": (None, [P(LayerTensorCache)]),
    "orome_moe_forward": (I, [VP, P(ModelConfig), P(ExpertLayerRef), P(LayerTensorCache), VP, VP,
                              VP, VP, VP, I, I, VP]),
    "orome_moe_layer_forward": (I, [VP, P(ModelConfig), P(ExpertLayerRef), P(LayerTensorCache), VP,
                                    I, I, VP]),
    "orome_moe_stack_forward": (I, [VP, P(ModelConfig), P(ExpertLayerRef), P(LayerTensorCache), I,
                                    VP, I, I, VP]),
    "orome_moe_forward_noalloc": (I, [P(ModelConfig), P(ExpertLayerRef), P(LayerTensorCache), VP, VP, VP,
                                      VP, VP, I, I, VP]),
    "orome_moe_debug_outputs": (I, [VP, VP, VP, VP, VP, VP]),
    "orome_moe_topk": (I, [VP, VP, VP, I, I, I, VP, VP]),
    "orome_dequant_rows": (I, [VP, I, VP, U32, U32, VP]),
    "orome_dequant_rows_f16": (I, [VP, I, VP, U32, U32, VP]),
    "orome_debug_mfma_weights": (I, [VP, I, I, VP, U32, U32, VP]),
    "orome_hip_debug_inject_failure": (I, [VP]),
    "orome_version": (C.c_char_p, []),
    "orome_hip_capture_begin": (I, [VP]),
    "orome_hip_capture_end": (I, [VP, P(VP)]),
    "orome_hip_graph_launch": (I, [VP, VP]),
    "orome_hip_graph_destroy": (I, [VP]),
    "orome_hip_stage_timing": (I, [VP, I]),
    "orome_hip_stream_delay": (I, [VP, U32]),
    "orome_hip_stage_times": (I, [VP, F32P, P(I), I]),
    "orome_synth_gguf_size": (SZ, [P(SynthSpec)]),
    "orome_synth_gguf_write": (I, [P(SynthSpec), VP, SZ]),
    "orome_synth_normal": (I, [C.c_uint64, C.c_uint64, C.c_float, VP, SZ]),
}


class OromeError(RuntimeError):
    pass


def load(path=LIB_PATH):
    if not os.path.exists(path):
        raise ImportError("liborome_moe.so is not built (%s); run `python orome_amd/build.py`" % path)
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def check(rc, what=""):
    if rc != 0:
        msg = lib.orome_last_error().decode(errors="replace")
        raise OromeError("%s: %s (%s)" % (what, ERRORS.get(rc, rc), msg))
    return rc
