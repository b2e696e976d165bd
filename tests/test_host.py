"""Host-side checks that need no GPU: the C ABI exports, the GGUF parser
against an independent reader, error paths, and the synthetic generator."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import orome_amd
import oracle as O
from orome_amd import _lib
from orome_amd._lib import lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in ("orome_moe.h", "orome_synth.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef struct[^;]*?\{.*?\}[^;]*;", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert names <= set(_lib.SIGNATURES), sorted(names - set(_lib.SIGNATURES))
    assert b"gfx950" in lib.orome_version()


# The reference's own C-visible names on the MoE path (inference/include/orome.h:
# 29, 40-43, 49-98, 227-279, 413-444; inference/src/gguf.m, format.m): a
# translation unit that declares them must still be able to include this
# library's header, and the library must not export any of them.
REFERENCE_NAMES_TU = r"""
#define OROME_MAX_ACTIVE 16
typedef enum { FFN_MOE, FFN_DENSE } FFNType;
typedef struct { char name[64]; int hidden_dim; int num_layers; int vocab_size; } ModelConfig;
typedef enum { QFMT_GGUF_Q4_K, QFMT_GGUF_Q5_K, QFMT_GGUF_Q6_K, QFMT_GGUF_Q8_0, QFMT_F16, QFMT_BF16,
               QFMT_F32 } QuantFormat;
typedef struct { void *buffer; unsigned long offset; void *pipeline; QuantFormat format; } TensorRef;
typedef struct { unsigned long offset, expert_stride; QuantFormat format; } ExpertProjRef;
typedef struct { void *buffer; ExpertProjRef gate, up, down; } ExpertLayerRef;
typedef struct { TensorRef routing_gate, shared_gate; } LayerTensorCache;
typedef struct GGUFTensorInfo GGUFTensorInfo;
typedef struct GGUFFile GGUFFile;
typedef struct FormatProvider FormatProvider;
GGUFFile *gguf_open(const char *path);
void gguf_close(GGUFFile *gf);
GGUFTensorInfo *gguf_find_tensor(GGUFFile *gf, const char *name);
QuantFormat format_from_ggml_type(unsigned type);
ExpertLayerRef format_resolve_expert_layer(FormatProvider *fp, int layer, unsigned E);
#include "orome_moe.h"
int use_both(ModelConfig *a, OromeHipModelConfig *b) {
    b->hidden_dim = a->hidden_dim;
    return (int)QFMT_GGUF_Q6_K == (int)OROME_QFMT_GGUF_Q6_K && (int)FFN_MOE == (int)OROME_FFN_MOE;
}
"""
REFERENCE_SYMBOLS = ["gguf_open", "gguf_close", "gguf_find_tensor", "gguf_tensor_size", "ggml_type_name",
                     "format_from_ggml_type", "format_provider_open_gguf", "format_provider_close",
                     "format_resolve_expert_layer", "build_tensor_cache_gguf", "free_tensor_cache"]


def test_header_coexists_with_reference_names(tmp_path):
    src = tmp_path / "both.c"
    src.write_text(REFERENCE_NAMES_TU)
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_exports_only_prefixed_symbols():
    for name in REFERENCE_SYMBOLS:
        assert not hasattr(lib, name), name
    r = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = [l.split()[-1] for l in r.stdout.splitlines() if " T " in l]
    bad = [n for n in exported if not n.startswith("orome_") and not n.startswith("_")]
    assert not bad, bad


def tiny_spec(**kw):
    args = dict(layers=2, H=512, E=16, K=4, M=512, S=512, seed=3)
    args.update(kw)
    return orome_amd.make_spec(**args)


def test_gguf_parser_matches_independent_reader(tmp_path):
    img = orome_amd.synth_gguf(tiny_spec(down=14, zipf=True, q6k_every=2))
    meta, tensors, data_off = O.read_gguf(img)
    path = tmp_path / "m.gguf"
    img.tofile(path)
    for gf in (lib.orome_hip_gguf_open_memory(img.ctypes.data, img.nbytes), lib.orome_hip_gguf_open(str(path).encode())):
        assert gf
        g = gf.contents
        assert g.data_offset == data_off and g.num_tensors == len(tensors)
        for name, (dims, typ, off, nb) in tensors.items():
            ti = lib.orome_hip_gguf_find_tensor(gf, name.encode())
            assert ti, name
            t = ti.contents
            assert t.type == typ and list(t.dims[:t.n_dims]) == dims
            assert g.data_offset + t.offset == off and lib.orome_hip_gguf_tensor_size(ti) == nb
        assert not lib.orome_hip_gguf_find_tensor(gf, b"blk.0.nope")
        cfg = _lib.ModelConfig()
        assert lib.orome_hip_model_config_from_gguf(gf, C.byref(cfg)) == 0
        assert (cfg.hidden_dim, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate,
                cfg.shared_intermediate, cfg.num_layers) == (512, 16, 4, 512, 512, 2)
        assert cfg.ffn_type == _lib.FFN_MOE and abs(cfg.rms_norm_eps - 1e-6) < 1e-12
        lib.orome_hip_gguf_close(gf)
    # layer 1 (l % 2 == 1) got the Q6_K expert down
    assert tensors["blk.1.ffn_down_exps.weight"][1] == 14


def test_gguf_rejects_malformed():
    img = orome_amd.synth_gguf(tiny_spec())
    bad = img.copy()
    bad[0] ^= 0xFF
    assert not lib.orome_hip_gguf_open_memory(bad.ctypes.data, bad.nbytes)
    assert b"magic" in lib.orome_last_error()
    bad = img.copy()
    bad[4] = 7
    assert not lib.orome_hip_gguf_open_memory(bad.ctypes.data, bad.nbytes)
    assert b"version" in lib.orome_last_error()
    short = img[:200].copy()
    assert not lib.orome_hip_gguf_open_memory(short.ctypes.data, short.nbytes)
    cut = img[: img.nbytes - 1000].copy()  # last tensor runs past the end
    assert not lib.orome_hip_gguf_open_memory(cut.ctypes.data, cut.nbytes)
    assert not lib.orome_hip_gguf_open(b"/nonexistent/model.gguf")


def test_format_from_ggml_type():
    f = C.c_int()
    for t, q in ((12, _lib.QFMT_GGUF_Q4_K), (13, _lib.QFMT_GGUF_Q5_K), (14, _lib.QFMT_GGUF_Q6_K),
                 (8, _lib.QFMT_GGUF_Q8_0), (0, _lib.QFMT_F32), (1, _lib.QFMT_F16), (30, _lib.QFMT_BF16)):
        assert lib.orome_hip_format_from_ggml_type(t, C.byref(f)) == 0 and f.value == q
    # the reference silently maps unknown types to Q4_K (format.m:335); here it is an error
    assert lib.orome_hip_format_from_ggml_type(2, C.byref(f)) == -2
    assert lib.orome_hip_ggml_type_name(12) == b"Q4_K"


def test_synth_is_deterministic_and_seeded():
    a = orome_amd.synth_gguf(tiny_spec(seed=5))
    b = orome_amd.synth_gguf(tiny_spec(seed=5))
    c = orome_amd.synth_gguf(tiny_spec(seed=6))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    om = O.OracleModel(orome_amd.synth_gguf(tiny_spec(zipf=True)))
    bias = om.array("blk.0.exp_probs_b.bias", np.float32)
    assert abs(np.exp(bias.astype(np.float64)).sum() - 1) < 1e-5
    assert sorted(np.round(np.exp(bias) * 1e6)) == sorted(np.round(np.exp(bias) * 1e6))
    r = np.exp(np.sort(bias)[::-1].astype(np.float64))
    assert np.allclose(r[0] / r[1:5], (np.arange(2, 6)) ** 1.1, rtol=1e-4)  # Zipf ratios
    x = orome_amd.synth_normal(1, 2, 100000)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    w = om.array("blk.0.ffn_gate_inp.weight", np.float32)
    assert abs(w.std() - 0.02) < 0.002
    assert np.all(om.array("blk.0.ffn_norm.weight", np.float32) == 1)


def test_context_creation_without_device_fails_cleanly():
    cfg = _lib.ModelConfig()
    cfg.hidden_dim, cfg.num_experts, cfg.moe_intermediate = 512, 16, 512
    assert not lib.orome_hip_create(C.byref(cfg), 0, 0)  # bad max_tokens, checked first
    assert b"max_tokens" in lib.orome_last_error()


def test_synth_centered_q4k_mins_equal_scales():
    om = O.OracleModel(orome_amd.synth_gguf(tiny_spec(centered=True)))
    blk = om.array("blk.0.ffn_gate_exps.weight")[:144 * 64].reshape(64, 144)
    for b in blk:
        import test_oracle
        sc, mn = test_oracle.layout_table(list(b[4:16]))
        assert sc == mn
        d = float(b[0:2].view(np.float16)[0])
        assert float(b[2:4].view(np.float16)[0]) == float(np.float16(7.5 * d))
    w = O.decode_rows(O.Q4_K, om.array("blk.0.ffn_gate_exps.weight")[:144 * 8 * 512], 512, 2048)
    assert abs(w.mean()) < 0.02 * w.std()
