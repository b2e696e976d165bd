"""Host-side mirror of Orome's MoE engine interface over the HIP C ABI.

Mirrors the reference's load path (inference/src/main.m:443-684):
gguf_open -> ModelConfig from metadata -> FormatProvider (GGUF data in HBM)
-> format_resolve_expert_layer per layer -> build_tensor_cache_gguf, and the
per-layer MoE step of engine_step (inference/src/engine.m:656-694).
Every compute call goes through liborome_moe.so; nothing here computes.
"""
import ctypes as C
import weakref

import numpy as np

from . import _lib
from ._lib import check, lib


class DeviceBuffer:
    """A device allocation on a context's GPU.  The context frees every buffer
    still alive when it closes, so a buffer never outlives its context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.ptr = lib.orome_hip_malloc(ctx.handle, max(self.nbytes, 1))
        if not self.ptr:
            raise _lib.OromeError("orome_hip_malloc(%d): %s" % (nbytes, lib.orome_last_error()))
        ctx._buffers.add(self)

    @classmethod
    def from_array(cls, ctx, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(ctx, arr.nbytes)
        b.upload(arr)
        return b

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib.orome_hip_htod(self.ctx.handle, self.ptr, arr.ctypes.data, arr.nbytes), "htod")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib.orome_hip_dtoh(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes), "dtoh")
        return out

    def free(self):
        if self.ptr and self.ctx.handle:
            lib.orome_hip_free(self.ctx.handle, self.ptr)
        self.ptr = None
        self.ctx._buffers.discard(self)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """orome_hip_ctx: device binding, stream and scratch for up to max_tokens."""

    def __init__(self, cfg, max_tokens, device=0):
        self.cfg = cfg
        self._buffers = weakref.WeakSet()
        self.handle = lib.orome_hip_create(C.byref(cfg), int(max_tokens), int(device))
        if not self.handle:
            raise _lib.OromeError("orome_hip_create: %s" % lib.orome_last_error().decode())
        self.max_tokens = max_tokens

    def sync(self):
        check(lib.orome_hip_sync(self.handle), "sync")

    def set_path(self, path):
        check(lib.orome_hip_set_path(self.handle, int(path)), "set_path")

    def close(self):
        if self.handle:
            for b in list(self._buffers):
                b.free()
            lib.orome_hip_destroy(self.handle)
            self.handle = None


def synth_gguf(spec):
    """Build a synthetic GGUF image (numpy uint8) from an orome_synth_spec."""
    n = lib.orome_synth_gguf_size(C.byref(spec))
    if not n:
        raise _lib.OromeError("invalid synthetic spec")
    img = np.empty(n, dtype=np.uint8)
    check(lib.orome_synth_gguf_write(C.byref(spec), img.ctypes.data, n), "synth")
    return img


def synth_normal(seed, stream, n, std=1.0):
    out = np.empty(n, dtype=np.float32)
    check(lib.orome_synth_normal(seed, stream, std, out.ctypes.data, n), "synth_normal")
    return out


def make_spec(layers=1, H=2048, E=256, K=8, M=512, S=512, down=_lib.GGML_Q4_K,
              shared=_lib.GGML_Q4_K, shared_down=None, q6k_every=0, zipf=False, zipf_s=1.1,
              eps=1e-6, seed=0, centered=False, q4k_ggml=False):
    s = _lib.SynthSpec()
    s.num_layers, s.hidden_dim, s.num_experts, s.num_experts_per_tok = layers, H, E, K
    s.moe_intermediate, s.shared_intermediate = M, S
    s.gate_type = s.up_type = _lib.GGML_Q4_K
    s.down_type = down
    s.shared_gate_type = shared
    s.shared_down_type = shared if shared_down is None else shared_down
    s.q6k_down_every, s.zipf_bias, s.zipf_s = q6k_every, int(bool(zipf)), zipf_s
    s.rms_norm_eps, s.seed = eps, seed
    s.centered = int(bool(centered))
    s.q4k_ggml_layout = int(bool(q4k_ggml))
    return s


class MoEModel:
    """A GGUF MoE model resident in HBM (all layers), ready for forward calls."""

    def __init__(self, image=None, path=None, max_tokens=16, device=0, pack=None,
                 q4k_layout=_lib.OROME_Q4K_LAYOUT_FILE):
        """pack: register every layer's tile-major Q4_K copies for the grouped
        GEMMs (orome_hip_pack_layer); default when max_tokens > 2, the batch
        sizes that use those GEMMs.  q4k_layout: the Q4_K scale packing
        (OROME_Q4K_LAYOUT_*; FILE = what the file declares)."""
        if (image is None) == (path is None):
            raise ValueError("give exactly one of image or path")
        self._image = image  # keep the host image alive while parsed
        if path is not None:
            self.gf = lib.orome_hip_gguf_open(path.encode())
        else:
            self.gf = lib.orome_hip_gguf_open_memory(image.ctypes.data, image.nbytes)
        if not self.gf:
            raise _lib.OromeError("gguf_open: %s" % lib.orome_last_error().decode())
        self.cfg = _lib.ModelConfig()
        check(lib.orome_hip_model_config_from_gguf(self.gf, C.byref(self.cfg)), "orome_hip_model_config_from_gguf")
        self.ctx = Context(self.cfg, max_tokens, device)
        self.fp = lib.orome_hip_format_provider_open_gguf_layout(self.gf, self.ctx.handle, int(q4k_layout))
        if not self.fp:
            raise _lib.OromeError("format_provider_open_gguf: %s" % lib.orome_last_error().decode())
        L = self.cfg.num_layers
        self.elrs = (_lib.ExpertLayerRef * L)()
        for l in range(L):
            self.elrs[l] = lib.orome_hip_format_resolve_expert_layer(self.fp, l, self.cfg.num_experts)
        self._cache = lib.orome_hip_build_tensor_cache_gguf(self.fp, C.byref(self.cfg))
        if not self._cache:
            raise _lib.OromeError("build_tensor_cache_gguf failed")
        self.caches = C.cast(self._cache, C.POINTER(_lib.LayerTensorCache * L)).contents
        if pack if pack is not None else max_tokens > 2:
            self.pack_layers()

    def pack_layers(self):
        for l in range(self.cfg.num_layers):
            check(lib.orome_hip_pack_layer(self.ctx.handle, C.byref(self.cfg), C.byref(self.elrs[l]),
                                           C.byref(self.caches[l])), "orome_hip_pack_layer")

    def unpack(self):
        check(lib.orome_hip_unpack_all(self.ctx.handle), "orome_hip_unpack_all")

    @property
    def H(self):
        return self.cfg.hidden_dim

    def forward(self, layer, x, h_in, h_out, T, K=None, residual_out=None, sumsq_parts=None, stream=None):
        K = self.cfg.num_experts_per_tok if K is None else K
        check(lib.orome_moe_forward(self.ctx.handle, C.byref(self.cfg), C.byref(self.elrs[layer]),
                                    C.byref(self.caches[layer]), _ptr(x), _ptr(h_in), _ptr(h_out),
                                    _ptr(residual_out), _ptr(sumsq_parts), T, K, stream),
              "orome_moe_forward")

    def layer_forward(self, layer, h, T, K=None, stream=None):
        K = self.cfg.num_experts_per_tok if K is None else K
        check(lib.orome_moe_layer_forward(self.ctx.handle, C.byref(self.cfg),
                                          C.byref(self.elrs[layer]), C.byref(self.caches[layer]),
                                          _ptr(h), T, K, stream), "orome_moe_layer_forward")

    def stack_forward(self, h, T, K=None, n_layers=None, stream=None):
        K = self.cfg.num_experts_per_tok if K is None else K
        n = self.cfg.num_layers if n_layers is None else n_layers
        check(lib.orome_moe_stack_forward(self.ctx.handle, C.byref(self.cfg), self.elrs,
                                          self._cache, n, _ptr(h), T, K, stream),
              "orome_moe_stack_forward")

    def debug_outputs(self, T, K=None):
        K = self.cfg.num_experts_per_tok if K is None else K
        E = self.cfg.num_experts
        logits = np.empty((T, E + 1), np.float32)
        idx = np.empty((T, K), np.int32)
        w = np.empty((T, K), np.float32)
        offsets = np.empty(E + 1, np.uint32)
        pairs = np.empty(T * K, np.uint32)
        check(lib.orome_moe_debug_outputs(self.ctx.handle, logits.ctypes.data, idx.ctypes.data,
                                          w.ctypes.data, offsets.ctypes.data, pairs.ctypes.data),
              "debug_outputs")
        return dict(logits=logits, idx=idx, w=w, offsets=offsets, pairs=pairs)

    def tensor_device_ptr(self, name):
        ti = lib.orome_hip_gguf_find_tensor(self.gf, name.encode())
        if not ti:
            raise KeyError(name)
        return self.fp.contents.model_buf + self.gf.contents.data_offset + ti.contents.offset

    def close(self):
        if getattr(self, "_cache", None):
            lib.orome_hip_free_tensor_cache(self._cache)
            self._cache = None
        if getattr(self, "fp", None):
            lib.orome_hip_format_provider_close(self.fp)
            self.fp = None
        if getattr(self, "ctx", None):
            self.ctx.close()
        if getattr(self, "gf", None):
            lib.orome_hip_gguf_close(self.gf)
            self.gf = None


def _ptr(b):
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return b.ptr
    return int(b)
