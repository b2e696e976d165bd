"""TEST INFRASTRUCTURE ONLY: ctypes binding of the C oracle (moe_oracle.c)
plus a small independent GGUF reader used to locate tensors for it.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module.  The reader here is deliberately separate from the product's parser
(orome_amd/csrc/gguf.c) so that tests cross-check the two.
"""
import ctypes as C
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
Q4_K, Q5_K, Q6_K, Q8_0, F16, BF16, F32 = range(7)
GGML_TO_FMT = {12: Q4_K, 13: Q5_K, 14: Q6_K, 8: Q8_0, 1: F16, 30: BF16, 0: F32}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(name):
    path = os.path.join(HERE, name)
    if not os.path.exists(path):
        build()
    lib = C.CDLL(path)
    VP, I, U32, F = C.c_void_p, C.c_int, C.c_uint32, C.c_float
    sig = {
        "orc_fp16_to_f32": (F, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [F]),
        "orc_round_half": (F, [F]),
        "orc_bf16_trunc": (F, [F]),
        "orc_unpack_q4k_pair": (None, [VP, U32, VP, VP, VP, VP]),
        "orc_unpack_q4k_batch": (None, [VP, C.c_size_t, VP]),
        "orc_row_bytes": (C.c_size_t, [I, U32]),
        "orc_decode_row": (I, [I, VP, U32, VP]),
        "orc_decode_rows": (I, [I, VP, U32, U32, VP]),
        "orc_canon_dot": (F, [VP, VP, U32]),
        "orc_router_logits": (None, [VP, VP, VP, I, I, I, VP]),
        "orc_topk_route": (None, [VP, VP, I, I, I, VP, VP, VP]),
        "orc_dispatch": (None, [VP, I, I, I, VP, VP]),
        "orc_rmsnorm": (None, [VP, VP, I, I, F, VP]),
        "orc_moe_forward": (I, [VP, VP, VP, VP, I, I, VP, VP, VP, VP, VP]),
        "orc_num_threads": (I, []),
        "orc_set_threads": (None, [I]),
    }
    for n, (r, a) in sig.items():
        f = getattr(lib, n)
        f.restype, f.argtypes = r, a
    return lib


_libs = {}


def lib(omp=True):
    key = "omp" if omp else "st"
    if key not in _libs:
        _libs[key] = _load("liborome_oracle_omp.so" if omp else "liborome_oracle.so")
    return _libs[key]


class OrcLayer(C.Structure):
    _fields_ = [("E", C.c_int), ("H", C.c_int), ("M", C.c_int), ("S", C.c_int),
                ("router", C.c_void_p), ("shared_gate_vec", C.c_void_p), ("bias", C.c_void_p),
                ("gate", C.c_void_p), ("gate_stride", C.c_size_t), ("gate_fmt", C.c_int),
                ("up", C.c_void_p), ("up_stride", C.c_size_t), ("up_fmt", C.c_int),
                ("down", C.c_void_p), ("down_stride", C.c_size_t), ("down_fmt", C.c_int),
                ("sh_gate", C.c_void_p), ("sh_gate_fmt", C.c_int),
                ("sh_up", C.c_void_p), ("sh_up_fmt", C.c_int),
                ("sh_down", C.c_void_p), ("sh_down_fmt", C.c_int)]


def p(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------ GGUF reader
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q",
           12: "d"}
_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176),
          14: (256, 210)}


def read_gguf(buf):
    """Parse a GGUF v2/v3 image (bytes-like) -> (metadata dict, tensors dict,
    data_offset).  tensors[name] = (dims, ggml_type, absolute offset, nbytes)."""
    mv = memoryview(buf)
    pos = 0

    def rd(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, mv, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0]

    def rstr():
        n = rd("Q")
        nonlocal pos
        s = bytes(mv[pos:pos + n]).decode()
        pos += n
        return s

    def rval(t):
        if t in _SCALAR:
            return rd(_SCALAR[t])
        if t == 8:
            return rstr()
        if t == 9:
            et, n = rd("I"), rd("Q")
            return [rval(et) for _ in range(n)]
        raise ValueError("bad gguf type %d" % t)

    assert rd("I") == 0x46554747, "bad magic"
    ver = rd("I")
    assert ver in (2, 3)
    nt, nkv = rd("Q"), rd("Q")
    meta = {}
    for _ in range(nkv):
        k = rstr()
        meta[k] = rval(rd("I"))
    infos = []
    for _ in range(nt):
        name = rstr()
        nd = rd("I")
        dims = [rd("Q") for _ in range(nd)]
        t, off = rd("I"), rd("Q")
        infos.append((name, dims, t, off))
    align = meta.get("general.alignment", 32)
    data = (pos + align - 1) // align * align
    tensors = {}
    for name, dims, t, off in infos:
        be, bb = _BLOCK[t]
        n = int(np.prod(dims))
        tensors[name] = (dims, t, data + off, n // be * bb)
    return meta, tensors, data


class OracleModel:
    """Oracle view of a GGUF image: per-layer OrcLayer structs pointing into it."""

    def __init__(self, image):
        self.image = image
        self.meta, self.tensors, self.data_offset = read_gguf(image)
        a = self.meta.get("general.architecture", "llama")
        self.H = self.meta[a + ".embedding_length"]
        self.E = self.meta[a + ".expert_count"]
        self.K = self.meta[a + ".expert_used_count"]
        self.M = self.meta[a + ".expert_feed_forward_length"]
        self.L = self.meta[a + ".block_count"]
        self.eps = self.meta.get(a + ".attention.layer_norm_rms_epsilon", 1e-6)
        self.base = image.ctypes.data

    def t(self, name):
        return self.tensors.get(name)

    def addr(self, name):
        t = self.tensors.get(name)
        return None if t is None else self.base + t[2]

    def array(self, name, dtype=np.uint8):
        dims, typ, off, nb = self.tensors[name]
        return self.image[off:off + nb].view(dtype)

    def layer(self, l):
        L = OrcLayer()
        L.E, L.H, L.M = self.E, self.H, self.M
        L.router = self.addr("blk.%d.ffn_gate_inp.weight" % l)
        L.shared_gate_vec = self.addr("blk.%d.ffn_gate_inp_shexp.weight" % l)
        L.bias = self.addr("blk.%d.exp_probs_b.bias" % l)
        for proj in ("gate", "up", "down"):
            dims, typ, off, nb = self.tensors["blk.%d.ffn_%s_exps.weight" % (l, proj)]
            setattr(L, proj, self.base + off)
            setattr(L, proj + "_stride", nb // self.E)
            setattr(L, proj + "_fmt", GGML_TO_FMT[typ])
        sg = self.tensors.get("blk.%d.ffn_gate_shexp.weight" % l)
        if sg:
            L.S = sg[0][1]
            for proj, fld in (("gate", "sh_gate"), ("up", "sh_up"), ("down", "sh_down")):
                dims, typ, off, nb = self.tensors["blk.%d.ffn_%s_shexp.weight" % (l, proj)]
                setattr(L, fld, self.base + off)
                setattr(L, fld + "_fmt", GGML_TO_FMT[typ])
        return L

    def norm_weight(self, l):
        return self.array("blk.%d.ffn_norm.weight" % l, np.float32)

    def forward(self, l, x, h_in=None, K=None, omp=True, debug=False):
        """h_out = h_in + MoE_l(x); returns h_out (and debug dict)."""
        K = self.K if K is None else K
        T = x.shape[0]
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        L = self.layer(l)
        dbg = {}
        if debug:
            dbg = dict(logits=np.empty((T, self.E + 1), np.float32), idx=np.empty((T, K), np.int32),
                       w=np.empty((T, K), np.float32),
                       y=np.empty((T, K, self.H), np.float32), ysh=np.empty((T, self.H), np.float32))
        rc = lib(omp).orc_moe_forward(C.byref(L), p(x), p(h_in), p(out), T, K,
                                      p(dbg.get("logits")), p(dbg.get("idx")), p(dbg.get("w")),
                                      p(dbg.get("y")), p(dbg.get("ysh")))
        assert rc == 0
        return (out, dbg) if debug else out

    def rmsnorm(self, l, h):
        x = np.empty_like(h)
        lib().orc_rmsnorm(p(h), p(self.norm_weight(l)), h.shape[0], self.H, self.eps, p(x))
        return x

    def layer_forward(self, l, h, K=None, omp=True):
        return self.forward(l, self.rmsnorm(l, h), h_in=h, K=K, omp=omp)


def canon_dot(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return np.float32(lib().orc_canon_dot(p(a), p(b), a.size))


def sumsq_parts(h):
    """[T][H/256] sums of squares per 256-column block in the canonical order
    (the Sigma h^2 partials moe_combine_copy_sq_k8 writes,
    inference/src/shaders.metal:1079-1135, in this build's fixed order)."""
    T, H = h.shape
    out = np.empty((T, H // 256), np.float32)
    for t in range(T):
        for b in range(H // 256):
            blk = h[t, 256 * b:256 * (b + 1)]
            out[t, b] = canon_dot(blk, blk)
    return out


def dispatch(idx, E):
    T, K = idx.shape
    off = np.empty(E + 1, np.uint32)
    pairs = np.empty(T * K, np.uint32)
    idx = np.ascontiguousarray(idx, np.int32)
    lib().orc_dispatch(p(idx), T, K, E, p(off), p(pairs))
    return off, pairs


def topk(logits, bias, K):
    T, E1 = logits.shape
    idx = np.empty((T, K), np.int32)
    w = np.empty((T, K), np.float32)
    sg = np.empty(T, np.float32)
    lib().orc_topk_route(p(np.ascontiguousarray(logits, np.float32)),
                         p(None if bias is None else np.ascontiguousarray(bias, np.float32)),
                         T, E1 - 1, K, p(idx), p(w), p(sg))
    return idx, w, sg


def decode_rows(fmt, data, rows, n):
    out = np.empty((rows, n), np.float32)
    data = np.ascontiguousarray(data)
    assert lib().orc_decode_rows(fmt, p(data), rows, n, p(out)) == 0
    return out
