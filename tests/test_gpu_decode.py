"""GPU parity of the decode (GEMV) path and the routing kernels, through the C ABI,
against the C oracle on identical seeded inputs.

Contract: router logits, expert indices and dispatch order bit-exact;
dequantised weights bit-exact; outputs within 1e-3 relative L2."""
import hashlib
import json
import os

import numpy as np
import pytest

import orome_amd
import oracle as O
from conftest import banner
from orome_amd import _lib
from orome_amd._lib import check, lib
from orome_amd.moe import DeviceBuffer

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


class Pair:
    """A synthetic model resident on the GPU plus its oracle view."""

    def __init__(self, max_tokens=64, mutate=None, **kw):
        """mutate(img, om): edits the host image (e.g. router rows) before upload."""
        args = dict(layers=1, H=2048, E=256, K=8, M=512, S=512, seed=0)
        args.update(kw)
        self.img = orome_amd.synth_gguf(orome_amd.make_spec(**args))
        self.om = O.OracleModel(self.img)
        if mutate:
            mutate(self.img, self.om)
        self.gm = orome_amd.MoEModel(image=self.img, max_tokens=max_tokens)
        self.ctx = self.gm.ctx
        self.H = self.gm.H

    def inputs(self, T, seed):
        x = orome_amd.synth_normal(seed, 1, T * self.H).reshape(T, self.H)
        h = orome_amd.synth_normal(seed, 2, T * self.H).reshape(T, self.H)
        return x, h

    def run(self, layer, x, h, K=None, path=_lib.OROME_PATH_AUTO):
        T = x.shape[0]
        self.ctx.set_path(path)
        dx = DeviceBuffer.from_array(self.ctx, x)
        dh = DeviceBuffer.from_array(self.ctx, h)
        dout = DeviceBuffer(self.ctx, h.nbytes)
        self.gm.forward(layer, dx, dh, dout, T, K)
        self.ctx.sync()
        out = dout.download(np.float32, h.shape)
        return out, self.gm.debug_outputs(T, K)


@pytest.fixture(scope="module")
def base():
    banner("build base model H=2048 E=256 K=8 M=512 S=512 (Q4_K)")
    return Pair()


def assert_logits(dbg, rdbg):
    """Router logits against the oracle.  The winners' logits and the shared-gate
    logit are bit-exact on every path.  The two-pass large-batch router
    recomputes canonically only the experts that can win, so any other logit
    is an fp16 matrix-core approximation of the canonical value: it is checked
    against a tolerance far below the kernel's own error bound."""
    got, ref = dbg["logits"], rdbg["logits"]
    rows = np.arange(ref.shape[0])[:, None]
    win = rdbg["idx"]
    assert np.array_equal(got[rows, win].view(np.uint32), ref[rows, win].view(np.uint32)), "winner logits"
    assert np.array_equal(got[:, -1].view(np.uint32), ref[:, -1].view(np.uint32)), "shared-gate logit"
    scale = 1.0 + np.abs(ref).max(axis=1, keepdims=True)
    assert np.all(np.abs(got - ref) <= 5e-3 * scale), "approximate logits"


def check_routing(p, x, dbg, K, bias=None):
    om = p.om
    ref, rdbg = om.forward(0, x, np.zeros_like(x), K=K, debug=True)
    assert np.array_equal(dbg["logits"].view(np.uint32), rdbg["logits"].view(np.uint32)), "logits bits"
    assert np.array_equal(dbg["idx"], rdbg["idx"]), "expert indices"
    assert np.allclose(dbg["w"], rdbg["w"], rtol=2e-6, atol=1e-7)
    off, pairs = O.dispatch(rdbg["idx"], om.E)
    assert np.array_equal(dbg["offsets"], off), "dispatch offsets"
    assert np.array_equal(dbg["pairs"], pairs), "dispatch order"
    return rdbg


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_decode_forward_parity(base, T):
    banner("decode forward T=%d" % T)
    x, h = base.inputs(T, seed=100 + T)
    out, dbg = base.run(0, x, h)
    check_routing(base, x, dbg, 8)
    ref = base.om.forward(0, x, h)
    err = rel_l2(out - h, ref - h)
    print("T=%d rel_l2=%.3e" % (T, err))
    assert err < TOL


@pytest.mark.parametrize("T", [8, 3])
def test_forward_after_injected_failure(base, T):
    """A forward that fails between launches (test hook: the router's arrival
    counter is left torn, then the call returns an error) is followed by a
    forward whose routing is bit-exact and whose output is within tolerance
    of the oracle: the failing entry point returned the kernel-carried state
    to its initial value."""
    banner("forward after an injected failure T=%d" % T)
    x, h = base.inputs(T, seed=900 + T)
    base.ctx.set_path(_lib.OROME_PATH_AUTO)
    dx, dh, dout = DeviceBuffer.from_array(base.ctx, x), DeviceBuffer.from_array(base.ctx, h), DeviceBuffer(base.ctx, h.nbytes)
    check(lib.orome_hip_debug_inject_failure(base.ctx.handle), "inject")
    with pytest.raises(_lib.OromeError, match="injected failure"):
        base.gm.forward(0, dx, dh, dout, T)
    base.ctx.sync()
    out, dbg = base.run(0, x, h)
    check_routing(base, x, dbg, 8)
    ref = base.om.forward(0, x, h)
    assert rel_l2(out - h, ref - h) < TOL


@pytest.mark.parametrize("T,path", [(1, _lib.OROME_PATH_AUTO), (4, _lib.OROME_PATH_AUTO),
                                    (3, _lib.OROME_PATH_GEMV), (40, _lib.OROME_PATH_AUTO)])
def test_combine_residual_copy_and_sumsq_parts(base, T, path):
    """The combine's engine-level outputs (moe_combine_copy_sq_k8,
    inference/src/shaders.metal:1079-1135): residual_out is h_out bit for bit
    and each 256-column Sigma h^2 part equals the oracle's canonical dot of
    that block of the GPU's own h_out, bit for bit; h_out itself is unchanged
    by asking for them.  T=1 takes the fused down+combine and a separate parts
    kernel, T=4 the small-batch combine, T=3 on the GEMV path the GEMV down
    with the combine, T=40 the MFMA path."""
    banner("combine outputs T=%d path=%d" % (T, path))
    base.ctx.set_path(path)
    x, h = base.inputs(T, seed=900 + T)
    dx = DeviceBuffer.from_array(base.ctx, x)
    dh = DeviceBuffer.from_array(base.ctx, h)
    d1, d2, dr = (DeviceBuffer(base.ctx, h.nbytes) for _ in range(3))
    dp = DeviceBuffer(base.ctx, T * (base.H // 256) * 4)
    base.gm.forward(0, dx, dh, d1, T)
    base.gm.forward(0, dx, dh, d2, T, residual_out=dr, sumsq_parts=dp)
    base.ctx.sync()
    o1, o2, res = (d.download(np.float32, h.shape) for d in (d1, d2, dr))
    parts = dp.download(np.float32, (T, base.H // 256))
    base.ctx.set_path(_lib.OROME_PATH_AUTO)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(res.view(np.uint32), o2.view(np.uint32))
    ref = O.sumsq_parts(o2)
    assert np.array_equal(parts.view(np.uint32), ref.view(np.uint32))
    assert np.allclose(parts.astype(np.float64).sum(1), (o2.astype(np.float64) ** 2).sum(1), rtol=1e-5)


def test_decode_repeat_is_deterministic(base):
    banner("decode determinism")
    x, h = base.inputs(4, seed=7)
    a, _ = base.run(0, x, h)
    b, _ = base.run(0, x, h)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("K", [1, 4, 16])
def test_decode_other_k(base, K):
    banner("decode K=%d" % K)
    x, h = base.inputs(2, seed=300 + K)
    out, dbg = base.run(0, x, h, K=K)
    check_routing(base, x, dbg, K)
    ref = base.om.forward(0, x, h, K=K)
    assert rel_l2(out - h, ref - h) < TOL


@pytest.mark.parametrize("kw,T", [(dict(down=14, zipf=True, seed=1), 1),
                                   (dict(down=14, zipf=True, seed=1), 8),
                                   (dict(shared=8, seed=2), 4),
                                   (dict(shared=8, shared_down=14, seed=3), 3),
                                   (dict(S=0, seed=4), 2),
                                   (dict(down=13, seed=15), 1), (dict(down=13, shared_down=13, seed=16), 2),
                                   (dict(down=13, shared=8, seed=17), 1)])
def test_decode_variants(kw, T):
    banner("decode variant %s T=%d" % (kw, T))
    p = Pair(**kw)
    x, h = p.inputs(T, seed=500 + T)
    out, dbg = p.run(0, x, h)
    check_routing(p, x, dbg, 8)
    ref = p.om.forward(0, x, h)
    err = rel_l2(out - h, ref - h)
    print("variant rel_l2=%.3e" % err)
    assert err < TOL
    p.gm.close()


@pytest.mark.parametrize("E", [64, 128, 512, 1024])
def test_decode_expert_counts(E):
    """The one-token gate/up at every width of a lane's expert list (1, 2, 8
    and 16 experts a lane; 256 is the base model's 4): routing and dispatch
    bit-exact, output within tolerance of the oracle, at T=1 (selection folded
    into the gate/up, the down + combine kernel) and T=2."""
    banner("decode E=%d" % E)
    p = Pair(max_tokens=4, E=E, seed=70 + E % 97)
    for T in (1, 2):
        x, h = p.inputs(T, seed=700 + T)
        out, dbg = p.run(0, x, h)
        check_routing(p, x, dbg, 8)
        ref = p.om.forward(0, x, h)
        assert rel_l2(out - h, ref - h) < TOL, T
    p.gm.close()


def test_topk_teacher_forced(base):
    banner("teacher-forced top-k")
    rng = np.random.default_rng(1)
    T, E = 64, 256
    lg = rng.standard_normal((T, E + 1)).astype(np.float32)
    lg[:16] = np.round(lg[:16] * 2) / 2  # heavy ties
    lg[16, :E] = 0.0
    lg[17, :E] = -0.0
    lg[17, 9] = 0.0
    lg[18, :E] = -np.inf
    lg[18, 77] = 1.0
    bias = rng.standard_normal(E).astype(np.float32)
    ctx = base.ctx
    for b in (None, bias):
        for K in (1, 8, 16):
            dl = DeviceBuffer.from_array(ctx, lg)
            db = DeviceBuffer.from_array(ctx, b) if b is not None else None
            di = DeviceBuffer(ctx, T * K * 4)
            dw = DeviceBuffer(ctx, T * K * 4)
            check(lib.orome_moe_topk(ctx.handle, dl.ptr, db.ptr if db else None, T, E, K, di.ptr, dw.ptr))
            ctx.sync()
            idx = di.download(np.int32, (T, K))
            w = dw.download(np.float32, (T, K))
            ridx, rw, _ = O.topk(lg, b, K)
            assert np.array_equal(idx, ridx)
            ok = np.isfinite(rw)
            assert np.allclose(w[ok], rw[ok], rtol=2e-6, atol=1e-7)


def _tie_group(img, om):
    """Ten identical router rows scaled by 10: for about a quarter of the
    tokens their logit is among the K = 8 largest, and the winners then take
    some of the ten exact ties (the lowest ids must win)."""
    W = om.array("blk.0.ffn_gate_inp.weight", np.float32).reshape(om.E, om.H)
    W[16:26] = W[16] * 10


@pytest.mark.parametrize("T", [1, 2, 8])
def test_decode_planted_ties(T):
    """Decode with exact ties at the top-K boundary: the one-token gate/up
    (selection folded in), the two-token GEMV routing and the small-batch
    routing select what the oracle selects, bit for bit, and the outputs
    match."""
    banner("decode with a planted tie group, T=%d" % T)
    p = Pair(mutate=_tie_group, seed=71)
    split = 0
    for i in range(48 // T):
        x, h = p.inputs(T, seed=700 + i)
        out, dbg = p.run(0, x, h)
        rdbg = check_routing(p, x, dbg, 8)
        split += int(np.sum(np.isin(rdbg["idx"], np.arange(16, 26)).sum(axis=1) >= 1))
        ref = p.om.forward(0, x, h)
        assert rel_l2(out - h, ref - h) < TOL
    print("tokens whose winners take part of the tie group: %d" % split)
    assert split >= 4  # the planted case is exercised
    p.gm.close()


@pytest.mark.parametrize("fmt_name,kw", [("Q4_K", {}), ("Q5_K", dict(down=13)), ("Q6_K", dict(down=14)),
                                         ("Q8_0", dict(shared=8))])
def test_dequant_bit_exact(fmt_name, kw):
    banner("dequant %s" % fmt_name)
    p = Pair(E=8, **kw)
    om = p.om
    name, rows, n = {"Q4_K": ("blk.0.ffn_gate_exps.weight", 8 * 512, 2048),
                     "Q5_K": ("blk.0.ffn_down_exps.weight", 8 * 2048, 512),
                     "Q6_K": ("blk.0.ffn_down_exps.weight", 8 * 2048, 512),
                     "Q8_0": ("blk.0.ffn_gate_shexp.weight", 512, 2048)}[fmt_name]
    dims, typ, off, nb = om.tensors[name]
    fmt = O.GGML_TO_FMT[typ]
    ref = O.decode_rows(fmt, p.img[off:off + nb], rows, n)
    ctx = p.ctx
    out = DeviceBuffer(ctx, rows * n * 4)
    out16 = DeviceBuffer(ctx, rows * n * 2)
    src = p.gm.tensor_device_ptr(name)
    check(lib.orome_dequant_rows(ctx.handle, fmt, src, rows, n, out.ptr))
    check(lib.orome_dequant_rows_f16(ctx.handle, fmt, src, rows, n, out16.ptr))
    ctx.sync()
    got = out.download(np.float32, (rows, n))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got16 = out16.download(np.uint16, (rows, n))
    assert np.array_equal(got16, ref.astype(np.float16).view(np.uint16))
    p.gm.close()


def test_dequant_q4k_one_hot_fields(base):
    """The one-hot Q4_K scale and min fields of the CPU pins (decoded values
    written out by hand from format.m:41-64, sub-blocks 4..7 included)
    through the GPU dequant: fp32 bit for bit."""
    banner("dequant Q4_K one-hot scale/min fields")
    from test_oracle import MIN_ONE_HOT, SCALE_ONE_HOT, _q4k_block
    blocks, expect = [], []
    for table, nib, sign in ((MIN_ONE_HOT, 9, -1), (SCALE_ONE_HOT, 3, 3)):
        for byte, val, e in table:
            sc = [0] * 12
            sc[byte] = val
            blocks.append(_q4k_block(1.0, 1.0, sc, nib))
            expect.append(sign * np.repeat(np.float32(e), 32))
    rows = len(blocks)
    src = DeviceBuffer.from_array(base.ctx, np.frombuffer(b"".join(blocks), np.uint8).copy())
    out = DeviceBuffer(base.ctx, rows * 256 * 4)
    check(lib.orome_dequant_rows(base.ctx.handle, O.Q4_K, src.ptr, rows, 256, out.ptr))
    base.ctx.sync()
    got = out.download(np.float32, (rows, 256))
    assert np.array_equal(got, np.array(expect, np.float32))


@pytest.mark.parametrize("T", [1, 2, 5, 12, 16])
def test_layer_forward_and_stack(T):
    """T=1, 2: GEMV kernels; T=5, 12, 16: small-batch routing (RMSNorm in the
    router, 9..16 tokens with four waves per router row) feeding the
    small-tile grouped GEMMs."""
    banner("layer/stack forward, 3 layers, mixed Q6_K down, T=%d" % T)
    p = Pair(layers=3, q6k_every=2, seed=9, centered=True)
    h0 = (orome_amd.synth_normal(9, 3, T * p.H) * 4).reshape(T, p.H)
    dh = DeviceBuffer.from_array(p.ctx, h0)
    h = h0.copy()
    # layer by layer, teacher-forced: the oracle applies layer l to the GPU's h_l
    for l in range(3):
        p.gm.layer_forward(l, dh, T)
        p.ctx.sync()
        got = dh.download(np.float32, (T, p.H))
        dbg = p.gm.debug_outputs(T)
        xn = p.om.rmsnorm(l, h)
        ref, rdbg = p.om.forward(l, xn, h, debug=True)
        assert np.array_equal(dbg["logits"].view(np.uint32), rdbg["logits"].view(np.uint32))
        assert np.array_equal(dbg["idx"], rdbg["idx"])
        err = rel_l2(got - h, ref - h)
        print("layer %d rel_l2=%.3e" % (l, err))
        assert err < TOL
        h = got
    # the stack entry point computes the same as the three calls
    dh2 = DeviceBuffer.from_array(p.ctx, h0)
    p.gm.stack_forward(dh2, T)
    p.ctx.sync()
    assert np.array_equal(dh2.download(np.float32, (T, p.H)), h)
    p.gm.close()


def test_stack_prefill_fused_norm():
    """On the MFMA path the stack fuses each layer's combine with the next
    layer's RMSNorm: three layers at T=100 equal three separate layer calls
    bit for bit, and the last layer's logits (computed from the fused norm)
    equal the oracle's on the same input."""
    banner("stack forward with fused next-layer RMSNorm, 3 layers, T=100")
    p = Pair(max_tokens=100, layers=3, q6k_every=2, seed=19, centered=True)
    T = 100
    h0 = (orome_amd.synth_normal(19, 3, T * p.H) * 4).reshape(T, p.H)
    dh = DeviceBuffer.from_array(p.ctx, h0)
    for l in range(3):
        p.gm.layer_forward(l, dh, T)
        if l == 1:
            p.ctx.sync()
            h_in_last = dh.download(np.float32, (T, p.H))
    p.ctx.sync()
    want = dh.download(np.float32, (T, p.H))
    dh2 = DeviceBuffer.from_array(p.ctx, h0)
    p.gm.stack_forward(dh2, T)
    p.ctx.sync()
    assert np.array_equal(dh2.download(np.float32, (T, p.H)), want)
    dbg = p.gm.debug_outputs(T)
    xn = p.om.rmsnorm(2, h_in_last)
    _, rdbg = p.om.forward(2, xn, h_in_last, debug=True)
    assert np.array_equal(dbg["idx"], rdbg["idx"])
    assert_logits(dbg, rdbg)
    p.gm.close()


def test_graph_replay_matches_eager(base):
    """Capture three forwards in a HIP graph, replay it several times with eager
    work and synchronisations in between, and check every replay."""
    banner("graph replay vs eager")
    import ctypes as C
    ctx = base.ctx
    ins = [base.inputs(T, seed=900 + T) for T in (1, 4, 8)]
    bufs = [(DeviceBuffer.from_array(ctx, x), DeviceBuffer.from_array(ctx, h), DeviceBuffer(ctx, h.nbytes))
            for x, h in ins]
    ctx.set_path(_lib.OROME_PATH_AUTO)
    eager = []
    for (x, h), (dx, dh, do) in zip(ins, bufs):
        base.gm.forward(0, dx, dh, do, x.shape[0])
        ctx.sync()
        eager.append(do.download(np.float32, h.shape))
    check(lib.orome_hip_capture_begin(ctx.handle))
    for (x, h), (dx, dh, do) in zip(ins, bufs):
        base.gm.forward(0, dx, dh, do, x.shape[0])
    ex = C.c_void_p()
    check(lib.orome_hip_capture_end(ctx.handle, C.byref(ex)))
    for rep in range(3):
        for (_, h), (_, _, do) in zip(ins, bufs):
            do.upload(np.zeros_like(h))
        check(lib.orome_hip_graph_launch(ctx.handle, ex))
        ctx.sync()
        for e, (x, h), (_, _, do) in zip(eager, ins, bufs):
            assert np.array_equal(do.download(np.float32, h.shape), e), "replay %d" % rep
        # eager work between replays
        x, h = ins[1]
        base.gm.forward(0, bufs[1][0], bufs[1][1], bufs[1][2], x.shape[0])
        ctx.sync()
    check(lib.orome_hip_graph_destroy(ex))


@pytest.mark.parametrize("T", [1, 512])
def test_kernel_timing_stamps(T):
    """orome_hip_kernel_timing: every gate/up block writes a start and an end
    stamp (end >= start, spans of a few microseconds up to milliseconds), and
    the stamped launches compute bit-identical outputs."""
    banner("gate/up launch stamps T=%d" % T)
    p = Pair(max_tokens=T)
    x, h = p.inputs(T, seed=300 + T)
    ref, _ = p.run(0, x, h)
    nb = 16384
    buf = DeviceBuffer(p.ctx, nb * 2 * 8)
    buf.upload(np.zeros(nb * 2, np.uint64))
    check(lib.orome_hip_kernel_timing(p.ctx.handle, buf.ptr, nb), "kernel_timing")
    try:
        out, _ = p.run(0, x, h)
    finally:
        check(lib.orome_hip_kernel_timing(p.ctx.handle, None, 0), "kernel_timing")
    v = buf.download(np.uint64, (nb, 2)).astype(np.int64)
    buf.free()
    ok = v[:, 0] > 0
    assert ok.sum() > 0
    assert np.all(v[ok, 1] >= v[ok, 0])
    span_us = (v[ok, 1].max() - v[ok, 0].min()) * 0.01
    print("T=%d blocks=%d span=%.2f us" % (T, ok.sum(), span_us))
    assert 0.5 < span_us < 5000
    assert np.array_equal(out, ref)
    p.gm.close()


@pytest.mark.parametrize("T", [1, 8, 512])
def test_ggml_q4k_packing_file(T):
    """A file whose Q4_K tensors use the ggml scale packing (and declare it)
    gives bit for bit the outputs of the same weights in the reference
    packing: the upload permutes the scale bytes once and the kernels keep
    one decoder.  Read as the reference packing instead, it gives different
    outputs (the option is not a no-op)."""
    banner("ggml Q4_K packing, T=%d" % T)
    kw = dict(layers=1, H=2048, E=256, K=8, M=512, S=512, seed=66)
    outs = []
    for ggml, layout in ((False, _lib.OROME_Q4K_LAYOUT_FILE), (True, _lib.OROME_Q4K_LAYOUT_FILE),
                         (True, _lib.OROME_Q4K_LAYOUT_REFERENCE)):
        img = orome_amd.synth_gguf(orome_amd.make_spec(q4k_ggml=ggml, **kw))
        gm = orome_amd.MoEModel(image=img, max_tokens=T, q4k_layout=layout)
        x = orome_amd.synth_normal(80 + T, 1, T * 2048).reshape(T, 2048)
        h = orome_amd.synth_normal(80 + T, 2, T * 2048).reshape(T, 2048)
        dx, dh, do = (DeviceBuffer.from_array(gm.ctx, x), DeviceBuffer.from_array(gm.ctx, h),
                      DeviceBuffer(gm.ctx, h.nbytes))
        gm.forward(0, dx, dh, do, T)
        gm.ctx.sync()
        outs.append(do.download(np.float32, h.shape))
        if len(outs) == 1:
            ref = O.OracleModel(img).forward(0, x, h)
            assert rel_l2(outs[0] - h, ref - h) < TOL
        gm.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert not np.array_equal(outs[0], outs[2])


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", ["mini_q4k", "mini_q6k_down_zipf", "mini_q5k_down_q8_shared", "mini_no_shared_k8",
                                  "config0_b1"])
def test_gpu_matches_golden_fixture(name):
    """The HIP path against the committed oracle fixtures (not the oracle at
    run time): router logits, indices and dispatch bit-exact, weights to
    rounding, h_out within 1e-3 relative L2; forced GEMV and MFMA paths both."""
    banner("golden fixture %s" % name)
    f = np.load(os.path.join(GOLDEN, name + ".npz"))
    kw = json.loads(str(f["spec"]))
    img = orome_amd.synth_gguf(orome_amd.make_spec(**kw))
    assert hashlib.sha256(img.tobytes()).hexdigest() == str(f["image_sha256"])
    gm = orome_amd.MoEModel(image=img, max_tokens=16)
    x, h, K = f["x"], f["h"], int(f["K"])
    T = x.shape[0]
    gemv = T <= 8 and gm.cfg.moe_intermediate % 512 == 0  # the GEMV down kernels take in_dim % 512 == 0
    for path in (_lib.OROME_PATH_AUTO, _lib.OROME_PATH_MFMA) + ((_lib.OROME_PATH_GEMV,) if gemv else ()):
        gm.ctx.set_path(path)
        dx, dh, do = (DeviceBuffer.from_array(gm.ctx, x), DeviceBuffer.from_array(gm.ctx, h),
                      DeviceBuffer(gm.ctx, h.nbytes))
        gm.forward(0, dx, dh, do, T, K)
        gm.ctx.sync()
        out = do.download(np.float32, h.shape)
        dbg = gm.debug_outputs(T, K)
        assert np.array_equal(dbg["idx"], f["idx"]), path
        if path == _lib.OROME_PATH_MFMA:  # two-pass router: the winners' logits are the canonical ones
            assert_logits(dbg, dict(logits=f["logits"], idx=f["idx"]))
        else:
            assert np.array_equal(dbg["logits"].view(np.uint32), f["logits"].view(np.uint32)), path
        assert np.allclose(dbg["w"], f["w"], rtol=2e-6, atol=1e-7), path
        off, pairs = O.dispatch(f["idx"], gm.cfg.num_experts)
        assert np.array_equal(dbg["offsets"], off) and np.array_equal(dbg["pairs"], pairs), path
        err = rel_l2(out - h, f["out"] - h)
        print("%s path %d rel_l2 %.2e" % (name, path, err))
        assert err < TOL
    gm.close()
