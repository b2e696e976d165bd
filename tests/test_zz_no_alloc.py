"""GPU check of orome_moe_forward_noalloc (the entry point that allocates
nothing, with its scratch in a static per-GPU device array) against
orome_moe_forward on the same inputs, through the C ABI: calls in a row with
fewer tokens each time (8, 3, 2, 1: the folded small-batch router with its
arrival counter in the static array, the two-token GEMV path, and the
one-token path with routing folded into gate/up and the fused down +
combine), outputs, residual copy and sum-of-squares parts bit-identical to
orome_moe_forward (the same kernels on the same data; only the scratch
addresses differ), and within 1e-3 relative L2 of the oracle.  Routing is
not read back here (the array has no debug copy-out); the context path's
routing is pinned bit-exact by the other GPU tests."""
import ctypes as C

import numpy as np
import pytest

import orome_amd
import oracle as O
from conftest import banner
from orome_amd import _lib
from orome_amd._lib import lib
from orome_amd.moe import DeviceBuffer

pytestmark = pytest.mark.gpu


def _noalloc(gm, layer, dx, dh, dout, dres, dparts, T, K=8):
    """On the context's stream, so that the context's copies and syncs are
    ordered after it."""
    return lib.orome_moe_forward_noalloc(C.byref(gm.cfg), C.byref(gm.elrs[layer]), C.byref(gm.caches[layer]),
                                         dx.ptr, dh.ptr, dout.ptr, dres.ptr if dres else None,
                                         dparts.ptr if dparts else None, T, K, lib.orome_hip_get_stream(gm.ctx.handle))


def test_noalloc_matches_context_forward():
    banner("no-alloc forward: T=8, 3, 2, 1 against orome_moe_forward")
    img = orome_amd.synth_gguf(orome_amd.make_spec(layers=1, H=2048, E=256, K=8, M=512, S=512, seed=11))
    gm = orome_amd.MoEModel(image=img, max_tokens=16, pack=False)
    om = O.OracleModel(img)
    H = gm.H
    try:
        for T in (8, 3, 2, 1):
            x = orome_amd.synth_normal(70 + T, 1, T * H).reshape(T, H)
            h = orome_amd.synth_normal(70 + T, 2, T * H).reshape(T, H)
            dx, dh = DeviceBuffer.from_array(gm.ctx, x), DeviceBuffer.from_array(gm.ctx, h)
            d_ctx, d_na, d_res = (DeviceBuffer(gm.ctx, h.nbytes) for _ in range(3))
            d_pc, d_pn = (DeviceBuffer(gm.ctx, T * (H // 256) * 4) for _ in range(2))
            gm.forward(0, dx, dh, d_ctx, T, sumsq_parts=d_pc)
            gm.ctx.sync()
            rc = _noalloc(gm, 0, dx, dh, d_na, d_res, d_pn, T)
            assert rc == 0, lib.orome_last_error()
            gm.ctx.sync()
            assert lib.orome_hip_sync(gm.ctx.handle) == 0
            a = d_ctx.download(np.float32, h.shape)
            b = d_na.download(np.float32, h.shape)
            r = d_res.download(np.float32, h.shape)
            pa = d_pc.download(np.float32, (T, H // 256))
            pb = d_pn.download(np.float32, (T, H // 256))
            print("T=%d max|diff|=%g" % (T, float(np.abs(a - b).max())))
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "h_out differs from orome_moe_forward"
            assert np.array_equal(r.view(np.uint32), b.view(np.uint32)), "residual copy"
            assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32)), "sum-of-squares parts"
            ref = om.forward(0, x, h)
            err = float(np.linalg.norm(b - ref) / np.linalg.norm(ref - h))
            assert err < 1e-3, err
    finally:
        gm.close()


def test_noalloc_rejects_beyond_maximum():
    """More tokens than OROME_NOALLOC_MAX_TOKENS, and shapes whose scratch
    layout exceeds the static array, fail with OROME_EINVAL before any launch."""
    banner("no-alloc forward: limits")
    for H, T, what in ((512, 17, b"outside 1..16"), (8192, 1, b"bytes of scratch")):
        img = orome_amd.synth_gguf(orome_amd.make_spec(layers=1, H=H, E=16, K=4, M=256, S=256, seed=12))
        gm = orome_amd.MoEModel(image=img, max_tokens=32, pack=False)
        try:
            buf = DeviceBuffer(gm.ctx, 32 * H * 4)
            rc = lib.orome_moe_forward_noalloc(C.byref(gm.cfg), C.byref(gm.elrs[0]), C.byref(gm.caches[0]),
                                               buf.ptr, None, buf.ptr, None, None, T, 4, None)
            assert rc == -1, rc
            assert what in lib.orome_last_error(), lib.orome_last_error()
        finally:
            gm.close()
