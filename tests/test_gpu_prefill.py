"""GPU parity of the prefill path (router logits for many tokens, wave-per-token
top-k, LDS counting-sort dispatch, MFMA grouped GEMMs, combine) against the
C oracle.  Expert indices and dispatch order bit-exact; outputs within 1e-3
relative L2 (fp16 weight tiles: expected ~1e-4)."""
import numpy as np
import pytest

import orome_amd
import oracle as O
from conftest import banner
from orome_amd import _lib
from orome_amd._lib import lib
from orome_amd.moe import DeviceBuffer
from test_gpu_decode import Pair, assert_logits, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3


def run_and_check(p, T, seed, K=8, path=_lib.OROME_PATH_MFMA, tol=TOL):
    x, h = p.inputs(T, seed)
    out, dbg = p.run(0, x, h, K=K, path=path)
    ref, rdbg = p.om.forward(0, x, h, K=K, debug=True)
    assert np.array_equal(dbg["idx"], rdbg["idx"]), "expert indices"
    assert_logits(dbg, rdbg)
    assert np.allclose(dbg["w"], rdbg["w"], rtol=2e-6, atol=1e-7)
    off, pairs = O.dispatch(rdbg["idx"], p.om.E)
    assert np.array_equal(dbg["offsets"], off), "dispatch offsets"
    assert np.array_equal(dbg["pairs"], pairs), "dispatch order"
    err = rel_l2(out - h, ref - h)
    print("T=%d K=%d rel_l2=%.3e max_tokens_per_expert=%d" % (T, K, err, int(np.diff(off.astype(int)).max())))
    assert np.all(np.isfinite(out))
    assert err < tol
    return out, dbg


@pytest.fixture(scope="module")
def base():
    banner("prefill base model (Q4_K, E=256)")
    return Pair(max_tokens=2048, seed=21)


@pytest.mark.parametrize("T", [1, 5, 33, 100])
def test_mfma_path_small_batches(base, T):
    banner("mfma path T=%d" % T)
    run_and_check(base, T, seed=40 + T)


def test_mfma_path_k16(base):
    banner("mfma path T=64 K=16")
    run_and_check(base, 64, seed=77, K=16)


def test_prefill_512_balanced(base):
    banner("prefill T=512 balanced (config 2)")
    run_and_check(base, 512, seed=512, path=_lib.OROME_PATH_AUTO)


@pytest.mark.parametrize("T", [1500, 2048])
def test_prefill_2048_properties(base, T):
    """Full-size checks that need no oracle run: dispatch is a permutation
    grouped by expert in ascending pair order, offsets are the histogram
    prefix, and every token's weights sum to one.  Above 1024 tokens the
    dispatch runs in three launches over 256-token blocks; 1500 leaves the
    last block ragged."""
    banner("prefill T=%d properties" % T)
    x, h = base.inputs(T, seed=T)
    out, dbg = base.run(0, x, h)
    idx, w, off, pairs = dbg["idx"], dbg["w"], dbg["offsets"].astype(np.int64), dbg["pairs"]
    assert np.array_equal(np.sort(pairs), np.arange(T * 8))
    flat = idx.reshape(-1)
    assert np.array_equal(np.diff(off), np.bincount(flat, minlength=256))
    for e in range(256):
        seg = pairs[off[e]:off[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg.astype(np.int64)) > 0)
    assert np.allclose(w.sum(axis=1), 1, atol=1e-5)
    assert np.all(np.isfinite(out))
    # a sample of every 32nd token of the same call against the oracle (rows
    # are independent)
    sel = np.arange(0, T, 32)
    ref = base.om.forward(0, x[sel], h[sel])
    assert rel_l2(out[sel] - h[sel], ref - h[sel]) < TOL


@pytest.mark.parametrize("kw,T", [(dict(down=13, seed=32), 512), (dict(down=13, shared=8, seed=33), 2048),
                                   (dict(down=13, shared_down=13, seed=34), 12),
                                   (dict(down=14, zipf=True, seed=31), 512),
                                   (dict(shared=8, seed=32), 64),
                                   (dict(shared=8, shared_down=14, seed=33), 48),
                                   (dict(S=0, seed=34), 40)])
def test_prefill_variants(kw, T):
    banner("prefill variant %s T=%d" % (kw, T))
    p = Pair(max_tokens=T, **kw)
    run_and_check(p, T, seed=600 + T, path=_lib.OROME_PATH_MFMA)
    p.gm.close()


def test_prefill_matches_decode_path(base):
    """The GEMV and MFMA paths agree on the same 8 tokens (both within the
    tolerance of the oracle; fp16 weight tiles vs exact fp32 weights), and
    the AUTO path at 8 tokens (small-batch routing feeding the small-tile
    grouped GEMMs) equals the MFMA path bit for bit: same tiles, same fp16
    activations, same GEMM kernels."""
    banner("mfma vs gemv vs auto, T=8")
    x, h = base.inputs(8, seed=8)
    a, da = base.run(0, x, h, path=_lib.OROME_PATH_GEMV)
    b, db = base.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    c, dc = base.run(0, x, h, path=_lib.OROME_PATH_AUTO)
    assert np.array_equal(da["idx"], db["idx"]) and np.array_equal(da["pairs"], db["pairs"])
    assert np.array_equal(dc["idx"], db["idx"]) and np.array_equal(dc["pairs"], db["pairs"])
    assert rel_l2(b - h, a - h) < TOL
    assert np.array_equal(c, b), "small-batch grouped GEMMs vs MFMA path"


def test_persistent_gemm_bit_identical(base, monkeypatch):
    """The persistent GEMMs (a block walks its (tile, row block) units back to
    back; the weight ring and the activation chunks run on across unit
    boundaries) compute every unit exactly as the per-tile kernels do:
    outputs are bit-identical with the default grid, with the per-tile
    kernels (OROME_GEMM_PERSIST_BLOCKS=0) and with an 8-block grid, where
    each block walks many units.  T=2048 runs the big-tile kernels, T=512
    the small-tile down projection."""
    for T in (512, 2048):
        banner("persistent GEMM vs per-tile, T=%d" % T)
        x, h = base.inputs(T, seed=4096 + T)
        outs = {}
        for blocks in (None, "0", "8"):
            if blocks is None:
                monkeypatch.delenv("OROME_GEMM_PERSIST_BLOCKS", raising=False)
            else:
                monkeypatch.setenv("OROME_GEMM_PERSIST_BLOCKS", blocks)
            outs[blocks], _ = base.run(0, x, h, path=_lib.OROME_PATH_MFMA)
        monkeypatch.delenv("OROME_GEMM_PERSIST_BLOCKS", raising=False)
        assert np.array_equal(outs[None], outs["0"]), "T=%d" % T
        assert np.array_equal(outs["8"], outs["0"]), "T=%d" % T
        sel = np.arange(5, T, 64)
        ref = base.om.forward(0, x[sel], h[sel])
        assert rel_l2(outs[None][sel] - h[sel], ref - h[sel]) < TOL


@pytest.mark.parametrize("shared_down", [14, 12])
def test_persistent_gemm_zipf_q6k(monkeypatch, shared_down):
    """Skewed routing (a few experts with many tiles, many with none) and a
    Q6_K down projection through a 16-block persistent grid, against the
    oracle and bit-identical to the per-tile kernels.  With a Q4_K shared
    down the routed and shared tiles are walked by two launches."""
    banner("persistent GEMM, Zipf T=512, Q6_K down, shared down type %d" % shared_down)
    p = Pair(max_tokens=512, down=14, shared_down=shared_down, zipf=True, seed=35)
    monkeypatch.setenv("OROME_GEMM_PERSIST_BLOCKS", "16")
    out, _ = run_and_check(p, 512, seed=1512, path=_lib.OROME_PATH_MFMA)
    monkeypatch.setenv("OROME_GEMM_PERSIST_BLOCKS", "0")
    x, h = p.inputs(512, seed=1512)
    ref, _ = p.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    monkeypatch.delenv("OROME_GEMM_PERSIST_BLOCKS", raising=False)
    assert np.array_equal(out, ref)
    p.gm.close()


def test_tile_major_copies_bit_identical(base):
    """orome_hip_pack_layer's tile-major copies hold the same Q4_K bytes in
    another order, so the grouped GEMMs give bit-identical outputs with and
    without them: T=100 (small and big tiles, per-tile kernels) and T=2048
    (persistent kernels)."""
    banner("tile-major copies vs row-major, T=100 and T=2048")
    outs = {}
    for T in (100, 2048):
        x, h = base.inputs(T, seed=7000 + T)
        packed, _ = base.run(0, x, h, path=_lib.OROME_PATH_MFMA)
        base.gm.unpack()
        try:
            plain, _ = base.run(0, x, h, path=_lib.OROME_PATH_MFMA)
        finally:
            base.gm.pack_layers()
        assert np.array_equal(packed, plain), "T=%d" % T
        outs[T] = packed
    sel = np.arange(3, 2048, 128)
    x, h = base.inputs(2048, seed=9048)
    ref = base.om.forward(0, x[sel], h[sel])
    assert rel_l2(outs[2048][sel] - h[sel], ref - h[sel]) < TOL


def test_tile_major_q6k_down_and_q8_shared():
    """Q6_K and Q5_K down projections get tile-major copies (routed only, and
    routed + shared); a Q8_0 shared expert gets tile-major Q8_0 copies of its
    gate, up and down.  Each matches the oracle and its unpacked run bit for
    bit."""
    banner("tile-major copies: Q6_K / Q5_K down, Q8_0 shared")
    for kw, T in ((dict(down=14, seed=36), 300), (dict(down=14, shared_down=14, seed=38), 96),
                  (dict(shared=8, seed=37), 64), (dict(down=13, shared_down=13, seed=39), 200),
                  (dict(down=13, shared=8, E=32, seed=40), 300)):
        p = Pair(max_tokens=T, **kw)
        out, _ = run_and_check(p, T, seed=1700 + T, path=_lib.OROME_PATH_MFMA)
        p.gm.unpack()
        x, h = p.inputs(T, seed=1700 + T)
        plain, _ = p.run(0, x, h, path=_lib.OROME_PATH_MFMA)
        assert np.array_equal(out, plain)
        p.gm.close()


def _plant_ties(img, om):
    """Router rows with exact ties (8 identical rows), near-ties below fp16
    resolution (16 rows scaled by 1 + i 2^-22) and 16 rows perturbed by about
    1e-7, each group scaled by 1.5 so that it often reaches the top K."""
    W = om.array("blk.0.ffn_gate_inp.weight", np.float32).reshape(om.E, om.H)
    rng = np.random.default_rng(57)
    W[16:24] = W[16] * 1.5
    W[32:48] = ((W[32].astype(np.float64) * 1.5)[None, :] * (1 + np.arange(16)[:, None] * 2.0 ** -22)).astype(np.float32)
    W[64:80] = W[64] * 1.5 + (rng.standard_normal((16, om.H)) * 1e-7).astype(np.float32)


def _same_routing(a, b):
    assert np.array_equal(a["idx"], b["idx"])
    assert np.array_equal(a["w"].view(np.uint32), b["w"].view(np.uint32))
    assert np.array_equal(a["offsets"], b["offsets"])
    assert np.array_equal(a["pairs"], b["pairs"])
    rows = np.arange(a["idx"].shape[0])[:, None]
    assert np.array_equal(a["logits"][rows, a["idx"]].view(np.uint32), b["logits"][rows, b["idx"]].view(np.uint32))
    assert np.array_equal(a["logits"][:, -1].view(np.uint32), b["logits"][:, -1].view(np.uint32))


def test_two_pass_router_ties(monkeypatch):
    """Exact ties and near-ties at the top-K boundary: the two-pass router
    (matrix-core approximation, canonical recomputation of the candidates)
    selects exactly what the oracle and the one-pass canonical router select."""
    banner("two-pass router, planted ties, T=256")
    p = Pair(max_tokens=256, mutate=_plant_ties, seed=57)
    T = 256
    x, h = p.inputs(T, seed=58)
    ref, rdbg = p.om.forward(0, x, h, debug=True)
    lg = np.sort(rdbg["logits"][:, :-1], axis=1)[:, ::-1]
    close = int(np.sum(np.min(np.diff(-lg[:, :9], axis=1), axis=1) < 1e-4))
    ties = int(np.sum(np.isin(rdbg["idx"], np.arange(17, 24)).any(axis=1)))
    print("tokens with top-9 gaps < 1e-4: %d, with tied rows among the winners: %d" % (close, ties))
    assert close >= 20 and ties >= 10  # the planted cases are exercised
    out, dbg = run_and_check(p, T, seed=58, path=_lib.OROME_PATH_MFMA)
    monkeypatch.setenv("OROME_ROUTE_EXACT", "1")
    out1, dbg1 = p.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    assert np.array_equal(dbg1["logits"].view(np.uint32), rdbg["logits"].view(np.uint32)), "one-pass logits bits"
    _same_routing(dbg, dbg1)
    assert np.array_equal(out, out1)
    p.gm.close()


@pytest.mark.parametrize("T", [512, 2048])
def test_two_pass_router_matches_one_pass(base, monkeypatch, T):
    """Full-size property check without the oracle: the two routers produce
    the same routing, the same winner and shared-gate logits and the same
    layer output, bit for bit."""
    banner("two-pass vs one-pass router T=%d" % T)
    x, h = base.inputs(T, seed=900 + T)
    out, dbg = base.run(0, x, h)
    monkeypatch.setenv("OROME_ROUTE_EXACT", "1")
    out1, dbg1 = base.run(0, x, h)
    _same_routing(dbg, dbg1)
    assert np.array_equal(out, out1)


def test_persistent_down_mixed_formats_2048(monkeypatch):
    """Q6_K routed down with a Q4_K shared down at T=2048 (the shared tiles
    then end the big-tile list): the two persistent walks equal the per-tile
    kernels bit for bit, and a token sample matches the oracle."""
    banner("persistent down, Q6_K routed + Q4_K shared, T=2048")
    p = Pair(max_tokens=2048, down=14, shared_down=12, seed=36)
    x, h = p.inputs(2048, seed=2036)
    out, _ = p.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    monkeypatch.setenv("OROME_GEMM_PERSIST_BLOCKS", "0")
    ref1, _ = p.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    monkeypatch.delenv("OROME_GEMM_PERSIST_BLOCKS", raising=False)
    assert np.array_equal(out, ref1)
    sel = np.arange(0, 2048, 32)
    ref = p.om.forward(0, x[sel], h[sel])
    assert rel_l2(out[sel] - h[sel], ref - h[sel]) < TOL
    p.gm.close()


@pytest.mark.parametrize("T", [12, 16])
def test_small_batch_path_up_to_16(base, T):
    """9..16 tokens take the small-batch routing feeding the small-tile
    grouped GEMMs under AUTO: routing bit-exact and output within tolerance
    of the oracle, and equal bit for bit to the MFMA path (same tiles, same
    fp16 activations, same GEMM kernels)."""
    banner("small-batch path, T=%d" % T)
    out, dbg = run_and_check(base, T, seed=1200 + T, path=_lib.OROME_PATH_AUTO)
    x, h = base.inputs(T, seed=1200 + T)
    ref, _ = base.run(0, x, h, path=_lib.OROME_PATH_MFMA)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("kw,T,K", [(dict(S=0, seed=61), 12, 8), (dict(S=0, seed=62), 8, 8),
                                    (dict(seed=63), 16, 16)])
def test_small_batch_path_edges(kw, T, K):
    """The small-batch path without a shared expert (T=8, 12) and at its
    single-block dispatch limit T K = 256 (T=16, K=16): routing bit-exact,
    output within tolerance of the oracle and bit for bit the MFMA path's."""
    banner("small-batch edge %s T=%d K=%d" % (kw, T, K))
    p = Pair(max_tokens=64, **kw)
    out, _ = run_and_check(p, T, seed=1300 + T, K=K, path=_lib.OROME_PATH_AUTO)
    x, h = p.inputs(T, seed=1300 + T)
    ref, _ = p.run(0, x, h, K=K, path=_lib.OROME_PATH_MFMA)
    assert np.array_equal(out, ref)
    p.gm.close()


@pytest.mark.parametrize("T", [12, 512, 2048])
def test_q8_shared_expert_registered(T):
    """The reference's 35B layout: a Q8_0 shared expert (gate, up and down).
    Registration repacks the routed matrices, the router and the Q8_0 shared
    matrices (tile-major Q8_0), and the grouped GEMMs read them (T=2048:
    persistent kernels, one walk over the routed tiles and one over the
    shared).  Routing bit-exact, output within
    tolerance of the oracle and bit-identical to the unregistered layer; at
    T=512 the two-pass router runs (some non-winning logits are its
    approximations, not the canonical values)."""
    banner("Q8_0 shared expert, registered layer, T=%d" % T)
    p = Pair(max_tokens=T, shared=8, seed=64)
    x, h = p.inputs(T, seed=1400 + T)
    if T <= 512:
        out, dbg = run_and_check(p, T, seed=1400 + T, path=_lib.OROME_PATH_AUTO)
        if T == 512:
            ref, rdbg = p.om.forward(0, x, h, debug=True)
            assert not np.array_equal(dbg["logits"].view(np.uint32), rdbg["logits"].view(np.uint32)), \
                "registered Q8_0-shared layer was routed in one pass"
    else:
        out, dbg = p.run(0, x, h, path=_lib.OROME_PATH_AUTO)
        sel = np.arange(5, T, 97)
        ref = p.om.forward(0, x[sel], h[sel])
        assert rel_l2(out[sel] - h[sel], ref - h[sel]) < TOL
    p.gm.unpack()
    plain, _ = p.run(0, x, h, path=_lib.OROME_PATH_AUTO)
    assert np.array_equal(out, plain)
    p.gm.close()


def f16(x):
    return np.asarray(x, np.float64).astype(np.float16)


def mfma_weights_model(fmt_blocks):
    """The documented in-register fp16 dequant of the grouped GEMMs, emulated
    in numpy (every step's rounding explicit) for whole matrices:
      Q4_K, Q5_K  t = q sc (exact in fp16), w = fp16(t d - fp16(dmin m))
      Q6_K        w = fp16(fp16(q sc) d)
      Q8_0        w = fp16(q d)
    blocks -> [rows, cols] float16."""
    fmt, blocks, rows, cols = fmt_blocks
    if fmt in ("Q4_K", "Q5_K"):
        bb = 144 if fmt == "Q4_K" else 176
        b = blocks.reshape(-1, bb)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        from test_oracle import layout_table_np
        sc, mn = layout_table_np(b[:, 4:16])
        out = np.empty((len(b), 256), np.float16)
        for j in range(4):
            for h in range(2):
                s = 2 * j + h
                if fmt == "Q4_K":
                    q = (b[:, 16 + 32 * j:16 + 32 * j + 32].astype(np.int64) >> (4 * h)) & 0xF
                else:
                    qh = b[:, 16:48].astype(np.int64)
                    q = ((b[:, 48 + 32 * j:48 + 32 * j + 32].astype(np.int64) >> (4 * h)) & 0xF) + \
                        16 * ((qh >> (2 * j + h)) & 1)
                t = q * sc[:, s][:, None]                      # exact (< 2048)
                mb = f16(dmin * mn[:, s]).astype(np.float64)   # fp16(dmin m)
                out[:, 64 * j + 32 * h:64 * j + 32 * h + 32] = f16(t * d[:, None] - mb[:, None])
        return out.reshape(rows, cols)
    if fmt == "Q6_K":
        b = blocks.reshape(-1, 210).astype(np.int64)
        d = blocks.reshape(-1, 210)[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
        sc = blocks.reshape(-1, 210)[:, 192:208].view(np.int8).astype(np.int64)
        out = np.empty((len(b), 256), np.float16)
        for h in range(2):
            ql, qh = b[:, 64 * h:64 * h + 64], b[:, 128 + 32 * h:128 + 32 * h + 32]
            for l in range(32):
                q = [(ql[:, l] & 15) | ((qh[:, l] & 3) << 4), (ql[:, 32 + l] & 15) | (((qh[:, l] >> 2) & 3) << 4),
                     (ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4), (ql[:, 32 + l] >> 4) | (((qh[:, l] >> 6) & 3) << 4)]
                for g in range(4):
                    a = f16((q[g] - 32) * sc[:, 8 * h + l // 16 + 2 * g]).astype(np.float64)
                    out[:, 128 * h + 32 * g + l] = f16(a * d)
        return out.reshape(rows, cols)
    b = blocks.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    q = b[:, 2:34].view(np.int8).astype(np.float64)
    return f16(q * d[:, None]).reshape(rows, cols)


def f16_ulp(v):
    """Spacing of fp16 numbers at |v| (2^-24 below the normal range)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.exp2(e - 10)


def q4k_q5k_exact_and_min(fmt, blocks, rows, cols):
    """Per weight of a Q4_K / Q5_K matrix: the exact value d sc q - dmin m
    (float64) and fp16(dmin m), the min term as the GEMMs round it."""
    bb = 144 if fmt == "Q4_K" else 176
    b = blocks.reshape(-1, bb)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    from test_oracle import layout_table_np
    sc, mn = layout_table_np(b[:, 4:16])
    ex = np.empty((len(b), 256))
    mb = np.empty((len(b), 256))
    for j in range(4):
        for h in range(2):
            s_ = 2 * j + h
            if fmt == "Q4_K":
                q = (b[:, 16 + 32 * j:16 + 32 * j + 32].astype(np.int64) >> (4 * h)) & 0xF
            else:
                qh = b[:, 16:48].astype(np.int64)
                q = ((b[:, 48 + 32 * j:48 + 32 * j + 32].astype(np.int64) >> (4 * h)) & 0xF) + \
                    16 * ((qh >> (2 * j + h)) & 1)
            cols_ = slice(64 * j + 32 * h, 64 * j + 32 * h + 32)
            ex[:, cols_] = d[:, None] * sc[:, s_][:, None] * q - (dmin * mn[:, s_])[:, None]
            mb[:, cols_] = f16(dmin * mn[:, s_]).astype(np.float64)[:, None]
    return ex.reshape(rows, cols), mb.reshape(rows, cols)


@pytest.mark.parametrize("fmt,tiled", [("Q4_K", 0), ("Q4_K", 1), ("Q5_K", 0), ("Q5_K", 1), ("Q6_K", 0), ("Q6_K", 1),
                                       ("Q8_0", 0), ("Q8_0", 1)])
def test_mfma_fp16_weights_bit_exact(fmt, tiled):
    """The fp16 weights the matrix cores multiply (read back through the real
    grouped down GEMM with one-hot activations, orome_debug_mfma_weights)
    equal, bit for bit, the numpy emulation of the documented factored fp16
    dequant, for row-major and tile-major copies; and each is within the
    stated rounding of the oracle's exact fp32 value."""
    banner("MFMA fp16 weights %s tiled=%d" % (fmt, tiled))
    ggml = {"Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_0": 8}[fmt]
    kw = dict(down=ggml) if fmt != "Q8_0" else dict(shared=8)
    p = Pair(max_tokens=32, E=8, seed=71, **kw)
    name = "blk.0.ffn_down_exps.weight" if fmt != "Q8_0" else "blk.0.ffn_down_shexp.weight"
    dims, typ, off, nb = p.om.tensors[name]
    H, M = 2048, 512
    one = nb // 8 if fmt != "Q8_0" else nb          # expert 0's matrix
    blocks = p.img[off:off + one]
    out = DeviceBuffer(p.ctx, M * H * 4)
    fmt_id = O.GGML_TO_FMT[typ]
    _lib.check(lib.orome_debug_mfma_weights(p.ctx.handle, fmt_id, tiled, p.gm.tensor_device_ptr(name), H, M,
                                            out.ptr), "orome_debug_mfma_weights")
    got = out.download(np.float32, (M, H)).T              # [H rows, M cols]
    model = mfma_weights_model((fmt, blocks, H, M))
    assert np.array_equal(got.astype(np.float16).view(np.uint16), model.view(np.uint16))
    assert np.array_equal(got, model.astype(np.float32))  # the GEMM's fp32 outputs are those fp16 values
    exact = O.decode_rows(fmt_id, blocks, H, M)
    if fmt in ("Q6_K", "Q8_0"):  # one or two roundings of the exact value
        ulp = np.abs(exact) * 2.0 ** -10 + 2.0 ** -24
        assert np.all(np.abs(got.astype(np.float64) - exact) <= 2 * ulp)
    else:
        # two roundings, bounded per weight: w = fp16(q sc d - fp16(dmin m)),
        # so |w - exact| <= ulp(w)/2 + ulp(fp16(dmin m))/2, with exact the
        # real value d sc q - dmin m (float64, from the block fields)
        ex64, mb = q4k_q5k_exact_and_min(fmt, blocks, H, M)
        bound = 0.5 * f16_ulp(got) + 0.5 * f16_ulp(mb)
        err = np.abs(got.astype(np.float64) - ex64)
        assert np.all(err <= bound), float((err / bound).max())
        # and the oracle's fp32 value is the float32 rounding of that exact value
        assert np.array_equal(exact, ex64.astype(np.float32))
    p.gm.close()


@pytest.mark.parametrize("T", [200, 1100])
def test_more_than_256_experts(T):
    """E = 384 (above the one-block dispatch's 256): the three-launch dispatch
    with its block-wide scan over 6 waves of experts, the 8-expert-per-lane
    top-k, and the grouped GEMMs at H = 512, M = S = 256.  Routing bit-exact,
    output within tolerance of the oracle."""
    banner("E=384 H=512 M=256, T=%d" % T)
    p = Pair(max_tokens=T, E=384, H=512, M=256, S=256, seed=91)
    run_and_check(p, T, seed=3300 + T, path=_lib.OROME_PATH_MFMA)
    p.gm.close()


def test_two_pass_router_h4096():
    """H = 4096 (the largest hidden size the two-pass router takes): the
    approximation pass walks its k-slice in two chunks of loads and the exact
    top-k holds 16 f4 of x per lane.  Routing bit-exact, output within
    tolerance of the oracle."""
    banner("H=4096, T=48")
    p = Pair(max_tokens=48, H=4096, seed=77)
    run_and_check(p, 48, seed=4048, path=_lib.OROME_PATH_MFMA)
    p.gm.close()


@pytest.mark.parametrize("shape", [dict(E=256, H=2048, M=512, S=512), dict(E=384, H=1024, M=256, S=256),
                                   dict(E=128, H=3072, M=512, S=512)])
def test_two_pass_router_sweep(shape):
    """The two-pass router over batch sizes covering its three tile sizes (16,
    32 and 64 tokens a block) and both sides of the self-dispatching gate/up's
    limit (1024 tokens), three router shapes (E = 384 takes the dispatch
    kernel), activations at two scales: expert indices bit-exact against the
    oracle's router and top-k, the winners' and shared-gate logits bit-exact,
    weights to the softmax's rounding; the dispatch (offsets, pair order) bit-exact
    against the oracle's."""
    banner("two-pass sweep E=%(E)d H=%(H)d" % shape)
    p = Pair(max_tokens=2048, seed=5, **shape)
    L = O.lib(omp=True)
    lr = p.om.layer(0)
    E, H, K = p.om.E, p.om.H, p.om.K
    for T in (17, 129, 512, 1024, 1025, 2048):
        for s in range(2):
            x = orome_amd.synth_normal(700 + s, T, T * H).reshape(T, H)
            if s:
                x *= np.float32(37.0)
            _, dbg = p.run(0, x, np.zeros_like(x), path=_lib.OROME_PATH_MFMA)
            lg = np.empty((T, E + 1), np.float32)
            L.orc_router_logits(lr.router, lr.shared_gate_vec, O.p(x), T, E, H, O.p(lg))
            idx = np.empty((T, K), np.int32)
            w = np.empty((T, K), np.float32)
            sg = np.empty(T, np.float32)
            L.orc_topk_route(O.p(lg), lr.bias, T, E, K, O.p(idx), O.p(w), O.p(sg))
            assert np.array_equal(dbg["idx"], idx), "indices T=%d s=%d" % (T, s)
            assert np.allclose(dbg["w"], w, rtol=2e-6, atol=1e-7)
            win = np.take_along_axis(lg[:, :E], idx, 1)
            gwin = np.take_along_axis(dbg["logits"][:, :E], idx, 1)
            assert np.array_equal(win.view(np.uint32), gwin.view(np.uint32)), "winner logits"
            assert np.array_equal(lg[:, E].view(np.uint32), dbg["logits"][:, E].view(np.uint32)), "shared-gate logit"
            off, pairs = O.dispatch(idx, E)
            assert np.array_equal(dbg["offsets"], off), "dispatch offsets T=%d" % T
            assert np.array_equal(dbg["pairs"], pairs), "dispatch order T=%d" % T
    p.gm.close()
