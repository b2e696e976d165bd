"""The ggml Q4_K scale packing as a file-format option (no GPU needed).

The reference decodes sub-blocks 4..7 of a Q4_K block from scale bytes 8..11
in its own packing (inference/src/format.m:41-64); ggml/llama.cpp files pack
byte 8 + j as scale 4+j | min 4+j << 4 (get_scale_min_k4 of the published
block_q4_K format; the reference's llama-style kernel reads it so,
inference/src/shaders.metal:1575-1578).  A file declares ggml packing with
the metadata key orome.q4_k.scale_layout = "ggml", and the library permutes
bytes 8..11 of each block into the reference packing at upload.  These tests
pin that permutation: a ggml decoder written from the published format, fed
the ggml bytes, gives bit for bit the oracle's decode of the permuted bytes."""
import ctypes as C

import numpy as np

import orome_amd
import oracle as O
from orome_amd import _lib
from orome_amd._lib import lib


def ggml_decode_q4k(blocks):
    """Published block_q4_K dequantisation (ggml get_scale_min_k4 packing):
    per 64-value group j: y = d*sc*(q & 15) - dmin*m for the low nibbles of
    qs[32 j .. 32 j + 31] with (sc, m) of sub-block 2 j, and the high nibbles
    with sub-block 2 j + 1.  blocks: [n, 144] uint8 -> [n, 256] float32."""
    b = blocks.astype(np.uint32)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    q = b[:, 4:16]
    sc = np.empty((len(b), 8), np.uint32)
    mn = np.empty((len(b), 8), np.uint32)
    for j in range(8):
        if j < 4:
            sc[:, j], mn[:, j] = q[:, j] & 63, q[:, j + 4] & 63
        else:
            sc[:, j] = (q[:, j + 4] & 0xF) | ((q[:, j - 4] >> 6) << 4)
            mn[:, j] = (q[:, j + 4] >> 4) | ((q[:, j] >> 6) << 4)
    qs = b[:, 16:144]
    y = np.empty((len(b), 256), np.float32)
    for j in range(4):
        for h in range(2):
            s = 2 * j + h
            d1 = d * sc[:, s].astype(np.float32)
            m1 = dmin * mn[:, s].astype(np.float32)
            nib = ((qs[:, 32 * j:32 * j + 32] >> (4 * h)) & 0xF).astype(np.float32)
            y[:, 64 * j + 32 * h:64 * j + 32 * h + 32] = d1[:, None] * nib - m1[:, None]
    return y


def ggml_to_reference(blocks):
    """Bytes 8..11 of the scales (block bytes 12..15), ggml -> reference
    packing, restated in numpy from the two layouts' definitions."""
    out = blocks.copy()
    g = blocks[:, 12:16].astype(np.uint32)
    out[:, 12] = (g[:, 0] & 0xF) | ((g[:, 1] & 0xF) << 4)   # scales 4, 5
    out[:, 13] = (g[:, 2] & 0xF) | ((g[:, 3] & 0xF) << 4)   # scales 6, 7
    out[:, 14] = (g[:, 0] >> 4) | (g[:, 1] & 0xF0)          # mins 4, 5
    out[:, 15] = (g[:, 2] >> 4) | (g[:, 3] & 0xF0)          # mins 6, 7
    return out


def oracle_decode(blocks):
    out = np.empty((len(blocks), 256), np.float32)
    blocks = np.ascontiguousarray(blocks)
    assert O.lib().orc_decode_rows(O.Q4_K, blocks.ctypes.data, len(blocks), 256, out.ctypes.data) == 0
    return out


def random_blocks(rng, n):
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.abs(rng.standard_normal(n)).astype(np.float16).tobytes(), np.uint8).reshape(n, 2)
    b[:, 2:4] = np.frombuffer((np.abs(rng.standard_normal(n)) * 0.5).astype(np.float16).tobytes(),
                              np.uint8).reshape(n, 2)
    return b


def test_ggml_packing_permutes_into_reference_decode():
    """Every value of each nibble pair the permutation moves: all 65536 values
    of (byte 8, byte 9) and of (byte 10, byte 11), the other bytes random."""
    rng = np.random.default_rng(5)
    v = np.arange(65536)
    for lo in (12, 14):
        b = random_blocks(rng, 65536)
        b[:, lo], b[:, lo + 1] = v & 0xFF, v >> 8
        ref = ggml_decode_q4k(b)
        got = oracle_decode(ggml_to_reference(b))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), lo


def test_packings_differ_where_the_survey_says():
    """The two packings agree on sub-blocks 0..3 and differ on 4..7 (so a
    ggml file read as the reference's decodes wrongly there)."""
    rng = np.random.default_rng(6)
    b = random_blocks(rng, 4096)
    g, r = ggml_decode_q4k(b), oracle_decode(b)
    assert np.array_equal(g[:, :32], r[:, :32]) and np.array_equal(g[:, 64:96], r[:, 64:96])
    assert not np.array_equal(g[:, 128:], r[:, 128:])


def test_synth_ggml_image_declares_and_holds_the_same_values():
    """A synthetic file written in the ggml packing declares it in its
    metadata, the parser reports it, and its Q4_K tensors decode (ggml
    decoder) to the reference-packed file's values (oracle) bit for bit."""
    kw = dict(layers=1, H=512, E=8, K=2, M=256, S=256, seed=9)
    ref_img = orome_amd.synth_gguf(orome_amd.make_spec(**kw))
    g_img = orome_amd.synth_gguf(orome_amd.make_spec(q4k_ggml=True, **kw))
    for img, want in ((ref_img, _lib.OROME_Q4K_LAYOUT_REFERENCE), (g_img, _lib.OROME_Q4K_LAYOUT_GGML)):
        gf = lib.orome_hip_gguf_open_memory(img.ctypes.data, img.nbytes)
        assert gf and gf.contents.q4k_layout == want
        lib.orome_hip_gguf_close(gf)
    om_r, om_g = O.OracleModel(ref_img), O.OracleModel(g_img)
    assert om_g.meta["orome.q4_k.scale_layout"] == "ggml"
    n = 0
    for name, (dims, typ, off, nb) in om_r.tensors.items():
        if typ != 12:
            continue
        a = om_r.array(name).reshape(-1, 144)
        b = om_g.array(name).reshape(-1, 144)
        assert np.array_equal(np.delete(a, np.s_[12:16], axis=1), np.delete(b, np.s_[12:16], axis=1))
        assert np.array_equal(ggml_decode_q4k(b).view(np.uint32), oracle_decode(a).view(np.uint32)), name
        assert np.array_equal(ggml_to_reference(b), a)
        n += 1
    assert n >= 4
