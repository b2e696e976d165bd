"""Pins the C oracle (oracle/moe_oracle.c) against the reference's known-answer
tests, exhaustive enumerations and independent float64 restatements.
CPU only."""
import ctypes as C
import struct

import numpy as np
import pytest

import oracle as O

L = O.lib(omp=False)


def f16_trunc(f):
    """The truncating float->fp16 conversion of the reference KATs
    (tests/test_q4k.m:38-41, tests/test_q8_0.m:44-52)."""
    b = struct.unpack("<I", struct.pack("<f", f))[0]
    sign = (b >> 31) & 1
    e = ((b >> 23) & 0xFF) - 127 + 15
    m = (b >> 13) & 0x3FF
    if e <= 0:
        return 0
    if e >= 31:
        return (sign << 15) | (31 << 10)
    return (sign << 15) | (e << 10) | m


# ------------------------------------------------------------------ A1
def test_fp16_to_f32_exhaustive():
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([L.orc_fp16_to_f32(int(h)) for h in codes], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne():
    h = np.arange(65536, dtype=np.uint16)
    vals = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(vals)
    # exact fp16 values round-trip, midpoints between neighbours tie to even,
    # and random values match numpy's RNE conversion
    pos = vals[fin & (vals >= 0)]
    pos = np.sort(pos)
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    rnd = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s
                          for s in (1e-6, 1e-3, 1, 300, 7e4)])
    cases = np.concatenate([vals[fin], mids, -mids, rnd, np.float32([65519.0, 65520.0, 1e9, -1e9])])
    with np.errstate(over="ignore"):
        ref = cases.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f32_to_f16(float(v)) for v in cases], np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_truncation():
    for v in (1.0, 1.0078125 + 2 ** -12, -3.14159, 1e-30):
        b = struct.unpack("<I", struct.pack("<f", v))[0] & 0xFFFF0000
        assert L.orc_bf16_trunc(v) == struct.unpack("<f", struct.pack("<I", b))[0]


# ------------------------------------------------------------------ A2
def layout_table(s):
    """Scales/mins of the 8 sub-blocks from the reference layout
    (inference/src/format.m:41-64 read as a per-sub-block table):
    sc[j] = s[j] & 63, mn[j] = s[j+4] & 63 for j < 4;
    sc[4+i] = nibble (i&1) of s[8 + i//2] | (s[i] >> 6) << 4;
    mn[4+i] = nibble (i&1) of s[10 + i//2] | (s[4+i] >> 6) << 4."""
    sc, mn = [0] * 8, [0] * 8
    for j in range(4):
        sc[j], mn[j] = s[j] & 63, s[j + 4] & 63
    for i in range(4):
        nib = lambda b: (b >> (4 * (i & 1))) & 0xF
        sc[4 + i] = nib(s[8 + i // 2]) | ((s[i] >> 6) << 4)
        mn[4 + i] = nib(s[10 + i // 2]) | ((s[4 + i] >> 6) << 4)
    return sc, mn


def oracle_pairs(s):
    arr = (C.c_uint8 * 12)(*s)
    sc, mn = [0] * 8, [0] * 8
    for g in range(4):
        a, b, c, d = C.c_float(), C.c_float(), C.c_float(), C.c_float()
        L.orc_unpack_q4k_pair(arr, g, C.byref(a), C.byref(b), C.byref(c), C.byref(d))
        sc[2 * g], sc[2 * g + 1], mn[2 * g], mn[2 * g + 1] = int(a.value), int(b.value), int(c.value), int(d.value)
    return sc, mn


def layout_table_np(s):
    """layout_table over rows of an [n, 12] uint8 array (numpy, vectorised)."""
    s = s.astype(np.int64)
    sc = np.empty((s.shape[0], 8), np.int64)
    mn = np.empty((s.shape[0], 8), np.int64)
    for j in range(4):
        sc[:, j], mn[:, j] = s[:, j] & 63, s[:, j + 4] & 63
    for i in range(4):
        sh = 4 * (i & 1)
        sc[:, 4 + i] = ((s[:, 8 + i // 2] >> sh) & 0xF) | ((s[:, i] >> 6) << 4)
        mn[:, 4 + i] = ((s[:, 10 + i // 2] >> sh) & 0xF) | ((s[:, 4 + i] >> 6) << 4)
    return sc, mn


def test_q4k_scale_unpack_exhaustive():
    """Every field reads at most two bytes: for each (low byte, high byte) pair
    that feeds a field, all 65536 values of the pair (the other ten bytes
    random), through the oracle against the per-sub-block table."""
    rng = np.random.default_rng(2)
    pairs = [(j, j) for j in range(8)] + [(8 + i // 2, i) for i in range(4)] + \
            [(10 + i // 2, 4 + i) for i in range(4)]
    v = np.arange(65536)
    for lo_b, hi_b in pairs:
        s = np.repeat(rng.integers(0, 256, 12, dtype=np.uint8)[None, :], 65536, axis=0)
        s[:, hi_b] = v >> 8
        s[:, lo_b] = v & 0xFF if lo_b != hi_b else v >> 8
        s = np.ascontiguousarray(s)
        out = np.empty((65536, 16), np.float32)
        L.orc_unpack_q4k_batch(s.ctypes.data, 65536, out.ctypes.data)
        sc, mn = layout_table_np(s)
        assert np.array_equal(out[:, :8], sc) and np.array_equal(out[:, 8:], mn), (lo_b, hi_b)
    s = rng.integers(0, 256, (100000, 12), dtype=np.uint8)
    out = np.empty((100000, 16), np.float32)
    L.orc_unpack_q4k_batch(s.ctypes.data, 100000, out.ctypes.data)
    sc, mn = layout_table_np(s)
    assert np.array_equal(out[:, :8], sc) and np.array_equal(out[:, 8:], mn)
    # the scalar entry point agrees with the batch one
    for r in range(50):
        assert oracle_pairs(list(s[r])) == (list(out[r, :8].astype(int)), list(out[r, 8:].astype(int)))


def test_q4k_layout_differs_from_ggml():
    # ggml's get_scale_min_k4 reads sc[4+j] from byte 8+j; the reference reads
    # byte 8 + j//2 (Finding: layout).  The test_q4k.m fixture (scales bytes
    # 12,13 = 0x11, bytes 14,15 = 0) separates them.
    s = [1, 1, 1, 1, 0, 0, 0, 0, 0x11, 0x11, 0, 0]
    sc, mn = oracle_pairs(s)
    assert sc == [1] * 8 and mn == [0] * 8
    ggml_sc = [(s[8 + j] & 0xF) | ((s[j] >> 6) << 4) for j in range(4)]
    assert ggml_sc[2:] == [0, 0]


def _q4k_block(d, dmin, scales, nib):
    """One 144-byte Q4_K super-block: fp16 d, dmin, the 12 scale bytes as
    given, every quant nibble = nib."""
    b = bytearray(144)
    b[0:2] = np.float16(d).tobytes()
    b[2:4] = np.float16(dmin).tobytes()
    b[4:16] = bytes(scales)
    b[16:144] = bytes([nib | (nib << 4)]) * 128
    return bytes(b)


# (scale byte index, value) -> the 8 sub-block mins (or scales) that
# inference/src/format.m:41-64 decodes from it, written out by hand:
#   bytes 0..3  -> scales of sub-blocks 0..3 (low 6 bits); bits 6..7 are the
#                  high bits of the scales of sub-blocks 4..7
#   bytes 4..7  -> mins of sub-blocks 0..3; bits 6..7 the high bits of the
#                  mins of sub-blocks 4..7
#   byte 8 / 9  -> low nibble: scale of sub-block 4 / 6, high nibble: 5 / 7
#   byte 10 / 11 -> the same for the mins
MIN_ONE_HOT = [
    (4, 0x01, [1, 0, 0, 0, 0, 0, 0, 0]), (7, 0x3F, [0, 0, 0, 63, 0, 0, 0, 0]),
    (10, 0x01, [0, 0, 0, 0, 1, 0, 0, 0]), (10, 0x10, [0, 0, 0, 0, 0, 1, 0, 0]),
    (11, 0x01, [0, 0, 0, 0, 0, 0, 1, 0]), (11, 0x10, [0, 0, 0, 0, 0, 0, 0, 1]),
    (10, 0x0F, [0, 0, 0, 0, 15, 0, 0, 0]), (11, 0xF0, [0, 0, 0, 0, 0, 0, 0, 15]),
    (4, 0x40, [0, 0, 0, 0, 16, 0, 0, 0]), (5, 0x40, [0, 0, 0, 0, 0, 16, 0, 0]),
    (6, 0x40, [0, 0, 0, 0, 0, 0, 16, 0]), (7, 0x80, [0, 0, 0, 0, 0, 0, 0, 32]),
]
SCALE_ONE_HOT = [
    (0, 0x01, [1, 0, 0, 0, 0, 0, 0, 0]), (3, 0x3F, [0, 0, 0, 63, 0, 0, 0, 0]),
    (8, 0x01, [0, 0, 0, 0, 1, 0, 0, 0]), (8, 0x10, [0, 0, 0, 0, 0, 1, 0, 0]),
    (9, 0x01, [0, 0, 0, 0, 0, 0, 1, 0]), (9, 0x10, [0, 0, 0, 0, 0, 0, 0, 1]),
    (0, 0x40, [0, 0, 0, 0, 16, 0, 0, 0]), (1, 0x40, [0, 0, 0, 0, 0, 16, 0, 0]),
    (2, 0x40, [0, 0, 0, 0, 0, 0, 16, 0]), (3, 0x80, [0, 0, 0, 0, 0, 0, 0, 32]),
]


@pytest.mark.parametrize("byte,val,expect", MIN_ONE_HOT)
def test_q4k_min_fields_one_hot(byte, val, expect):
    """A single min field set (scales zero, d = dmin = 1): every weight of
    sub-block j (elements 32j .. 32j+31) decodes to -min_j, with the mins
    read off format.m:57-63 by hand (MIN_ONE_HOT).  Swapping the min bytes
    10/11, or reading them as ggml's packing does, fails these cases."""
    sc = [0] * 12
    sc[byte] = val
    w = O.decode_rows(O.Q4_K, np.frombuffer(_q4k_block(1.0, 1.0, sc, 9), np.uint8), 1, 256)[0]
    assert np.array_equal(w, -np.repeat(np.float32(expect), 32))


@pytest.mark.parametrize("byte,val,expect", SCALE_ONE_HOT)
def test_q4k_scale_fields_one_hot(byte, val, expect):
    """A single scale field set (mins zero, d = 1, every nibble 3): sub-block j
    decodes to 3 sc_j."""
    sc = [0] * 12
    sc[byte] = val
    w = O.decode_rows(O.Q4_K, np.frombuffer(_q4k_block(1.0, 1.0, sc, 3), np.uint8), 1, 256)[0]
    assert np.array_equal(w, 3 * np.repeat(np.float32(expect), 32))


# ------------------------------------------------------------------ A3-A5
def test_q4k_kat_reference():
    """tests/test_q4k.m:18-66: 4 rows x 256, scale 1, min 0, all nibbles 5, x=0.01."""
    rows = []
    for row in range(4):
        sb = bytearray(144)
        d = f16_trunc(0.1 * (row + 1))
        dm = f16_trunc(0.01)
        sb[0:2] = struct.pack("<H", d)
        sb[2:4] = struct.pack("<H", dm)
        for i in range(4):
            sb[4 + i] = 1
            sb[8 + i] = 0
        sb[12] = sb[13] = 0x11
        sb[14] = sb[15] = 0
        sb[16:144] = bytes([0x55]) * 128
        rows.append(bytes(sb))
    data = np.frombuffer(b"".join(rows), np.uint8)
    w = O.decode_rows(O.Q4_K, data, 4, 256)
    for row in range(4):
        d16 = np.uint16(f16_trunc(0.1 * (row + 1))).view(np.float16).astype(np.float32)
        assert np.all(w[row] == np.float32(d16 * 5))
        dot = np.sum(w[row].astype(np.float64) * 0.01)
        expected = 256 * 5 * (0.1 * (row + 1)) * 0.01  # the KAT's own formula
        assert abs(dot - expected) / expected < 0.1  # the KAT's tolerance (test_q4k.m:93)


def test_q8_0_kat_reference():
    """tests/test_q8_0.m:27-70: 64 rows x 256, scale 0.01(row+1), q=(blk*32+j)%127-63."""
    out_dim, in_dim = 64, 256
    x = np.array([0.01 * (j % 10) for j in range(in_dim)], np.float32)
    buf = bytearray()
    expected = np.zeros(out_dim)
    for row in range(out_dim):
        scale = np.float32(0.01 * (row + 1))
        for blk in range(in_dim // 32):
            buf += struct.pack("<H", f16_trunc(float(scale)))
            for j in range(32):
                q = (blk * 32 + j) % 127 - 63
                buf += struct.pack("<b", q)
                expected[row] += float(scale) * q * float(x[blk * 32 + j])
    w = O.decode_rows(O.Q8_0, np.frombuffer(bytes(buf), np.uint8), out_dim, in_dim)
    got = w.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - expected)) < 0.01  # the KAT's tolerance (test_q8_0.m:106)
    q = np.array([[(blk * 32 + j) % 127 - 63 for blk in range(8) for j in range(32)]], np.float32)
    d16 = np.array([np.uint16(f16_trunc(float(np.float32(0.01 * (r + 1))))).view(np.float16)
                    for r in range(out_dim)], np.float32)[:, None]
    assert np.array_equal(w, d16 * q)


def test_f32_matvec_kat_reference():
    """tests/test_f32.m:17-30: W[i][j] = 0.01(i-j), x[j] = 0.1(j%5), 32 x 64,
    zero-padded to 256 columns for the canonical order."""
    W = np.zeros((32, 256), np.float32)
    x = np.zeros(256, np.float32)
    for i in range(32):
        for j in range(64):
            W[i, j] = np.float32(0.01 * (i - j))
    for j in range(64):
        x[j] = np.float32(0.1 * (j % 5))
    exp = W.astype(np.float64) @ x.astype(np.float64)
    got = np.array([L.orc_canon_dot(W[i].ctypes.data, x.ctypes.data, 256) for i in range(32)])
    assert np.max(np.abs(got - exp)) < 1e-5  # (the KAT allows 0.01)


def q4k_block(d, dmin, sc, mn, nibbles):
    """Build one Q4_K super-block from per-sub-block scales/mins (inverse of
    layout_table) and a list of 256 nibbles."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[4 + j] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[4 + j] >> 4) << 6)
    for i in range(4):
        s[8 + i // 2] |= (sc[4 + i] & 0xF) << (4 * (i & 1))
        s[10 + i // 2] |= (mn[4 + i] & 0xF) << (4 * (i & 1))
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            qs[g * 32 + l] = nibbles[g * 64 + l] | (nibbles[g * 64 + 32 + l] << 4)
    return struct.pack("<HH", d, dmin) + bytes(s) + bytes(qs)


def test_q4k_closed_form_random():
    rng = np.random.default_rng(3)
    for _ in range(200):
        d = int(np.float16(abs(rng.standard_normal()) * 2e-3).view(np.uint16))
        dm = int(np.float16(abs(rng.standard_normal()) * 1e-3).view(np.uint16))
        sc = list(rng.integers(0, 64, 8))
        mn = list(rng.integers(0, 64, 8))
        nib = list(rng.integers(0, 16, 256))
        blk = np.frombuffer(q4k_block(d, dm, sc, mn, nib), np.uint8)
        assert layout_table(list(blk[4:16])) == ([int(v) for v in sc], [int(v) for v in mn])
        w = O.decode_rows(O.Q4_K, blk, 1, 256)[0]
        df = np.float32(np.uint16(d).view(np.float16))
        dmf = np.float32(np.uint16(dm).view(np.float16))
        exp = np.array([np.float32(df * np.float32(sc[k // 32])) * np.float32(nib[k]) -
                        np.float32(dmf * np.float32(mn[k // 32])) for k in range(256)], np.float32)
        assert np.array_equal(w, exp)
        # products are exact: the float64 value rounds to the same float32
        e64 = np.array([float(df) * sc[k // 32] * nib[k] - float(dmf) * mn[k // 32] for k in range(256)])
        assert np.array_equal(w, e64.astype(np.float32))


def q6k_ggml_layout(block):
    """Independent Q6_K decoder written from the ggml block_q6_K description
    (ql[128], qh[64], scales[16] int8, d): weight 128*h + 32*g + l (g=0..3,
    l=0..31) takes the low (g even) / high (g odd... see mapping) nibble."""
    ql, qh = block[:128], block[128:192]
    sc = block[192:208].view(np.int8).astype(np.float32)
    d = np.float32(block[208:210].view(np.float16)[0])
    out = np.zeros(256, np.float32)
    for h in range(2):
        for l in range(32):
            hb = int(qh[32 * h + l])
            lo_a, lo_b = int(ql[64 * h + l]), int(ql[64 * h + 32 + l])
            q = [(lo_a & 15) | ((hb & 3) << 4), (lo_b & 15) | (((hb >> 2) & 3) << 4),
                 (lo_a >> 4) | (((hb >> 4) & 3) << 4), (lo_b >> 4) | (((hb >> 6) & 3) << 4)]
            for g in range(4):
                out[128 * h + 32 * g + l] = np.float32(d * sc[8 * h + l // 16 + 2 * g]) * np.float32(q[g] - 32)
    return out


def test_q6k_matches_ggml_layout_and_one_hot():
    rng = np.random.default_rng(4)
    for _ in range(100):
        blk = rng.integers(0, 256, 210).astype(np.uint8)
        blk[208:210] = np.frombuffer(np.float16(abs(rng.standard_normal()) * 2e-3).tobytes(), np.uint8)
        assert np.array_equal(O.decode_rows(O.Q6_K, blk, 1, 256)[0], q6k_ggml_layout(blk))
    # one-hot: a single high-bit field set moves exactly one weight by 16*d*sc
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    base = O.decode_rows(O.Q6_K, blk, 1, 256)[0]
    assert np.all(base == -32)
    blk[128 + 5] = 0b00000100  # qh byte 5, bits 2-3 -> q2 of l=5 in half 0 -> weight 32+5
    w = O.decode_rows(O.Q6_K, blk, 1, 256)[0]
    assert np.nonzero(w != base)[0].tolist() == [37] and w[37] == -16


def q5k_independent(blocks):
    """Q5_K blocks [n, 176] -> [n, 256]: the published ggml q5_K formula (per
    64-value group j, the low nibble of ql[32 j + l] plus 16 if bit 2 j of
    qh[l] is set, the high nibble plus 16 if bit 2 j + 1 is set; y = d sc q
    - dmin m), with the scales and mins of the reference packing
    (layout_table_np, format.m:41-64)."""
    b = blocks.astype(np.uint32)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = layout_table_np(blocks[:, 4:16])
    qh, ql = b[:, 16:48], b[:, 48:176]
    y = np.empty((len(b), 256), np.float32)
    for j in range(4):
        for h in range(2):
            s = 2 * j + h
            q = ((ql[:, 32 * j:32 * j + 32] >> (4 * h)) & 0xF) + 16 * ((qh >> (2 * j + h)) & 1)
            y[:, 64 * j + 32 * h:64 * j + 32 * h + 32] = (d * sc[:, s].astype(np.float32))[:, None] * \
                q.astype(np.float32) - (dmin * mn[:, s].astype(np.float32))[:, None]
    return y


def test_q5k_matches_independent_decoder_and_one_hot():
    """Q5_K (inference/src/format.m:110-141): random blocks against the
    independent decoder bit for bit; a single qh bit moves exactly one weight
    by 16 d sc."""
    rng = np.random.default_rng(14)
    blk = rng.integers(0, 256, (2000, 176)).astype(np.uint8)
    blk[:, 0:2] = np.frombuffer((np.abs(rng.standard_normal(2000)) * 1e-2).astype(np.float16).tobytes(),
                                np.uint8).reshape(-1, 2)
    blk[:, 2:4] = np.frombuffer((np.abs(rng.standard_normal(2000)) * 1e-2).astype(np.float16).tobytes(),
                                np.uint8).reshape(-1, 2)
    got = O.decode_rows(O.Q5_K, blk, 2000, 256)
    assert np.array_equal(got.view(np.uint32), q5k_independent(blk).view(np.uint32))
    one = np.zeros(176, np.uint8)
    one[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    one[4:16] = 1  # every scale 1 (and the packed high parts 0), every min 1
    base = O.decode_rows(O.Q5_K, one, 1, 256)[0]
    one[16 + 7] = 1 << 4  # qh[7] bit 4: group 2, low half -> weight 2*64 + 7 (sub-block 4, scale 1)
    w = O.decode_rows(O.Q5_K, one, 1, 256)[0]
    assert sc_of(one, 4) == 1
    assert np.nonzero(w != base)[0].tolist() == [135] and w[135] - base[135] == 16.0


def sc_of(blk, s):
    return layout_table(list(blk[4:16]))[0][s]


# ------------------------------------------------------------------ A6
def test_canonical_dot_exact_on_integers_and_bounded():
    rng = np.random.default_rng(5)
    for n in (256, 2048):
        a = rng.integers(-50, 50, n).astype(np.float32)
        b = rng.integers(-50, 50, n).astype(np.float32)
        assert L.orc_canon_dot(a.ctypes.data, b.ctypes.data, n) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = (n.bit_length() + 40) * 2 ** -24 * float(np.sum(np.abs(a.astype(np.float64) * b)))
        assert abs(L.orc_canon_dot(a.ctypes.data, b.ctypes.data, n) - exact) <= bound


def test_router_logits_layout():
    rng = np.random.default_rng(6)
    T, E, H = 3, 8, 256
    W = rng.integers(-8, 8, (E, H)).astype(np.float32)
    wsg = rng.integers(-8, 8, H).astype(np.float32)
    x = rng.integers(-8, 8, (T, H)).astype(np.float32)
    out = np.empty((T, E + 1), np.float32)
    L.orc_router_logits(W.ctypes.data, wsg.ctypes.data, x.ctypes.data, T, E, H, out.ctypes.data)
    assert np.array_equal(out[:, :E], (x.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32))
    assert np.array_equal(out[:, E], (x.astype(np.int64) @ wsg.astype(np.int64)).astype(np.float32))


# ------------------------------------------------------------------ A7
def brute_topk(v, K):
    order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))
    return order[:K]


@pytest.mark.parametrize("K", [1, 4, 8, 16])
def test_topk_brute_force(K):
    rng = np.random.default_rng(7 + K)
    T, E = 64, 256
    for quant in (None, 0.25):  # quantised logits create many ties
        lg = rng.standard_normal((T, E + 1)).astype(np.float32)
        if quant:
            lg = (np.round(lg / quant) * quant).astype(np.float32)
        bias = rng.standard_normal(E).astype(np.float32) if quant else None
        idx, w, sg = O.topk(lg, bias, K)
        for t in range(T):
            v = lg[t, :E] + (bias if bias is not None else 0)
            v = v.astype(np.float32)
            exp_idx = brute_topk(v, K)
            assert idx[t].tolist() == exp_idx.tolist()
            sel = v[exp_idx].astype(np.float64)
            e = np.exp(sel - sel[0])
            assert np.allclose(w[t], e / e.sum(), rtol=1e-6, atol=1e-7)
            assert abs(w[t].sum() - 1) < 1e-5
            assert sg[t] == lg[t, E]


def test_topk_special_cases():
    E, K = 256, 8
    lg = np.zeros((3, E + 1), np.float32)
    lg[1, :E] = -0.0
    lg[1, 3] = 0.0
    lg[2, :] = -np.inf
    lg[2, 200] = 5.0
    lg[2, 100] = 4.0
    idx, w, _ = O.topk(lg, None, K)
    assert idx[0].tolist() == list(range(8))           # all equal -> lowest indices
    assert idx[1].tolist() == list(range(8))           # -0 and +0 tie by index
    assert idx[2][:2].tolist() == [200, 100]
    assert np.allclose(w[0], 1 / 8)


# ------------------------------------------------------------------ A8
def test_dispatch_stable_counting_sort():
    rng = np.random.default_rng(8)
    for T, K, E in ((1, 8, 256), (8, 8, 256), (512, 8, 256), (33, 4, 16)):
        idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        off, pairs = O.dispatch(idx, E)
        flat = idx.reshape(-1)
        assert pairs.tolist() == np.argsort(flat, kind="stable").tolist()
        assert off.tolist() == [0] + np.cumsum(np.bincount(flat, minlength=E)).tolist()
        assert sorted(pairs.tolist()) == list(range(T * K))


# ------------------------------------------------------------------ A9-A14
def small_model(seed=0, **kw):
    import orome_amd
    args = dict(layers=2, H=512, E=16, K=4, M=512, S=512, seed=seed)
    args.update(kw)
    img = orome_amd.synth_gguf(orome_amd.make_spec(**args))
    return O.OracleModel(img)


def f64_forward(om, l, x, h_in):
    """Float64 restatement from decoded weights (half-rounded activations)."""
    T = x.shape[0]
    E, H, M = om.E, om.H, om.M
    Lr = om.layer(l)
    W = om.array("blk.%d.ffn_gate_inp.weight" % l, np.float32).reshape(E, H).astype(np.float64)
    logits = x.astype(np.float64) @ W.T
    bname = "blk.%d.exp_probs_b.bias" % l
    if bname in om.tensors:
        logits = logits + om.array(bname, np.float32)
    sgv = om.array("blk.%d.ffn_gate_inp_shexp.weight" % l, np.float32).astype(np.float64)
    sg = x.astype(np.float64) @ sgv
    hx = x.astype(np.float16).astype(np.float64)

    def dec(name, rows, n, e=None):
        dims, typ, off, nb = om.tensors[name]
        per = nb // (om.E if e is not None else 1)
        start = off + (e or 0) * per
        return O.decode_rows(O.GGML_TO_FMT[typ], om.image[start:start + per], rows, n).astype(np.float64)

    out = h_in.astype(np.float64).copy()
    for t in range(T):
        order = np.lexsort((np.arange(E), -logits[t]))[:om.K]
        v = logits[t, order]
        w = np.exp(v - v[0]); w /= w.sum()
        for k, e in enumerate(order):
            g = dec("blk.%d.ffn_gate_exps.weight" % l, M, H, e) @ hx[t]
            u = dec("blk.%d.ffn_up_exps.weight" % l, M, H, e) @ hx[t]
            act = (g / (1 + np.exp(-g)) * u).astype(np.float16).astype(np.float64)
            out[t] += w[k] * (dec("blk.%d.ffn_down_exps.weight" % l, H, M, e) @ act)
        S = Lr.S
        g = dec("blk.%d.ffn_gate_shexp.weight" % l, S, H) @ hx[t]
        u = dec("blk.%d.ffn_up_shexp.weight" % l, S, H) @ hx[t]
        act = (g / (1 + np.exp(-g)) * u).astype(np.float16).astype(np.float64)
        out[t] += 1 / (1 + np.exp(-sg[t])) * (dec("blk.%d.ffn_down_shexp.weight" % l, H, S) @ act)
    return out


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("kw", [{}, dict(down=14, zipf=True), dict(shared=8)])
def test_moe_forward_matches_float64(kw):
    om = small_model(seed=11, **kw)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, om.H)).astype(np.float32)
    h = rng.standard_normal((3, om.H)).astype(np.float32)
    out = om.forward(0, x, h)
    ref = f64_forward(om, 0, x, h)
    # fp32 sums vs float64 sums; the fp16 staging of act can land one fp16
    # ulp apart when the two sums straddle a rounding boundary
    assert rel_l2(out - h, ref - h) < 5e-5


def test_moe_forward_closed_forms():
    om = small_model(seed=12)
    x = np.zeros((2, om.H), np.float32)
    h = np.arange(2 * om.H, dtype=np.float32).reshape(2, om.H)
    # x = 0: router logits 0, every gate 0, SiLU(0) = 0 -> output == residual
    out, dbg = om.forward(0, x, h, debug=True)
    assert np.array_equal(out, h)
    assert dbg["idx"][0].tolist() == list(range(om.K))       # all-equal logits
    assert np.allclose(dbg["w"], 1.0 / om.K)


def test_rmsnorm_definition():
    om = small_model(seed=13)
    rng = np.random.default_rng(10)
    h = (rng.standard_normal((4, om.H)) * 3).astype(np.float32)
    x = om.rmsnorm(0, h)
    h64 = h.astype(np.float64)
    ref = h64 / np.sqrt((h64 ** 2).mean(axis=1, keepdims=True) + om.eps)
    assert np.max(np.abs(x - ref)) < 1e-5 * np.max(np.abs(ref))
