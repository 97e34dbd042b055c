"""CPU: pins the oracle's row gather (oracle/emel_oracle_getrows.c) against
the fixtures of snapshots/parity/kernel-get-rows/manifest.txt, the known
answers of crates/emel-kernels/tests/any/get_rows_ops.rs, and closed forms
(numpy fancy indexing, exact f16/bf16 widening, independent block decoders)."""
import struct

import numpy as np
import pytest

import oracle as orc
from helpers import assert_bits_equal, rng

F32, F16, Q4_0, Q8_0, Q4_K, I32, BF16 = 0, 1, 2, 8, 12, 26, 30


def dense(ne, elem=4):
    nb = [elem]
    for d in range(1, 4):
        nb.append(nb[-1] * ne[d - 1])
    return nb


def gr(kind, src, sne, snb, sdtype, idx, ine, inb=None, dne=None, dnb=None, fill=9.0, src_bytes=None, ilen=None):
    """Runs orc_get_rows; returns (status, output array)."""
    dne = dne if dne is not None else [sne[0], ine[0], ine[1], ine[2]]
    count = int(np.prod(dne))
    out = np.full(max(count, 1), fill, np.float32)
    dv = orc.view(out, dne, dnb if dnb is not None else dense(dne), F32, 4 * count)
    sv = orc.view(src, sne, snb, sdtype, src.nbytes if src_bytes is None else src_bytes)
    iv = orc.index_view(np.ascontiguousarray(idx, np.int32), ine, inb, ilen)
    return orc.get_rows(kind, sv, iv, dv), out[:count]


def bf16(values):
    return (np.array(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ---- manifest fixtures (snapshots/parity/kernel-get-rows/manifest.txt) -----------------

ROWS4 = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 40, 50, 60], np.float32)
WANT4 = [4, 5, 6, 1, 2, 3, 10, 20, 30, 40, 50, 60]


def test_manifest_f32_fixtures():
    st, out = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, [1, 0, 0, 1], [2, 2, 1])
    assert st == orc.OK and out.tolist() == WANT4
    st, out = gr(orc.GR_F32, np.array([1, 2, 99, 3, 4], np.float32), [2, 2, 1, 1], [4, 12, 24, 24], F32, [1, 0],
                 [2, 1, 1])
    assert st == orc.OK and out.tolist() == [3, 4, 1, 2]
    # non-unit element stride: the pinned memcpy copies contiguous floats from the row start
    st, out = gr(orc.GR_F32, np.array([1, 99, 2, 99, 3, 99, 4], np.float32), [2, 2, 1, 1], [8, 16, 32, 32], F32,
                 [1, 0], [2, 1, 1])
    assert st == orc.OK and out.tolist() == [3, 99, 1, 99]
    st, out = gr(orc.GR_F32, np.array([1, 2], np.float32), [2, 1, 1, 1], [4, 0, 0, 0], F32, [0], [1, 1, 1])
    assert st == orc.OK and out.tolist() == [1, 2]
    st, out = gr(orc.GR_F32, np.array([1, 2, 3, 4], np.float32), [2, 2, 1, 1], [0, 7, 7, 7], F32, [1, 0], [2, 1, 1])
    assert st == orc.OK and out.tolist() == [3, 4, 1, 2]


def test_manifest_unaligned_outer_f32_bytes():
    src = np.zeros(17, np.uint8)
    src[0:4] = np.frombuffer(struct.pack("=f", 1.0), np.uint8)
    src[4:8] = np.frombuffer(struct.pack("=f", 2.0), np.uint8)
    src[9:13] = np.frombuffer(struct.pack("=f", 3.0), np.uint8)
    src[13:17] = np.frombuffer(struct.pack("=f", 4.0), np.uint8)
    st, out = gr(orc.GR_F32_BYTES, src, [2, 2, 1, 1], [4, 9, 18, 18], F32, [1, 0], [2, 1, 1])
    assert st == orc.OK and out.tolist() == [3, 4, 1, 2]
    st, out = gr(orc.GR_F32_BYTES, src[:16].copy(), [2, 2, 1, 1], [4, 9, 18, 18], F32, [1, 0], [2, 1, 1])
    assert st == orc.INVALID_VIEW and out.tolist() == [9] * 4  # unaligned_outer_span_short


def test_manifest_bf16_fixtures():
    st, out = gr(orc.GR_BF16, bf16([1, 2, 3, 4]), [2, 2, 1, 1], [0, 5, 5, 5], BF16, [1, 0], [2, 1, 1])
    assert st == orc.OK and out.tolist() == [3, 4, 1, 2]
    st, out = gr(orc.GR_BF16, bf16([1, 2]), [2, 1, 1, 1], [2, 0, 0, 0], BF16, [0], [1, 1, 1])
    assert st == orc.OK and out.tolist() == [1, 2]
    st, out = gr(orc.GR_BF16, bf16(ROWS4), [3, 2, 2, 1], dense([3, 2, 2, 1], 2), BF16, [1, 0, 0, 1], [2, 2, 1])
    assert st == orc.OK and out.tolist() == WANT4
    st, out = gr(orc.GR_BF16, bf16([1, 2, 3, 4]), [2, 2, 1, 1], [2, 0, 4, 4], BF16, [1, 0], [2, 1, 1])
    assert st == orc.INVALID_VIEW  # bf16_non_singleton_zero_stride


def test_manifest_index_fixtures():
    st, out = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, [1, 0, 99, 99, 0, 1], [2, 2, 1],
                 [4, 16, 32])
    assert st == orc.OK and out.tolist() == WANT4
    st, out = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, [1, 0, 0, 1], [2, 2, 1],
                 [0, 2**64 - 1, 3])
    assert st == orc.OK and out.tolist() == WANT4
    # accepted metadata forms with an empty index tensor: no-op routes
    for ine, dne in (([0, 1, 1], [3, 0, 1, 1]), ([0, 0, 0], [3, 0, 0, 0])):
        src_ne = [3, 2, ine[1], ine[2]]
        st, _ = gr(orc.GR_F32, np.zeros(6, np.float32), src_ne, [4, 12, 24, 24], F32, np.zeros(0, np.int32), ine,
                   dne=dne)
        assert st == orc.OK, (ine, dne)
    st, _ = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, np.zeros(0, np.int32), [0, 2, 1],
               [0, 0, 0], dne=[3, 0, 2, 1], dnb=[4, 12, 0, 0])
    assert st == orc.OK
    # rejected metadata: [0, 2, 1] row-major (a zero stride on an extent of 2), u64::MAX extent,
    # odd / zero / overflowing strides, short storage
    st, _ = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, np.zeros(0, np.int32), [0, 2, 1],
               dne=[3, 0, 2, 1], dnb=[4, 12, 0, 0])
    assert st == orc.INVALID_VIEW
    for nb, data in (([2, 8, 8], [0, 1, 0, 1]), ([4, 0, 8], [0, 1, 0, 1]),
                     ([2**64 - 4, 2**64 - 4, 4], [0, 1, 0, 1]), ([4, 16, 32], [0, 1])):
        st, out = gr(orc.GR_F32, np.zeros(12, np.float32), [3, 2, 2, 1], dense([3, 2, 2, 1]), F32, data, [2, 2, 1], nb)
        assert st == orc.INVALID_VIEW and (out == 9).all(), nb


def test_manifest_rejection_routes():
    s = dense([3, 2, 2, 1])
    st, out = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], s, F32, [1, 0, 0, 1], [2, 2, 1], dne=[3, 4, 1, 1])
    assert st == orc.SHAPE_MISMATCH and (out == 9).all()
    for bad in ([1, -1, 0, 1], [1, 2, 0, 1]):
        st, out = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], s, F32, bad, [2, 2, 1])
        assert st == orc.INDEX_OUT_OF_BOUNDS and (out == 9).all()
    st, _ = gr(orc.GR_F32, ROWS4.view(np.int32).copy(), [3, 2, 2, 1], s, I32, [1, 0, 0, 1], [2, 2, 1])
    assert st == orc.INVALID_VIEW  # unsupported_source_dtype
    st, _ = gr(orc.GR_F32, ROWS4, [3, 2, 2, 1], s, F32, [1, 0, 0], [2, 2, 1])
    assert st == orc.INVALID_VIEW  # short_index_storage
    st, _ = gr(orc.GR_F32, np.array([1, 2], np.float32), [2, 2, 1, 1], [4, 0, 8, 8], F32, [0], [1, 1, 1],
               dne=[2, 1, 1, 1])
    assert st == orc.INVALID_VIEW  # f32_non_singleton_zero_stride (shape would also fail: views come first)


# ---- known answers (tests/any/get_rows_ops.rs) ------------------------------------------


def q4_0_block(scale, packed):
    return np.array([scale & 0xFF, scale >> 8] + [packed] * 16, np.uint8)


def q8_0_block(scale, value):
    return np.array([scale & 0xFF, scale >> 8] + [value & 0xFF] * 32, np.uint8)


def q4_k_block(scale, minimum, packed, scales=(1, 1, 1, 1, 1, 1, 1, 1, 0x11, 0x11, 0x11, 0x11)):
    return np.array([scale & 0xFF, scale >> 8, minimum & 0xFF, minimum >> 8] + list(scales) + [packed] * 128, np.uint8)


def packed(code, cols, rows, outer2=1, outer3=1):
    bv, bb = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144)}[code]
    row = cols // bv * bb
    return [cols, rows, outer2, outer3], [1, row, row * rows, row * rows * outer2]


def test_quantized_known_answers():
    ne, nb = packed(Q4_0, 32, 2)
    src = np.concatenate([q4_0_block(0x3C00, 0x98), q4_0_block(0x3C00, 0xA7)])
    st, out = gr(orc.GR_Q4_0, src, ne, nb, Q4_0, [1, 0], [2, 1, 1])
    assert st == orc.OK
    assert out.tolist() == [-1.0] * 16 + [2.0] * 16 + [0.0] * 16 + [1.0] * 16
    ne, nb = packed(Q8_0, 32, 2)
    src = np.concatenate([q8_0_block(0x3C00, -2), q8_0_block(0x3C00, 1)])
    st, out = gr(orc.GR_Q8_0, src, ne, nb, Q8_0, [1, 0], [2, 1, 1])
    assert st == orc.OK and out.tolist() == [1.0] * 32 + [-2.0] * 32
    ne, nb = packed(Q4_K, 256, 2)
    src = np.concatenate([q4_k_block(0x3C00, 0x3800, 0x43), q4_k_block(0x3C00, 0x3800, 0x21)])
    st, out = gr(orc.GR_Q4_K, src, ne, nb, Q4_K, [1, 0], [2, 1, 1])
    assert st == orc.OK
    assert out[:256].reshape(4, 64)[:, :32].tolist() == [[0.5] * 32] * 4
    assert out[:256].reshape(4, 64)[:, 32:].tolist() == [[1.5] * 32] * 4
    assert out[256:].reshape(4, 64)[:, :32].tolist() == [[2.5] * 32] * 4
    assert out[256:].reshape(4, 64)[:, 32:].tolist() == [[3.5] * 32] * 4
    # upper scale/min groups
    ne, nb = packed(Q4_K, 256, 1)
    src = q4_k_block(0x3C00, 0x3800, 0x21, (0x41, 0x82, 0xC3, 0x04, 0x45, 0x86, 0xC7, 0x08, 0x89, 0x9A, 0xAB, 0xBC))
    st, out = gr(orc.GR_Q4_K, src, ne, nb, Q4_K, [0], [1, 1, 1])
    assert st == orc.OK
    for g, (low, high) in enumerate([(-1.5, 1.0), (-0.5, 4.0), (13.0, 63.5), (30.0, 18.5)]):
        assert out[g * 64:g * 64 + 32].tolist() == [low] * 32
        assert out[g * 64 + 32:(g + 1) * 64].tolist() == [high] * 32


def test_quantized_multiblock_outer_batches():
    indices = [0, 1, 1, 0, 0, 1, 1, 0]
    source_rows = [0, 1, 3, 2, 4, 5, 7, 6]
    # Q4_0: nibble pairs per (row, block)
    blocks = []
    for r in range(8):
        for b in range(2):
            blocks.append(q4_0_block(0x3C00, ((8 + r + b) & 15) | (((9 + r + b) & 15) << 4)))
    ne, nb = packed(Q4_0, 64, 2, 2, 2)
    st, out = gr(orc.GR_Q4_0, np.concatenate(blocks), ne, nb, Q4_0, indices, [2, 2, 2])
    assert st == orc.OK
    for d, r in enumerate(source_rows):
        row = out[d * 64:(d + 1) * 64]
        for b in range(2):
            assert row[b * 32:b * 32 + 16].tolist() == [((8 + r + b) & 15) - 8.0] * 16
            assert row[b * 32 + 16:b * 32 + 32].tolist() == [((9 + r + b) & 15) - 8.0] * 16
    blocks = [q8_0_block(0x3C00, r * 3 + b) for r in range(8) for b in range(2)]
    ne, nb = packed(Q8_0, 64, 2, 2, 2)
    st, out = gr(orc.GR_Q8_0, np.concatenate(blocks), ne, nb, Q8_0, indices, [2, 2, 2])
    assert st == orc.OK
    for d, r in enumerate(source_rows):
        for b in range(2):
            assert out[d * 64 + b * 32:d * 64 + b * 32 + 32].tolist() == [float(r * 3 + b)] * 32
    blocks = [q4_k_block(0x3C00, 0x3800, (1 + r + b) | ((2 + r + b) << 4)) for r in range(8) for b in range(2)]
    ne, nb = packed(Q4_K, 512, 2, 2, 2)
    st, out = gr(orc.GR_Q4_K, np.concatenate(blocks), ne, nb, Q4_K, indices, [2, 2, 2])
    assert st == orc.OK
    for d, r in enumerate(source_rows):
        row = out[d * 512:(d + 1) * 512]
        for b in range(2):
            for g in range(4):
                o = b * 256 + g * 64
                assert row[o:o + 32].tolist() == [1 + r + b - 0.5] * 32
                assert row[o + 32:o + 64].tolist() == [2 + r + b - 0.5] * 32


def test_quantized_empty_indices_are_no_ops_and_malformed_views_invalid():
    for kind, code, cols, block in ((orc.GR_Q4_0, Q4_0, 32, q4_0_block(0x3C00, 0x98)),
                                    (orc.GR_Q8_0, Q8_0, 32, q8_0_block(0x3C00, 1)),
                                    (orc.GR_Q4_K, Q4_K, 256, q4_k_block(0x3C00, 0x3800, 0x21))):
        ne, nb = packed(code, cols, 1)
        st, _ = gr(kind, block, ne, nb, code, np.zeros(0, np.int32), [0, 1, 1], dne=[cols, 0, 1, 1])
        assert st == orc.OK
        st, out = gr(kind, block, ne, [2] + nb[1:], code, [0], [1, 1, 1], fill=7.0)
        assert st == orc.INVALID_VIEW and (out == 7).all()  # nb[0] must be 1
        st, out = gr(kind, block, ne, nb, code, [-1], [1, 1, 1], fill=7.0)
        assert st == orc.INDEX_OUT_OF_BOUNDS and (out == 7).all()
        st, out = gr(kind, block[:-1].copy(), ne, nb, code, [0], [1, 1, 1], fill=7.0)
        assert st == orc.INVALID_VIEW  # the row extends past the storage


# ---- closed forms ------------------------------------------------------------------------


def test_f32_matches_numpy_fancy_indexing_over_batches():
    g = rng(3)
    sne = [17, 40, 3, 2]
    src = g.standard_normal(int(np.prod(sne))).astype(np.float32)
    ine = [25, 3, 2]
    idx = g.integers(0, 40, int(np.prod(ine))).astype(np.int32)
    st, out = gr(orc.GR_F32, src, sne, dense(sne), F32, idx, ine)
    assert st == orc.OK
    s4 = src.reshape(2, 3, 40, 17)
    i3 = idx.reshape(2, 3, 25)
    want = np.stack([np.stack([s4[a, b][i3[a, b]] for b in range(3)]) for a in range(2)])
    assert_bits_equal(out, want.reshape(-1), "f32 gather")


def test_f16_widening_is_exact_including_nan_payloads():
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    st, out = gr(orc.GR_F16, halves, [256, 256, 1, 1], dense([256, 256, 1, 1], 2), F16,
                 np.arange(256, dtype=np.int32), [256, 1, 1])
    assert st == orc.OK
    ref = halves.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref)
    assert_bits_equal(out[finite], ref[finite], "f16 widening")
    # NaNs keep their payload in the high mantissa bits, and quiet/signalling stays as encoded
    nan_bits = halves[~finite].astype(np.uint32)
    want = ((nan_bits & 0x8000) << 16) | 0x7F800000 | ((nan_bits & 0x3FF) << 13)
    assert (out[~finite].view(np.uint32) == want).all()


def test_bf16_widening_and_strided_f16_source():
    g = rng(4)
    vals = g.standard_normal(4 * 6).astype(np.float32)
    st, out = gr(orc.GR_BF16, bf16(vals), [4, 6, 1, 1], dense([4, 6, 1, 1], 2), BF16, [5, 0, 2], [3, 1, 1])
    assert st == orc.OK
    b = (vals.view(np.uint32) & 0xFFFF0000).view(np.float32).reshape(6, 4)
    assert_bits_equal(out, b[[5, 0, 2]].reshape(-1), "bf16")
    # F16 with a column stride of 2 elements reads every other half
    h = g.standard_normal(2 * 4 * 6).astype(np.float16)
    st, out = gr(orc.GR_F16, h.view(np.uint16), [4, 6, 1, 1], [4, 16, 96, 96], F16, [1, 3], [2, 1, 1])
    assert st == orc.OK
    assert_bits_equal(out, h.reshape(6, 8)[[1, 3], ::2].astype(np.float32).reshape(-1), "strided f16")


def q4_0_numpy(blocks):
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32)[:, 0:1]
    q = blocks[:, 2:]
    lo = ((q & 15).astype(np.float32) - 8) * d
    hi = ((q >> 4).astype(np.float32) - 8) * d
    return np.concatenate([lo, hi], axis=1)


def test_quantized_decoders_match_independent_numpy_formulas():
    g = rng(5)
    nblk = 64
    raw = g.integers(0, 256, (nblk, 18), dtype=np.uint8)
    raw[:, :2] = np.frombuffer(g.standard_normal(nblk).astype(np.float16).tobytes(), np.uint8).reshape(nblk, 2)
    ne, nb = packed(Q4_0, 32 * 8, 8)
    st, out = gr(orc.GR_Q4_0, raw.reshape(-1).copy(), ne, nb, Q4_0, np.arange(8)[::-1].astype(np.int32), [8, 1, 1])
    assert st == orc.OK
    want = q4_0_numpy(raw).reshape(8, 8 * 32)[::-1].reshape(-1)
    assert_bits_equal(out, want, "q4_0")
    raw8 = g.integers(0, 256, (nblk, 34), dtype=np.uint8)
    raw8[:, :2] = np.frombuffer(g.standard_normal(nblk).astype(np.float16).tobytes(), np.uint8).reshape(nblk, 2)
    ne, nb = packed(Q8_0, 32 * 8, 8)
    st, out = gr(orc.GR_Q8_0, raw8.reshape(-1).copy(), ne, nb, Q8_0, np.arange(8).astype(np.int32), [8, 1, 1])
    assert st == orc.OK
    d = raw8[:, :2].copy().view(np.float16).astype(np.float32)
    assert_bits_equal(out, (raw8[:, 2:].view(np.int8).astype(np.float32) * d).reshape(-1), "q8_0")
    # Q4_K: scale/min bits of every sub-block from a random 12-byte table
    rawk = g.integers(0, 256, (4, 144), dtype=np.uint8)
    rawk[:, :4] = np.frombuffer(np.abs(g.standard_normal(8)).astype(np.float16).tobytes(), np.uint8).reshape(4, 4)
    ne, nb = packed(Q4_K, 256, 4)
    st, out = gr(orc.GR_Q4_K, rawk.reshape(-1).copy(), ne, nb, Q4_K, np.arange(4).astype(np.int32), [4, 1, 1])
    assert st == orc.OK
    for r in range(4):
        blk = rawk[r]
        d = np.float32(blk[:2].view(np.float16)[0])
        dm = np.float32(blk[2:4].view(np.float16)[0])
        s = blk[4:16].astype(np.uint32)
        sc = [s[j] & 63 if j < 4 else (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4) for j in range(8)]
        mn = [s[j + 4] & 63 if j < 4 else (s[j + 4] >> 4) | ((s[j] >> 6) << 4) for j in range(8)]
        qs = blk[16:]
        want = []
        for grp in range(4):
            q = qs[grp * 32:(grp + 1) * 32]
            want += list(d * np.float32(sc[2 * grp]) * (q & 15).astype(np.float32) - dm * np.float32(mn[2 * grp]))
            want += list(d * np.float32(sc[2 * grp + 1]) * (q >> 4).astype(np.float32) - dm * np.float32(mn[2 * grp + 1]))
        assert_bits_equal(out[r * 256:(r + 1) * 256], np.array(want, np.float32), f"q4_k row {r}")
