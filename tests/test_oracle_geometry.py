"""Packed-VQ geometry (R4): oracle and product host code vs the reference's KATs and its
compiled sources (oracle/_ref)."""
import numpy as np
import pytest

import oracle_lib


def kat_pack(codes, bits):
    # packing loop of tests/quantization_geometry_test.cpp:52-62 (test data generator)
    words = [0] * (((len(codes) + 31) // 32) * bits)
    for i, c in enumerate(codes):
        bit = (i % 32) * bits
        w = (i // 32) * bits + bit // 32
        sh = bit % 32
        v = c << sh
        words[w] |= v & 0xFFFFFFFF
        if sh + bits > 32:
            words[w + 1] |= (v >> 32) & 0xFFFFFFFF
    return np.array(words, np.uint32)


def test_kat_14bit_67_codes(orc):
    expected = [(i * 997 + 17) & 0x3FFF for i in range(67)]
    packed = kat_pack(expected, 14)
    assert len(packed) == 42 == orc.word_count(67, 14)
    assert np.array_equal(orc.pack_row(expected, 14), packed)
    for i, e in enumerate(expected):
        assert orc.unpack(packed, i, 14) == (0, e)


def test_kat_short_buffer_rejected(orc):
    packed = kat_pack([(i * 997 + 17) & 0x3FFF for i in range(67)], 14)
    assert orc.unpack(packed[:13], 31, 14)[0] == -2  # std::out_of_range in the reference


def test_kat_8bit_160_codes(orc):
    codes = [(i * 17 + 255) % 256 for i in range(160)]
    packed = np.zeros(40, np.uint32)
    for i, c in enumerate(codes):
        packed[i // 4] |= np.uint32(c << ((i % 4) * 8))
    assert orc.word_count(160, 8) == 40
    assert np.array_equal(orc.pack_row(codes, 8), packed)
    for i, c in enumerate(codes):
        assert orc.unpack(packed, i, 8) == (0, c)


def test_invalid_bits(orc):
    assert orc.word_count(10, 0) == -1
    assert orc.word_count(10, 32) == -1


@pytest.mark.parametrize("bits", [8, 14, 3, 31])
def test_random_roundtrip_vs_reference_build(orc, bits):
    ref = oracle_lib.load_ref()
    rng = np.random.default_rng(bits)
    for n in (1, 31, 32, 33, 64, 256, 257):
        codes = rng.integers(0, 1 << bits, n, dtype=np.uint64).astype(np.uint32)
        words = orc.pack_row(codes, bits)
        assert np.array_equal(words, kat_pack([int(c) for c in codes], bits))
        for i in range(n):
            assert orc.unpack(words, i, bits) == (0, int(codes[i]))
            if ref is not None:
                assert ref.unpack(words, i, bits) == (0, int(codes[i]))
        if ref is not None:
            assert ref.lib.ref_packed_vq_word_count(n, bits) == orc.word_count(n, bits)
            # short-buffer rejection agrees
            if len(words) > 1:
                assert ref.unpack(words[:-1], n - 1, bits)[0] == orc.unpack(words[:-1], n - 1, bits)[0] == -2


def test_product_host_unpack_matches(orc, q38):
    import ctypes as C
    rng = np.random.default_rng(7)
    for bits in (8, 14):
        codes = rng.integers(0, 1 << bits, 100).astype(np.uint32)
        words = orc.pack_row(codes, bits)
        out = C.c_uint32()
        for i in range(100):
            rc = q38.lib.q38_unpack_vq_code(words.ctypes.data, len(words), i, bits, C.byref(out))
            assert rc == 0 and out.value == codes[i]
        assert q38.lib.q38_unpack_vq_code(words.ctypes.data, 1, 99, bits, C.byref(out)) == q38.Q38_ERANGE
        assert q38.lib.q38_packed_vq_word_count(100, bits) == orc.word_count(100, bits)


def test_supports_segmented_vq_truth_table(q38):
    ref = oracle_lib.load_ref()
    table = {(2, 0): 1, (4, 8): 1, (8, 14): 1, (4, 14): 0, (8, 8): 0, (3, 8): 0}
    for (d, b), v in table.items():
        assert q38.lib.q38_supports_segmented_vq(d, b) == v
        if ref is not None:
            assert ref.lib.ref_supports_segmented_vq(d, b) == v
