"""CPU check of the W4A16 kernels' in-register nibble decodes over every
byte value: i4x8_to_f16_natural (the LDS-staged GEMM) and
i4x8_to_f16_pairs (the 64 x 128-tile GEMM and the GEMVs), both in
csrc/w4a16.hip.

Per pair i of a packed word the kernel copies byte i to bytes 0 and 2
(v_perm_b32 selector 0x0C000C00 | i << 16 | i), keeps bits 0-3 of the low
half and bits 4-7 of the high half (mask 0x00F0000F), xors 0x54806408 (the
exponents of 1024.0 and 64.0 and bit 3 of each nibble) and subtracts the
fp16 pair (1032, 72). The steps are restated here on uint32 / float16
arrays and must give the two's-complement codes of K positions 2i and
2i + 1 that the oracle's unpack_int4_along_k gives, for all 2^8 byte values
in every byte position. A planted wrong exponent constant must fail.
"""
from __future__ import annotations

import numpy as np

from oracle import w4a16 as ow


def _decode(words: np.ndarray, x: int = 0x54806408) -> np.ndarray:
    """uint32 [n] -> int codes [n, 8] in K order, as the kernel forms them."""
    w = words.astype(np.uint32)
    out = np.empty((w.size, 8), dtype=np.float64)
    for i in range(4):
        b = (w >> np.uint32(8 * i)) & np.uint32(0xFF)            # byte i
        dup = b | (b << np.uint32(16))                            # bytes 0 and 2
        y = (dup & np.uint32(0x00F0000F)) ^ np.uint32(x)
        lo = (y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16)
        hi = (y >> np.uint32(16)).astype(np.uint16).view(np.float16)
        out[:, 2 * i] = (lo - np.float16(1032.0)).astype(np.float16)
        out[:, 2 * i + 1] = (hi - np.float16(72.0)).astype(np.float16)
    return out


def _words():
    # every byte value in every byte position, other bytes random
    rng = np.random.default_rng(5)
    base = rng.integers(0, 2 ** 32, size=(4, 256), dtype=np.uint64).astype(np.uint32)
    for i in range(4):
        base[i] = (base[i] & np.uint32(~(0xFF << (8 * i)) & 0xFFFFFFFF)) | (np.arange(256, dtype=np.uint32) << np.uint32(8 * i))
    return base.reshape(-1)


def test_decode_matches_oracle_unpack_for_every_byte():
    w = _words()
    want = ow.unpack_int4_along_k(w.view(np.int32).reshape(1, -1)).reshape(8, -1).T.astype(np.float64)
    got = _decode(w)
    assert np.array_equal(got, want)
    assert set(np.unique(got)) == set(range(-8, 8))


def test_planted_wrong_exponent_fails():
    w = _words()
    want = ow.unpack_int4_along_k(w.view(np.int32).reshape(1, -1)).reshape(8, -1).T.astype(np.float64)
    assert not np.array_equal(_decode(w, x=0x54006408), want)   # nibble bit 3 not flipped in the high half
    assert not np.array_equal(_decode(w, x=0x64806408), want)   # high half at 1024 instead of 64


def _decode_pairs(words: np.ndarray, x_lo: int = 0x64086408, x_hi: int = 0x64806480) -> np.ndarray:
    """i4x8_to_f16_pairs: pair j holds the codes of K positions (j, j + 4).
    Masks 0x000F000F / 0x00F000F0 on the word and on the word >> 8; the
    low-nibble pairs become 1024 + u, the high-nibble pairs 1024 + 16 u,
    scaled by 1/16 and biased by (1032) or (72) in fp16. Returns K order."""
    w = words.astype(np.uint32)
    w8 = w >> np.uint32(8)
    out = np.empty((w.size, 8), dtype=np.float64)

    def halves(y):
        return ((y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16),
                (y >> np.uint32(16)).astype(np.uint16).view(np.float16))

    for j, (src, mask, x, sixteenth) in enumerate(((w, 0x000F000F, x_lo, False), (w, 0x00F000F0, x_hi, True),
                                                   (w8, 0x000F000F, x_lo, False), (w8, 0x00F000F0, x_hi, True))):
        lo, hi = halves((src & np.uint32(mask)) ^ np.uint32(x))
        for pos, v in ((j, lo), (j + 4, hi)):
            if sixteenth:
                r = ((v * np.float16(0.0625)).astype(np.float16) - np.float16(72.0)).astype(np.float16)
            else:
                r = (v - np.float16(1032.0)).astype(np.float16)
            out[:, pos] = r
    return out


def test_pair_decode_matches_oracle_unpack_for_every_byte():
    w = _words()
    want = ow.unpack_int4_along_k(w.view(np.int32).reshape(1, -1)).reshape(8, -1).T.astype(np.float64)
    assert np.array_equal(_decode_pairs(w), want)
    assert not np.array_equal(_decode_pairs(w, x_lo=0x64006400), want)   # nibble bit 3 not flipped

