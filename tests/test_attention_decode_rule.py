"""CPU check of the INT8 attention operands' in-register decodes
(csrc/attention.hip: MfmaTile<KvFormat::I8>::kop / vop and i8x4_to_f16)
over every byte value in every byte position.

K operand: the dword is xor-ed with 0x80808080 (code + 128 as an unsigned
byte), v_perm_b32 with the constant 0x64646464 as the high operand and
selectors 0x07010600 / 0x07030602 puts bytes (0, 1) / (2, 3) under 0x64
exponent bytes, the fp16 pair is 1024 + (code + 128) and subtracting 1152
leaves the code. V operand: v_perm_b32 of two dwords with selector
0x0C000C00 | (4 + b) << 16 | b takes byte b of each under zero bytes, xor
0x64806480 sets the exponents and flips the sign bit, giving the biased
value 1152 + code (the bias is removed later from the sum of P).
i8x4_to_f16: the same as the K operand with zero bytes and an or of
0x64006400. The steps are restated on uint32 / float16 arrays; the decoded
values must equal the int8 codes exactly, and planted wrong constants must
fail.
"""
from __future__ import annotations

import numpy as np


def _perm(hi: np.ndarray, lo: np.ndarray, sel: int) -> np.ndarray:
    """v_perm_b32: byte k of the result is byte sel_k of {hi, lo} (0-3 lo,
    4-7 hi), 0x0C gives 0x00."""
    out = np.zeros_like(lo, dtype=np.uint32)
    for k in range(4):
        s = (sel >> (8 * k)) & 0xFF
        if s == 0x0C:
            b = np.zeros_like(lo, dtype=np.uint32)
        elif s < 4:
            b = (lo >> np.uint32(8 * s)) & np.uint32(0xFF)
        else:
            b = (hi >> np.uint32(8 * (s - 4))) & np.uint32(0xFF)
        out |= b << np.uint32(8 * k)
    return out


def _halves(y: np.ndarray):
    return ((y & np.uint32(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64),
            (y >> np.uint32(16)).astype(np.uint16).view(np.float16).astype(np.float64))


def _codes_and_words():
    codes = np.arange(-128, 128, dtype=np.int64)
    rng = np.random.default_rng(9)
    words = []
    for pos in range(4):   # every code in every byte position, the other bytes random
        w = rng.integers(0, 2 ** 32, size=256, dtype=np.uint64).astype(np.uint32)
        w = (w & np.uint32(~(0xFF << (8 * pos)) & 0xFFFFFFFF)) | ((codes & 0xFF).astype(np.uint32) << np.uint32(8 * pos))
        words.append(w)
    return codes, words


def _byte_codes(w: np.ndarray) -> np.ndarray:
    """int8 codes of the 4 bytes of each word, [n, 4]."""
    return np.stack([((w >> np.uint32(8 * k)) & np.uint32(0xFF)).astype(np.uint8).view(np.int8).astype(np.float64)
                     for k in range(4)], axis=1)


def _kop(w: np.ndarray, e8: int = 0x64646464, bias: float = 1152.0) -> np.ndarray:
    wi = w ^ np.uint32(0x80808080)
    e = np.full_like(w, e8)
    a0, a1 = _halves(_perm(e, wi, 0x07010600))
    a2, a3 = _halves(_perm(e, wi, 0x07030602))
    return np.stack([a0, a1, a2, a3], axis=1) - bias


def _vop(w_even: np.ndarray, w_odd: np.ndarray, byte: int, x: int = 0x64806480) -> np.ndarray:
    sel = 0x0C000C00 | ((4 + byte) << 16) | byte
    lo, hi = _halves(_perm(w_odd, w_even, sel) ^ np.uint32(x))
    return np.stack([lo, hi], axis=1)   # biased: 1152 + code


def _i8x4(w: np.ndarray, orc: int = 0x64006400) -> np.ndarray:
    wi = w ^ np.uint32(0x80808080)
    z = np.zeros_like(w)
    lo0, lo1 = _halves(_perm(z, wi, 0x0C010C00) | np.uint32(orc))
    hi0, hi1 = _halves(_perm(z, wi, 0x0C030C02) | np.uint32(orc))
    return np.stack([lo0, lo1, hi0, hi1], axis=1) - 1152.0


def test_k_operand_and_i8x4_decode_every_byte():
    _, words = _codes_and_words()
    for w in words:
        assert np.array_equal(_kop(w), _byte_codes(w))
        assert np.array_equal(_i8x4(w), _byte_codes(w))


def test_v_operand_is_code_plus_1152_every_byte():
    _, words = _codes_and_words()
    rng = np.random.default_rng(11)
    for w in words:
        other = rng.integers(0, 2 ** 32, size=w.size, dtype=np.uint64).astype(np.uint32)
        for byte in range(4):
            got = _vop(w, other, byte)
            assert np.array_equal(got[:, 0] - 1152.0, _byte_codes(w)[:, byte])
            assert np.array_equal(got[:, 1] - 1152.0, _byte_codes(other)[:, byte])


def test_planted_wrong_constants_fail():
    _, words = _codes_and_words()
    w = words[0]
    assert not np.array_equal(_kop(w, bias=1024.0), _byte_codes(w))
    assert not np.array_equal(_kop(w, e8=0x64006400), _byte_codes(w))
    other = words[1]
    assert not np.array_equal(_vop(w, other, 0, x=0x64006400)[:, 0] - 1152.0, _byte_codes(w)[:, 0])
