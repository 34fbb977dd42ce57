"""Bit-level bf16 and fp8-e4m3fn rounding in numpy (oracle; test infrastructure).

The reference computes in bf16 under ``torch.autocast`` (engine.py:180-185):
every elementwise op takes bf16 operands, computes in fp32 and rounds the
result to bf16 with round-to-nearest-even. This module emulates exactly that
rounding so that the oracle can predict the reference's bytes.

fp8-e4m3fn is not in the reference (it has no quantized cache). The format is
the OCP "e4m3fn" one used by ``torch.float8_e4m3fn``: bias 7, 3 mantissa bits,
no infinities, 0x7F/0xFF are NaN, max finite 448, subnormals m * 2**-9.

Pinned by tests/test_oracle_numerics.py: bf16 rounding against torch's
``.to(torch.bfloat16)`` on random bit patterns and edge values; fp8 decode
against torch for all 256 codes; fp8 encode against torch's cast on random
values, every representable value, every midpoint and the overflow edges.
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------
# bf16
# ----------------------------------------------------------------------------


def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round to nearest even; NaN -> quiet."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if np.any(nan):
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round fp32 values to the nearest bf16 value (returned as fp32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ----------------------------------------------------------------------------
# fp8 e4m3fn
# ----------------------------------------------------------------------------

E4M3_MAX = 448.0
_E4M3_NAN = 0x7F


def e4m3fn_decode_table() -> np.ndarray:
    """All 256 codes -> fp32 value, from the format definition."""
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * 2.0 ** -9
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out


_DECODE = e4m3fn_decode_table()


def e4m3fn_decode(codes) -> np.ndarray:
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


def e4m3fn_encode(x) -> np.ndarray:
    """fp32 -> e4m3fn code, round to nearest even, the way torch casts.

    Magnitudes above 464 (the midpoint between 448 and the unrepresentable
    480) and non-finite inputs become NaN (0x7F with the input's sign bit);
    464 itself ties to the even mantissa, i.e. 448.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = ((x.view(np.uint32) >> 24) & 0x80).astype(np.uint8)
    bad = ~np.isfinite(x) | (np.abs(x) > 464.0)
    a = np.where(bad, 0.0, np.abs(x).astype(np.float64))
    code = np.zeros(x.shape, dtype=np.int64)

    sub = a < 2.0 ** -6
    # subnormal range: value = q * 2**-9, q in [0, 8]; q == 8 is the code of
    # the smallest normal (exp 1, man 0), so the code is q itself.
    code = np.where(sub, np.rint(a * 2.0 ** 9).astype(np.int64), code)

    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(sub, 1.0, a)))
    e = np.clip(e, -6, 8)
    # q in [8, 16]: (1 + man/8) * 8 rounded half-to-even at the 3-bit mantissa
    q = np.rint(np.where(sub, 8.0, a) / 2.0 ** (e - 3)).astype(np.int64)
    bump = q >= 16
    e = np.where(bump, e + 1, e)
    q = np.where(bump, q // 2, q)
    normal_code = ((e.astype(np.int64) + 7) << 3) | (q - 8)
    code = np.where(sub, code, normal_code)

    code = np.where(bad, _E4M3_NAN, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def quantize_e4m3_rows(x_f32: np.ndarray):
    """Per-row symmetric fp8 quantization: this build's fp8-e4m3 cache format
    (the reference has no fp8 cache; one scale per (token, head) row).

    For each row (last axis = head_dim): absmax = max|x| in fp32 (NaN if the
    row holds a NaN), scale = absmax / 448 (fp32 division, round to nearest),
    q = e4m3(x / scale) with fp32 division; an all-zero row stores zeros with
    scale 0, and a row whose scale is not finite (it holds a NaN or an
    infinity, which the format cannot represent) stores NaN codes (0x7F).
    Returns (codes uint8 [..., D], scales fp32 [...]).
    """
    x = np.asarray(x_f32, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        absmax = np.max(np.abs(x), axis=-1).astype(np.float32)
        scale = (absmax / np.float32(E4M3_MAX)).astype(np.float32)
        bad = ~np.isfinite(scale)
        safe = np.where((scale == 0) | bad, np.float32(1.0), scale).astype(np.float32)
        ratio = np.where(bad[..., None], np.float32(0.0), x / safe[..., None]).astype(np.float32)
    codes = e4m3fn_encode(ratio)
    codes = np.where((scale == 0)[..., None], np.uint8(0), codes).astype(np.uint8)
    codes = np.where(bad[..., None], np.uint8(_E4M3_NAN), codes).astype(np.uint8)
    return codes, scale


def dequantize_e4m3_rows(codes, scales) -> np.ndarray:
    """float(q) * scale, per row (fp32)."""
    return (e4m3fn_decode(codes) * np.asarray(scales, np.float32)[..., None]).astype(np.float32)
