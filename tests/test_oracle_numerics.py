"""Pins oracle/numerics.py against torch's own bf16 and float8_e4m3fn casts.

torch is the reference's arithmetic library (autocast bf16 rounding,
engine.py:180-185); fp8 follows torch.float8_e4m3fn, the format the build's
quantized cache uses. The decode table is checked for all 256 codes; the
encoder on random values, every representable value, every midpoint (ties)
and the overflow edges. A planted truncating encoder must fail the same
checks, so they can tell a rounding mistake from the real thing.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import numerics as nm


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_bf16_rounding_random_bits():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    ours = nm.f32_to_bf16_bits(x)
    ref = _torch_bf16_bits(x)
    assert np.array_equal(ours[finite], ref[finite])
    # NaN stays NaN
    assert np.all(np.isnan(nm.bf16_bits_to_f32(ours[~finite & np.isnan(x)])))


def test_bf16_rounding_edges():
    vals = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4028235e38, 1.1754944e-38, 1e-45,
                     1.00390625, 1.01171875, 1.0078125, 1.00390625 + 2**-20, 65504.0, 3.0e38], dtype=np.float32)
    # exact halfway cases between consecutive bf16 values, both parities
    base = nm.bf16_bits_to_f32(np.arange(0x3F80, 0x3F90, dtype=np.uint16))
    mids = ((base[:-1].astype(np.float64) + base[1:]) / 2).astype(np.float32)
    x = np.concatenate([vals, mids, -mids])
    assert np.array_equal(nm.f32_to_bf16_bits(x), _torch_bf16_bits(x))


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = nm.e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.nanmax(ours) == 448.0 and np.sum(np.isnan(ours)) == 2


def _encode_cases():
    rng = np.random.default_rng(1)
    reps = nm.e4m3fn_decode(np.arange(256, dtype=np.uint8))
    reps = np.unique(reps[np.isfinite(reps)]).astype(np.float64)
    mids = (reps[:-1] + reps[1:]) / 2
    nudged = np.concatenate([mids * (1 + 2**-20), mids * (1 - 2**-20)])
    edges = np.array([448, 449, 463.99, 464, 464.01, 479, 480, 500, 1e6, 2.0**-6, 2.0**-7, 2.0**-9, 2.0**-10,
                      1.5 * 2.0**-10, 3 * 2.0**-11, 1e-12, 0.0, np.inf, np.nan])
    rand = np.concatenate([rng.standard_normal(200_000) * s for s in (1e-3, 0.05, 1.0, 30.0, 300.0)])
    x = np.concatenate([reps, mids, nudged, edges, rand]).astype(np.float32)
    return np.concatenate([x, -x])


def test_e4m3_encode_matches_torch():
    x = _encode_cases()
    assert np.array_equal(nm.e4m3fn_encode(x), _torch_e4m3(x))


def test_planted_truncating_encoder_is_caught():
    """A truncating (round-toward-zero) encoder must disagree with torch."""
    x = _encode_cases()
    x = x[np.isfinite(x) & (np.abs(x) < 448)]
    ours = nm.e4m3fn_encode(x)
    table = nm.e4m3fn_decode(np.arange(128, dtype=np.uint8))
    a = np.abs(x)
    trunc = np.searchsorted(table[:127], a, side="right") - 1  # largest code with value <= |x|
    trunc = (trunc.astype(np.uint8) | np.where(np.signbit(x), 0x80, 0).astype(np.uint8))
    assert not np.array_equal(trunc, _torch_e4m3(x))
    assert np.array_equal(ours, _torch_e4m3(x))


def test_quantize_rows_closed_form():
    rng = np.random.default_rng(2)
    x = nm.round_bf16(rng.standard_normal((500, 128)).astype(np.float32))
    x[7] = 0.0
    codes, scales = nm.quantize_e4m3_rows(x)
    absmax = np.abs(x).max(-1)
    assert np.array_equal(scales, (absmax / np.float32(448.0)).astype(np.float32))
    assert scales[7] == 0 and np.all(codes[7] == 0)
    # the absmax element encodes to +-448 (0x7E / 0xFE)
    idx = np.abs(x).argmax(-1)
    top = codes[np.arange(500), idx]
    assert np.all((top[np.arange(500) != 7] & 0x7F) == 0x7E)
    # dequantisation error within half an fp8 ulp (relative 2^-4) of the scaled value
    deq = nm.dequantize_e4m3_rows(codes, scales)
    err = np.abs(deq - x)
    bound = np.maximum(np.abs(x) * 2.0**-4, scales[:, None] * 2.0**-10) * 1.0001
    assert np.all(err <= bound)


def test_quantize_matches_torch_cast_of_ratio():
    """codes == torch's cast of x / scale (the spec's definition)."""
    rng = np.random.default_rng(3)
    x = nm.round_bf16(rng.standard_normal((300, 64)).astype(np.float32) * 3)
    codes, scales = nm.quantize_e4m3_rows(x)
    ratio = torch.from_numpy(x) / torch.from_numpy(scales)[:, None]
    ref = ratio.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, ref)


def test_quantize_rows_with_nan_or_inf_store_nan_codes():
    """A row holding a NaN or an infinity has a non-finite scale (torch's amax
    propagates NaN, as here) and stores NaN codes throughout; finite rows are
    unaffected by their neighbours; an all-zero row stays zeros."""
    x = np.zeros((5, 16), np.float32)
    x[0, :] = np.linspace(-3, 3, 16)
    x[1, :] = np.linspace(-3, 3, 16)
    x[1, 4] = np.nan
    x[2, :] = 1.0
    x[2, 9] = np.inf
    x[3, :] = -2.0
    x[3, 0] = -np.inf
    codes, scales = nm.quantize_e4m3_rows(x)
    assert np.isnan(scales[1]) and np.isinf(scales[2]) and np.isinf(scales[3])
    assert np.all(codes[1:4] == 0x7F)
    assert scales[4] == 0 and np.all(codes[4] == 0)
    want0, s0 = nm.quantize_e4m3_rows(x[:1])
    assert np.array_equal(codes[0], want0[0]) and scales[0] == s0[0]
    # torch's row recipe agrees on NaN-ness for the non-finite rows
    t = torch.from_numpy(x)
    ts = t.abs().amax(-1) / 448.0
    assert torch.equal(torch.isfinite(ts), torch.from_numpy(np.isfinite(scales)))
    # a planted mistake -- an absmax that skips NaN (fmax) -- gives finite codes
    planted = np.nanmax(np.abs(x[1])) / np.float32(448.0)
    assert np.isfinite(planted) and not np.isfinite(scales[1])
