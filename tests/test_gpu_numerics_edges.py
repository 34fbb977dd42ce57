"""GPU: the kernels' bf16 and fp8-e4m3fn conversions on crafted values,
against the oracle's integer formulations (oracle/numerics.py), byte for byte.

The device conversions are gfx950's v_cvt_pk_bf16_f32 and v_cvt_pk_fp8_f32
(plus a patch for positive NaN); random inputs rarely land on the cases where
a rounding rule shows. These rows do:

* bf16: fp32 round-to-nearest-even ties (both parities), values that round up
  into the next binade and past the largest finite value to inf, NaNs of both
  signs (signalling ones become quiet), +-inf, fp32 subnormals and their
  ties, signed zeros -- pushed through the V path of the q|k|v split-K partial
  inputs (one split: the kernel converts the fp32 value itself), bf16 cache.
* fp8: rows anchored at +-448 (scale exactly 1, so every code is e4m3fn of
  the crafted value): ties at every binade (ties to the even mantissa),
  subnormals on the 2^-9 grid and the ties between them, the tie into the
  smallest normal, signed zeros; a row holding a NaN, rows holding +-inf
  (NaN codes throughout, non-finite scale), an all-zero row (scale 0), a row of
  fp32-subnormal magnitude -- through the split-K partial path, the prompt
  path (T > 1, vector kernel) and the fused decode step (RoPE + append inside
  the attention launch).

K rows hold finite values only (RoPE multiplies by sin(0) = 0, and inf * 0
yields a NaN whose sign is the platform's choice); the oracle rotates them
with its own rope_apply.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import kvcache as okv
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits, quantize_e4m3_rows
from oracle.rope import rope_apply

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 64
P = 16


def _f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


# fp32 patterns whose bf16 rounding exercises every rule
BF16_EDGE = _f32([
    0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000,  # ties: to even (down), to even (up)
    0x3F80C000, 0x3F807FFF, 0x3F80FFFF, 0x3FFFFFFF,  # above / below a tie, carry into the next binade
    0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0xFF7FFFFF,  # largest finite: to inf, tie to inf, stays finite
    0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFA00000,  # NaNs (quiet / signalling, both signs)
    0x7F800000, 0xFF800000, 0x00000000, 0x80000000,  # +-inf, +-0
    0x00008000, 0x00018000, 0x00010001, 0x807FFFFF,  # fp32 subnormals: ties, truncation, carry to normal
    0x00800000, 0x00807FFF, 0x00808000, 0x00818000,  # smallest normal and its neighbours
])

# finite bf16-exact values whose e4m3fn code (scale 1) exercises every rule
_TIES = [(1 + (2 * m + 1) / 16.0) * 2.0 ** e for e in (-6, -3, 0, 2, 5, 7) for m in range(7)]
E4M3_EDGE = np.array(
    _TIES + [-t for t in _TIES[::5]]
    + [2.0 ** -10, 3 * 2.0 ** -10, 5 * 2.0 ** -10, 7 * 2.0 ** -10, 13 * 2.0 ** -10, 15 * 2.0 ** -10,
       2.0 ** -11, 2.0 ** -9, 6 * 2.0 ** -9, 2.0 ** -6, 432.0, 400.0, 448.0, -432.0, 0.0, -0.0,
       2.0 ** -12, -(2.0 ** -10)],
    dtype=np.float32)


def _rows(n_rows, rng):
    """Crafted fp32 rows of D values (the edge values, then random fill)."""
    rows = (rng.standard_normal((n_rows, D)) * 2).astype(np.float32)
    return rows


def _e4m3_rows(rng):
    """V rows for the fp8 rule: [anchor 448, edge values ...] in several rows,
    a NaN row, +inf / -inf rows, a zero row, a row of fp32-subnormal values."""
    edge = E4M3_EDGE
    per = D - 1
    n_edge = (len(edge) + per - 1) // per
    rows = []
    for r in range(n_edge):
        chunk = edge[r * per:(r + 1) * per]
        row = np.zeros(D, np.float32)
        row[0] = 448.0 if r % 2 == 0 else -448.0
        row[1:1 + len(chunk)] = chunk
        rows.append(row)
    nan_row = (rng.standard_normal(D) * 3).astype(np.float32)
    nan_row[17] = np.nan
    pinf = (rng.standard_normal(D)).astype(np.float32)
    pinf[5] = np.inf
    ninf = (rng.standard_normal(D)).astype(np.float32)
    ninf[40] = -np.inf
    tiny = (rng.standard_normal(D) * 1e-40).astype(np.float32)
    rows += [nan_row, pinf, ninf, np.zeros(D, np.float32), tiny]
    out = np.stack(rows)
    return bf16_bits_to_f32(f32_to_bf16_bits(out))  # the inputs are bf16 values


def _k_rows(n, rng):
    """Finite K rows: e4m3 edge values behind a 448 anchor (rotated at position 0)."""
    rows = np.zeros((n, D), np.float32)
    for r in range(n):
        vals = np.roll(E4M3_EDGE, 7 * r)[:D - 1]
        rows[r, 0] = 448.0
        rows[r, 1:1 + len(vals)] = vals
    return bf16_bits_to_f32(f32_to_bf16_bits(rows))


def _layout(B, fp8):
    from tinytron_amd import ops

    lay = okv.contiguous_layout(B, 1, D, 2 * P, P)
    numel = okv.contiguous_numel(B, 1, D, 2 * P, P)
    if fp8:
        k = torch.full((numel,), 0x55, dtype=torch.uint8, device=DEV)
        v = k.clone()
        ks = torch.full((okv.fp8_scale_numel(numel // D),), -1.0, dtype=torch.float32, device=DEV)
        vs = ks.clone()
    else:
        k = torch.zeros(numel, dtype=torch.bfloat16, device=DEV)
        v = k.clone()
        ks = vs = None
    kv = ops.KVLayout(k=k, v=v, strides=(lay.seq_stride, lay.page_stride, lay.head_stride), num_heads=1,
                      head_dim=D, page_size=P, capacity=2 * P, kind="fp8" if fp8 else "bf16", k_scale=ks,
                      v_scale=vs)
    return kv, lay


def _slot(lay, b, t):
    return int(lay.token_offsets(b, t + 1)[t, 0])


def _check_fp8_rows(kv, lay, rows_k, rows_v, positions):
    """Cache codes and scales at each row's slot == oracle.quantize_e4m3_rows."""
    kc, vc = kv.k.cpu().numpy(), kv.v.cpu().numpy()
    ksc, vsc = kv.k_scale.cpu().numpy(), kv.v_scale.cpu().numpy()
    for name, rows, codes, scales in (("k", rows_k, kc, ksc), ("v", rows_v, vc, vsc)):
        want_c, want_s = quantize_e4m3_rows(rows)
        for b, (row, t) in enumerate(zip(rows, positions)):
            off = _slot(lay, b, t)
            got = codes[off:off + D]
            assert np.array_equal(got, want_c[b]), (
                f"{name} row {b}: codes differ at {np.flatnonzero(got != want_c[b])[:8]} "
                f"(got {got[got != want_c[b]][:8]}, want {want_c[b][got != want_c[b]][:8]})")
            gs, ws = scales[okv.fp8_scale_index(off // D)], want_s[b]
            assert (np.isnan(gs) and np.isnan(ws)) or gs.view(np.uint32) == ws.view(np.uint32), (
                f"{name} row {b}: scale {gs!r} != {ws!r}")


def _rope_table(n):
    from tinytron_amd import ops

    t = ops.build_rope_table(n, D, dtype=torch.bfloat16, device=DEV)
    return t, t.float().cpu().numpy()


def test_bf16_rounding_of_partial_inputs():
    """The V path of rope_append_partials with one split: the kernel rounds the
    fp32 value to bf16 itself -- every edge pattern, compared bit for bit."""
    from tinytron_amd import ops

    rng = np.random.default_rng(0)
    n_rows = (len(BF16_EDGE) + D - 1) // D + 1
    B = n_rows
    vrows = _rows(n_rows, rng)
    flat = vrows.reshape(-1)
    flat[:len(BF16_EDGE)] = BF16_EDGE
    kv, lay = _layout(B, fp8=False)
    krows = _rows(B, rng)
    qrows = _rows(B, rng)
    parts = np.concatenate([qrows, krows, vrows], axis=1)[None]  # [1, B, (1 + 2) D]
    table, _ = _rope_table(4)
    pos = torch.zeros(B, dtype=torch.int32, device=DEV)
    ops.rope_append_partials(torch.from_numpy(np.ascontiguousarray(parts)).to(DEV), 1, table, pos, kv)
    torch.cuda.synchronize()
    got = kv.v.cpu().view(torch.int16).numpy().view(np.uint16)
    want = f32_to_bf16_bits(vrows)
    for b in range(B):
        off = _slot(lay, b, 0)
        bad = np.flatnonzero(got[off:off + D] != want[b])
        assert bad.size == 0, (f"row {b}: bf16 bits differ at {bad[:8]}: got "
                               f"{[hex(x) for x in got[off:off + D][bad[:8]]]}, want {[hex(x) for x in want[b][bad[:8]]]}")


@pytest.mark.parametrize("path", ["partials", "prompt", "fused"])
def test_fp8_row_quantization_edges(path):
    """fp8-e4m3 cache rows with crafted values: every code and scale equals the
    oracle's, including NaN / inf rows (NaN codes, non-finite scale)."""
    from tinytron_amd import ops

    rng = np.random.default_rng(1)
    vrows = _e4m3_rows(rng)
    B = vrows.shape[0]
    krows = _k_rows(B, rng)
    qrows = bf16_bits_to_f32(f32_to_bf16_bits(_rows(B, rng)))
    kv, lay = _layout(B, fp8=True)
    table, table_np = _rope_table(4)
    if path == "partials":
        parts = np.concatenate([qrows, krows, vrows], axis=1)[None]
        pos = torch.zeros(B, dtype=torch.int32, device=DEV)
        ops.rope_append_partials(torch.from_numpy(np.ascontiguousarray(parts)).to(DEV), 1, table, pos, kv)
        positions = [0] * B
        krot = rope_apply(krows[:, None, :], table_np[0][None, None, :], "bf16")[:, 0]
        _check_fp8_rows(kv, lay, krot, vrows, positions)
    elif path == "prompt":
        # T = 2 new tokens per sequence: token 0 the crafted row (position 0), token 1 a random one
        T = 2
        k_in = np.stack([krows, bf16_bits_to_f32(f32_to_bf16_bits(_rows(B, rng)))], axis=1)  # [B, T, D]
        v_in = np.stack([vrows, bf16_bits_to_f32(f32_to_bf16_bits(_rows(B, rng)))], axis=1)
        q_in = np.stack([qrows, qrows], axis=1)

        def dev(x):  # [B, T, D] -> bf16 [B, 1, T, D]
            return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)[:, None].to(DEV)

        pos = torch.zeros(B, dtype=torch.int32, device=DEV)
        ops.rope_append(dev(q_in), dev(k_in), dev(v_in), table, pos, kv)
        for t in range(T):
            krot = rope_apply(k_in[:, t][:, None, :], table_np[t][None, None, :], "bf16")[:, 0]
            _check_fp8_rows(kv, lay, krot, v_in[:, t], [t] * B)
    else:
        # the fused step at position 3 (three finite tokens cached before it)
        from tests.kv_inputs import bf16_randn

        L0 = 3
        pre_k = np.stack([bf16_randn(rng, (L0, D))[1] for _ in range(B)])
        pre_v = np.stack([bf16_randn(rng, (L0, D))[1] for _ in range(B)])

        def dev(x):
            return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)[:, None].to(DEV)

        zero = torch.zeros(B, dtype=torch.int32, device=DEV)
        ops.rope_append(dev(np.zeros((B, L0, D), np.float32)), dev(pre_k), dev(pre_v), table, zero, kv)
        pos = torch.full((B,), L0, dtype=torch.int32, device=DEV)

        def dev1(x):  # [B, D] -> bf16 [B, 1, D]
            return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)[:, None].to(DEV)

        table8, table8_np = _rope_table(8)
        ops.decode_attention_append(table8, pos, kv, L0 + 1, q=dev1(qrows), k=dev1(krows), v=dev1(vrows))
        krot = rope_apply(krows[:, None, :], table8_np[L0][None, None, :], "bf16")[:, 0]
        _check_fp8_rows(kv, lay, krot, vrows, [L0] * B)
    torch.cuda.synchronize()
