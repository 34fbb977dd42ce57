"""Pins oracle/rope.py.

* per-op rounding: bit-exact against torch's own bf16 / fp32 ops applied in
  the reference's order (oracle.ref_path.rope_impl restates attn.py:13-63);
* the table against the fp64 closed form within fp32 angle rounding;
* the rotation against the fp64 2-D rotation of (x_i, x_{i+D/2});
* planted mistakes (sign of rotate_half, paired index) fail the closed form.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import ref_path
from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits, round_bf16
from oracle.rope import rope_apply, rope_apply_at, rope_rotate_f64, rope_table


def _table_from_torch(n, D, dtype):
    """The cos/sin values rope_impl builds (attn.py:30-54), first half of emb."""
    pos = torch.arange(n).unsqueeze(0)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    freqs = torch.einsum("bt,d->btd", pos.float(), inv)[0]
    return torch.cat([freqs.cos().to(dtype), freqs.sin().to(dtype)], -1).float().numpy()


@pytest.mark.parametrize("D", [64, 128])
def test_table_closed_form(D):
    n = 8192
    t = rope_table(n, D, dtype="f32")
    pos = np.arange(n, dtype=np.float64)[:, None]
    ang = pos * (1.0 / 10000.0 ** (np.arange(0, D, 2) / D))
    exact = np.concatenate([np.cos(ang), np.sin(ang)], -1)
    bound = np.concatenate([ang, ang], -1) * 2.0 ** -21 + 2e-7
    assert np.all(np.abs(t - exact) <= bound)
    tb = rope_table(n, D, dtype="bf16")
    assert np.array_equal(tb, round_bf16(t))


@pytest.mark.parametrize("D", [64, 128])
def test_table_vs_torch_cpu(D):
    """numpy and torch fp32 pow/cos may differ in the last ulp; the bf16
    tables then agree everywhere except at rare rounding boundaries."""
    n = 4096
    ours = rope_table(n, D, dtype="f32")
    ref = _table_from_torch(n, D, torch.float32)
    pos = np.arange(n, dtype=np.float64)[:, None]
    ang = pos * (1.0 / 10000.0 ** (np.arange(0, D, 2) / D))
    assert np.all(np.abs(ours - ref) <= np.concatenate([ang, ang], -1) * 2.0 ** -20 + 4e-7)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_bitexact_vs_torch_ops(dtype, D):
    """Same table, same inputs: oracle == torch ops in the reference order."""
    rng = np.random.default_rng(D)
    B, H, T = 3, 5, 7
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = rng.standard_normal((B, H, T, D)).astype(np.float32) * 2
    if dtype == "bf16":
        x = round_bf16(x)
    pos = rng.integers(0, 3000, size=(B, T))
    # the reference builds cos/sin from positions; use its own op sequence
    q = torch.from_numpy(x).to(tdt)
    qr, kr = ref_path.rope_impl(q, q.clone(), torch.from_numpy(pos))
    table = _table_from_torch(3000, D, tdt)
    ours = rope_apply_at(x, pos, table, dtype)
    ref = qr.float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_rope_closed_form_and_invariants():
    rng = np.random.default_rng(5)
    B, H, T, D = 2, 3, 4, 128
    x = rng.standard_normal((B, H, T, D)).astype(np.float32)
    pos = rng.integers(0, 2000, size=(B, T))
    table = rope_table(2000, D, dtype="f32")
    got = rope_apply_at(x, pos, table, "f32").astype(np.float64)
    exact = rope_rotate_f64(x, pos, D)
    ang_max = 2000.0
    assert np.max(np.abs(got - exact)) < ang_max * 2.0 ** -20 * 8 + 1e-5
    # norm of every (x_i, x_{i+D/2}) pair preserved
    h = D // 2
    n_in = x[..., :h] ** 2 + x[..., h:] ** 2
    n_out = got[..., :h] ** 2 + got[..., h:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)
    # position 0 is the identity
    zero = rope_apply_at(x, np.zeros((B, T), np.int64), table, "f32")
    assert np.array_equal(zero, x)


def test_planted_rotation_mistakes_fail_closed_form():
    rng = np.random.default_rng(6)
    B, H, T, D = 1, 2, 3, 64
    x = rng.standard_normal((B, H, T, D)).astype(np.float32)
    pos = np.array([[5, 77, 901]])
    table = rope_table(1000, D, dtype="f32")
    rows = table[pos][:, None]
    exact = rope_rotate_f64(x, pos, D)
    h = D // 2
    c = np.concatenate([rows[..., :h]] * 2, -1)
    s = np.concatenate([rows[..., h:]] * 2, -1)
    wrong_sign = x * c + np.concatenate([x[..., h:], -x[..., :h]], -1) * s
    wrong_pair = x * c + np.concatenate([-x[..., 1::2], x[..., 0::2]], -1) * s
    for bad in (wrong_sign, wrong_pair):
        assert np.max(np.abs(bad - exact)) > 1e-2
    assert np.max(np.abs(rope_apply(x, rows, "f32") - exact)) < 1e-4
