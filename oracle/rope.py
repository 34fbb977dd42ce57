"""RoPE oracle (test infrastructure): table and per-op-rounded rotation.

Restates ``rope_impl`` of the reference (tinytron/model/modules/attn.py:13-63):

    inv_freq = 1 / (theta ** (arange(0, D, 2, fp32) / D))        attn.py:30-32
    freqs    = einsum("bt,d->btd", pos.float(), inv_freq)         attn.py:46
    emb      = cat(freqs, freqs)                                   attn.py:50
    cos, sin = emb.cos().to(q.dtype), emb.sin().to(q.dtype)        attn.py:53-54
    out      = (x * cos) + (rotate_half(x) * sin)                  attn.py:61-62
    rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])              attn.py:56-59

Under bf16 autocast each of ``*``, ``*`` and ``+`` rounds to bf16, so the
oracle rounds after each op (fp32 compute, RNE to bf16). In fp32 each op rounds
to fp32 and nothing is fused.

Because ``emb = cat(freqs, freqs)``, columns i and i + D/2 of cos (and sin) are
equal; the table therefore stores [cos(f_0..f_{D/2-1}) | sin(f_0..f_{D/2-1})]
per position, D values per row.

Pinned by tests/test_oracle_rope.py: the table against the fp64 closed form
cos/sin(pos * theta**(-2i/D)); the rotation against the fp64 2-D rotation of
the pairs (x_i, x_{i+D/2}) (norm preserved, pos 0 is the identity); and the
per-op rounding against torch's own bf16 / fp32 elementwise ops applied in the
reference's order.
"""
from __future__ import annotations

import numpy as np

from .numerics import round_bf16


def rope_inv_freq(head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """attn.py:30-32 in fp32."""
    exps = (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), exps).astype(np.float32)).astype(np.float32)


def rope_table(num_positions: int, head_dim: int, theta: float = 10000.0, dtype: str = "bf16") -> np.ndarray:
    """[num_positions, D] fp32 values: cos in [:, :D/2], sin in [:, D/2:].

    Values are rounded to ``dtype`` ("bf16" or "f32"), attn.py:53-54.
    """
    inv = rope_inv_freq(head_dim, theta)
    pos = np.arange(num_positions, dtype=np.float32)
    freqs = (pos[:, None] * inv[None, :]).astype(np.float32)
    cos = np.cos(freqs).astype(np.float32)
    sin = np.sin(freqs).astype(np.float32)
    table = np.concatenate([cos, sin], axis=-1)
    if dtype == "bf16":
        table = round_bf16(table)
    return table.astype(np.float32)


def rope_apply(x: np.ndarray, table_rows: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Rotate x [..., D] with table rows [..., D] (cos | sin) broadcast to x.

    Each op rounds to ``dtype`` exactly as the reference's three tensor ops do.
    """
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    h = d // 2
    cos = table_rows[..., :h].astype(np.float32)
    sin = table_rows[..., h:].astype(np.float32)
    c = np.concatenate([cos, cos], axis=-1)
    s = np.concatenate([sin, sin], axis=-1)
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)
    rnd = round_bf16 if dtype == "bf16" else (lambda v: np.asarray(v, np.float32))
    a = rnd((x * c).astype(np.float32))
    b = rnd((rot * s).astype(np.float32))
    return rnd((a + b).astype(np.float32))


def rope_apply_at(x: np.ndarray, positions: np.ndarray, table: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """x [B, H, T, D]; positions [B, T] (int) -> rotated x (same shape)."""
    rows = table[np.asarray(positions, dtype=np.int64)]  # [B, T, D]
    return rope_apply(x, rows[:, None, :, :], dtype)


def rope_rotate_f64(x: np.ndarray, positions: np.ndarray, head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """Closed form in fp64: rotate pair (x_i, x_{i+D/2}) by pos * theta**(-2i/D)."""
    x = np.asarray(x, dtype=np.float64)
    h = head_dim // 2
    inv = theta ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.asarray(positions, np.float64)[..., None] * inv  # [B, T, D/2]
    ang = ang[:, None]  # broadcast over heads
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :h], x[..., h:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
