"""GPU parity: a seeded sweep of RoPE + append shapes against the oracle, bit
for bit (the checks of test_gpu_rope_append._case: rotated q, every cache
byte, fp8 codes and scales, untouched slots), beyond its hand-picked cases:
head_dim 16-128 including ones that are not powers of two (those take the
one-element-per-lane kernel, the others the four-pair-per-lane one), one to
33 new tokens with ragged counts, bf16 / fp8 / fp32 caches, paged /
contiguous layouts and group sizes.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_rope_append import _case

pytestmark = pytest.mark.gpu


def _params(i):
    rng = np.random.default_rng(4000 + i)
    kind = str(rng.choice(["bf16", "fp8", "f32"]))
    D = int(rng.choice([16, 32, 48, 64, 96, 128]))
    T = int(rng.choice([1, 2, 9, 17, 33]))
    hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    paged = bool(rng.integers(0, 2))
    return dict(kind=kind, paged=paged, D=D, T=T, seed=600 + i, Hq=G * hkv, Hkv=hkv, ragged_new=bool(T > 1 and rng.integers(0, 2)))


@pytest.mark.parametrize("i", range(30))
def test_rope_append_sweep(i):
    p = _params(i)
    print(f"sweep case {i}: {p}", flush=True)
    _case(**p)


@pytest.mark.parametrize("i", range(20))
def test_rope_append_packed_rows_sweep(i):
    """Packed prompt rows equal the grid path bit for bit over head_dim 16-128
    (the four-pair lanes for powers of two, one element per lane otherwise),
    ragged new tokens (including none), cached prefixes, bf16 / fp8, layouts."""
    from tests.test_gpu_rope_append import packed_vs_grid

    rng = np.random.default_rng(4500 + i)
    kind = str(rng.choice(["bf16", "fp8"]))
    D = int(rng.choice([16, 32, 48, 64, 96, 128]))
    hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    paged = bool(rng.integers(0, 2))
    page = int(rng.choice([16, 32]))
    B = int(rng.integers(1, 7))
    new = [int(rng.choice([0, 1, 8, 9, 40])) if rng.random() < 0.4 else int(rng.integers(1, 70)) for _ in range(B)]
    if max(new) == 0:
        new[-1] = 3
    pre = [int(rng.integers(0, 50)) for _ in range(B)]
    print(f"sweep case {i}: {kind} D {D} G {G} hkv {hkv} paged {paged} page {page} new {new} pre {pre}", flush=True)
    packed_vs_grid(kind, paged, D, G * hkv, hkv, new, pre, seed=4600 + i, page=page)
