"""GPU: a seeded sweep of fused decode-step shapes (RoPE + append inside the
attention launch, tt_decode_attn_append_*) against the two-launch path, bit
for bit (test_gpu_decode_fused._run_both: output, every cache byte, fp8
scales, lengths): batch sizes, group sizes (3, 5, 6 too), head_dim 24-128, bf16 / fp8 caches,
paged / contiguous layouts and page sizes, bf16 inputs or 1-4 split-K
partials, edge and random lengths, balanced, per-segment or paired partition
(ranked on the GPU or with the caller's length order).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_decode_fused import _run_both, _setup

pytestmark = pytest.mark.gpu

EDGES = [1, 15, 16, 31, 32, 33, 64, 511, 512]


@pytest.mark.parametrize("i", range(24))
def test_fused_step_sweep(i):
    rng = np.random.default_rng(5000 + i)
    B = int(rng.integers(1, 10))
    G = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 16]))
    hkv = int(rng.choice([h for h in (1, 2, 4) if G * h <= 32]))
    D = int(rng.choice([24, 32, 48, 64, 64, 96, 128, 128]))
    kv = str(rng.choice(["bf16", "fp8"])) if D % 16 == 0 else "bf16"
    paged = bool(rng.integers(0, 2))
    page = int(rng.choice([16, 32, 64]))
    S = int(rng.integers(0, 5))
    split = int(rng.choice([0, 0, -1, -2, -2]))  # balanced, one workgroup per segment, or per rank pair
    sorted_order = bool(split == -2 and rng.integers(0, 2))  # paired: the caller's order, or ranked on the GPU
    lens = [int(rng.choice(EDGES)) if rng.random() < 0.4 else int(rng.integers(1, 700)) for _ in range(B)]
    print(f"sweep case {i}: B {B} G {G} hkv {hkv} D {D} kv {kv} paged {paged} page {page} S {S} split {split} "
          f"lens {lens}", flush=True)
    layer, table, g = _setup(kv, paged, D, G * hkv, hkv, lens, page=page, seed=i)
    _run_both(layer, table, g, G * hkv, from_partials=S > 0, S=max(S, 1), split_tokens=split,
              sorted_order=sorted_order)
