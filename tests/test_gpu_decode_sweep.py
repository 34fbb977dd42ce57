"""GPU parity: a seeded sweep of decode-attention shapes against the fp64
oracle, beyond the hand-picked cases of test_gpu_decode_attention.py.

Each case draws a batch size (1-12), group size (powers of two and 3, 5, 6)
and KV-head count (H_q <= 32), head_dim (24, 32, 48, 64, 96, 128: fp8 caches
at 24 run the VALU kernel), layout (paged with a power-of-two page, or the reference's
contiguous store with any page size), cache dtype (bf16 / fp8) and per-sequence
lengths from a mix of edge values (1, page and tile boundaries) and uniform
draws, and the partition (balanced; one workgroup per segment, split_tokens -1;
or one per length-rank pair, -2, ranked on the GPU or with the caller's order).
Tolerance as in test_gpu_decode_attention.py.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_decode_attention import assert_close, run_case

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 511, 512, 513]


def _case(i):
    rng = np.random.default_rng(9000 + i)
    B = int(rng.integers(1, 13))
    G = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 16]))
    hkv = int(rng.choice([h for h in (1, 2, 4, 8) if G * h <= 32]))
    D = int(rng.choice([24, 32, 48, 64, 64, 96, 128, 128]))
    paged = bool(rng.integers(0, 2))
    P = int(rng.choice([16, 32, 64])) if paged else int(rng.choice([16, 48, 100]))
    fp8 = bool(rng.integers(0, 2))
    lengths = [int(rng.choice(EDGES)) if rng.random() < 0.4 else int(rng.integers(1, 900)) for _ in range(B)]
    split = int(rng.choice([0, 0, -1, -2, -2]))  # balanced, one workgroup per segment, or per rank pair
    order = "sorted" if split == -2 and rng.integers(0, 2) else None  # paired: the caller's order, or ranked on the GPU
    return dict(lengths=lengths, Hq=G * hkv, Hkv=hkv, D=D, P=P, paged=paged, fp8=fp8, seed=100 + i,
                split_tokens=split, length_order=order)


@pytest.mark.parametrize("i", range(40))
def test_decode_attention_sweep(i):
    c = _case(i)
    print(f"sweep case {i}: {c}", flush=True)
    got, ref, _ = run_case(**c)
    assert_close(got, ref)
