"""GPU parity: a seeded sweep of prefill-attention shapes against the fp64
oracle, beyond the hand-picked cases of test_gpu_prefill_attention.py.

Each case draws a batch size (1-6), group size (including ones that do not
divide 16) and KV-head count, head_dim 24-128 (the presets' 24, 32, 48, 64, 128 and 96), layout and page size, cache
dtype (bf16 / fp8), the tokens already cached per sequence (0 or more) and
the new tokens per sequence (ragged, including 0 and 1). Tolerance and the
untouched-padding check as in test_gpu_prefill_attention.py.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_prefill_attention import check, run_prefill

pytestmark = pytest.mark.gpu


def _case(i):
    rng = np.random.default_rng(7000 + i)
    B = int(rng.integers(1, 7))
    G = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    hkv = int(rng.choice([h for h in (1, 2, 4) if G * h <= 32]))
    D = int(rng.choice([24, 32, 48, 64, 64, 96, 128, 128]))
    paged = bool(rng.integers(0, 2))
    P = int(rng.choice([16, 32, 64])) if paged else int(rng.choice([16, 48]))
    fp8 = bool(rng.integers(0, 2)) and D % 16 == 0  # fp8 tiles: head_dim % 16 == 0
    past = [int(rng.choice([0, 0, 1, 15, 16, 33])) if rng.random() < 0.5 else int(rng.integers(0, 400))
            for _ in range(B)]
    new = [int(rng.choice([0, 1, 2, 16, 17])) if rng.random() < 0.3 else int(rng.integers(1, 200)) for _ in range(B)]
    if max(new) == 0:
        new[0] = 1
    return dict(past=past, new=new, Hq=G * hkv, Hkv=hkv, D=D, P=P, paged=paged, fp8=fp8, seed=500 + i)


@pytest.mark.parametrize("i", range(30))
def test_prefill_attention_sweep(i):
    c = _case(i)
    print(f"sweep case {i}: {c}", flush=True)
    got, ref, new = run_prefill(**c)
    check(got, ref, new)
