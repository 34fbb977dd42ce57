"""GPU parity: prefill attention (causal GQA over each sequence's cache after
a ragged prompt chunk was appended) vs the fp64 oracle
(oracle.attention.prefill_attention, itself pinned to torch SDPA with the
reference's causal mask).

Tolerance (the path's stated target): |out - ref| <= 2e-3 + 2e-2 * |ref|; fp8
caches against the oracle on the dequantised values. Rows of padding tokens
(t >= new_lens[b]) must stay untouched.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle.attention import prefill_attention as ref_prefill
from tests.kv_inputs import bf16_randn, contiguous_geometry, fill_cache_values, paged_geometry, sm_scale

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 2e-2, 2e-3


def _dev_bf16(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def run_prefill(past, new, Hq=32, Hkv=8, D=128, P=16, paged=True, fp8=False, seed=0, transposed_q=False,
                key_gain=None):
    from tinytron_amd import ops

    rng = np.random.default_rng(seed)
    past = np.asarray(past, np.int32)
    new = np.asarray(new, np.int32)
    B = len(past)
    T = int(new.max())
    total = past + new
    max_len = int(total.max())
    if paged:
        layout, numel, ptab, num_pages = paged_geometry(total, Hkv, D, P, rng)
    else:
        cap = ((max_len + P - 1) // P) * P
        layout, numel = contiguous_geometry(B, Hkv, D, cap, P, fp8=fp8)
    data = fill_cache_values(layout, numel, B, total, rng, fp8=fp8, key_gain=key_gain)
    if transposed_q:
        qb, qf = bf16_randn(rng, (B, T, Hq, D))
        q = _dev_bf16(qb).transpose(1, 2)
        qf = qf.transpose(0, 2, 1, 3)
    else:
        qb, qf = bf16_randn(rng, (B, Hq, T, D))
        q = _dev_bf16(qb)
    kv = ops.KVLayout(
        k=_dev_bf16(data["k_store"]) if not fp8 else torch.from_numpy(data["k_store"]).to(DEV),
        v=_dev_bf16(data["v_store"]) if not fp8 else torch.from_numpy(data["v_store"]).to(DEV),
        strides=(layout.seq_stride, layout.page_stride, layout.head_stride), num_heads=Hkv, head_dim=D,
        page_size=P, capacity=int(layout.capacity), kind="fp8" if fp8 else "bf16",
        page_table=torch.from_numpy(ptab).to(DEV) if paged else None, num_pages=num_pages if paged else 0,
        k_scale=torch.from_numpy(data["k_scale"]).to(DEV) if fp8 else None,
        v_scale=torch.from_numpy(data["v_scale"]).to(DEV) if fp8 else None,
    )
    out = torch.full((B, T, Hq, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ops.prefill_attention(q, kv, torch.from_numpy(past).to(DEV), max_len, new_lens=torch.from_numpy(new).to(DEV),
                          out=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = ref_prefill(qf, data["keys"], data["values"], past, new, Hkv, sm_scale(D))
    return got, ref, new


def check(got, ref, new):
    for b, n in enumerate(new):
        g, r = got[b, :n], ref[b, :n]
        assert np.all(np.isfinite(g)), f"sequence {b}: non-finite output"
        err = np.abs(g - r)
        bad = err > ATOL + RTOL * np.abs(r)
        assert not bad.any(), f"sequence {b}: {bad.sum()} out of tolerance, max err {err.max():.3e}"
        assert np.all(np.isnan(got[b, n:])), f"sequence {b}: padding rows were written"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("paged", [False, True])
def test_prefill_ragged_bf16(D, paged):
    got, ref, new = run_prefill([0, 5, 100, 31], [40, 1, 77, 33], D=D, paged=paged, seed=D + paged)
    check(got, ref, new)


@pytest.mark.parametrize("paged", [False, True])
def test_prefill_ragged_fp8(paged):
    got, ref, new = run_prefill([0, 17, 64], [50, 16, 3], paged=paged, fp8=True, seed=9 + paged)
    check(got, ref, new)


@pytest.mark.parametrize("G", [1, 2, 3, 8, 16])
def test_prefill_group_sizes(G):
    """16 / G query tokens per wave (G = 3: five tokens and one padding column)."""
    Hkv = 2
    got, ref, new = run_prefill([3, 0, 20], [21, 9, 14], Hq=Hkv * G, Hkv=Hkv, D=64, seed=G)
    check(got, ref, new)


def test_prefill_transposed_q_and_long_prompt():
    """q as the transposed view Attention.forward produces; a prompt longer
    than one 8-tile chunk of keys (past 300 + 260 new)."""
    got, ref, new = run_prefill([300, 0], [260, 129], Hq=16, Hkv=4, D=64, seed=5, transposed_q=True)
    check(got, ref, new)


def test_prefill_single_token_equals_decode():
    """T = 1: the prefill kernel computes the decode step (same oracle)."""
    got, ref, new = run_prefill([10, 0, 333], [1, 1, 1], seed=2)
    check(got, ref, new)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("G", [1, 4])
def test_prefill_mask_edges_at_tile_boundaries(G, fp8):
    """The causal mask runs only on tiles reaching past the smallest key limit
    of a wave's columns: limits landing exactly on, just before and just after
    32-key tile boundaries, prompts ending there, and (G = 1) a wave spanning
    64 tokens, so up to three edge tiles per wave."""
    Hkv = 2
    past = [0, 31, 32, 33, 63, 95, 0, 1, 30, 62]
    new = [32, 1, 33, 64, 65, 97, 128, 31, 1, 2]  # 30 + 1, 62 + 2: a limit one key short of a tile end
    got, ref, n = run_prefill(past, new, Hq=Hkv * G, Hkv=Hkv, D=64, fp8=fp8, seed=40 + G + fp8)
    check(got, ref, n)


@pytest.mark.parametrize("fp8", [False, True])
def test_prefill_growing_scores(fp8):
    """Scores that keep growing along the sequence: the running maximum
    climbs past its slack (8 in log2 units) tile after tile in the middle of
    the key loop, so O and the sums are rescaled while holding mass; between
    those steps P runs above 1 under a stale maximum. Keys gain a factor 2
    every 24 tokens, and one sequence has a single spiking key in the middle."""
    def gain(b, L):
        t = np.arange(L, dtype=np.float64)
        g = 2.0 ** (t / 24.0)
        if b == 2:
            g = np.ones(L)
            g[L // 2] = 40.0
        return np.minimum(g, 2.0 ** 8)

    Hkv = 2
    got, ref, new = run_prefill([0, 150, 0], [300, 90, 257], Hq=Hkv * 4, Hkv=Hkv, D=64, fp8=fp8, seed=77 + fp8,
                                key_gain=gain)
    check(got, ref, new)
