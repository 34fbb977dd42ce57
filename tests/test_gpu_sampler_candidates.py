"""GPU: the sampler's candidate path (2 <= top_k <= 64 over more than 8192
logits: 8192-logit chunks reduced to their top-k candidates on workgroups of
their own, then one wave per row) against the one-workgroup-per-row path of
the same library (the C ABI with no workspace) and against oracle/sampler.py.

Both paths apply the same rules to the same fixed-point masses, so the drawn
tokens are equal; the token's log-probability differs only by the order in
which the kept tokens' exp() terms are added (within 1e-5 |ref| + 2e-5).
Against the oracle, tokens are compared on rows whose top-p cut is not within
1e-6 of a cumulative probability (as in the sampler sweep). The edge cases
force the whole-row fallback inside the same launch: ties at the row's
boundary beyond a chunk's 64 slots, more than 64 kept tokens, fewer than k
finite logits.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import sampler as osm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _whole_row(x, temperature, top_k, top_p, seed, offset):
    from tinytron_amd import _lib

    M, V = x.shape
    tok = torch.empty(M, dtype=torch.int64, device=DEV)
    lp = torch.empty(M, dtype=torch.float32, device=DEV)
    lib = _lib.load()
    fn = lib.tt_sample_bf16 if x.dtype == torch.bfloat16 else lib.tt_sample_f32
    st = fn(x.data_ptr(), x.stride(0), M, V, float(temperature), int(top_k or 0),
            1.0 if top_p is None else float(top_p), seed, offset, tok.data_ptr(), lp.data_ptr(), None, V, None, 0,
            torch._C._cuda_getCurrentRawStream(torch.cuda.current_device()))
    _lib.check(st, "whole-row sampler")
    return tok, lp


def _check(x_dev, temperature, top_k, top_p, seed, offset, oracle=True):
    from tinytron_amd import _lib, ops

    M, V = x_dev.shape
    assert _lib.load().tt_sample_workspace_bytes(M, V, top_k) > 0  # the candidate path runs
    tok, lp = ops.sample_tokens(x_dev, temperature, top_k, top_p, seed, offset, return_logprob=True)
    tok_w, lp_w = _whole_row(x_dev, temperature, top_k, top_p, seed, offset)
    torch.cuda.synchronize()
    assert torch.equal(tok, tok_w)
    assert torch.allclose(lp, lp_w, rtol=1e-5, atol=2e-5)
    if oracle:
        xn = x_dev.float().cpu().numpy()
        want = osm.sample(xn, temperature, top_k, top_p, seed, offset)
        rows = np.arange(M)
        if top_p is not None:
            rows = np.flatnonzero(osm.top_p_margin(xn, temperature, top_k, top_p) > 1e-6)
        got = tok.cpu().numpy()
        for r in rows:
            assert got[r] == want[r], f"row {r}: token {got[r]} != oracle {want[r]}"
    return tok


@pytest.mark.parametrize("i", range(24))
def test_candidate_path_sweep(i):
    rng = np.random.default_rng(9100 + i)
    f32 = bool(rng.integers(0, 2))
    V = int(rng.choice([8193, 16384, 32000, 50257] if not f32 else [8193, 20000, 32000, 32768]))
    M = int(rng.choice([1, 7, 64]))
    scale = float(rng.choice([0.5, 2.0, 8.0]))
    temperature = float(rng.choice([1.0, 0.8, 1.3]))
    top_k = int(rng.choice([2, 5, 50, 64]))
    top_p = [None, 0.05, 0.9, 0.999][int(rng.integers(0, 4))]
    pad = int(rng.choice([0, 3, 8]))
    print(f"candidate case {i}: f32 {f32} V {V} M {M} scale {scale} T {temperature} k {top_k} p {top_p} pad {pad}",
          flush=True)
    dtype = torch.float32 if f32 else torch.bfloat16
    g = torch.Generator().manual_seed(100 + i)
    wide = (torch.randn(M, V + pad, generator=g) * scale).to(dtype).to(DEV)
    _check(wide[:, :V], temperature, top_k, top_p, 500 + i, i)


def test_headline_shape_many_draws():
    """[64, 32000] bf16 at temperature 0.8, top-k 50, top-p 0.9 (the engine's
    sampling settings): 16 successive offsets."""
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(64, 32000, generator=g) * 3).to(torch.bfloat16).to(DEV)
    for offset in range(16):
        _check(x, 0.8, 50, 0.9, 1234, offset, oracle=offset < 2)


@pytest.mark.parametrize("case", ["boundary_ties", "flat", "few_finite", "many_kept", "ties_in_one_chunk"])
def test_candidate_path_edge_cases(case):
    g = torch.Generator().manual_seed(11)
    M, V = 6, 32000
    if case == "boundary_ties":      # values on a coarse grid: the k-th largest has ties across chunks
        x = torch.round(torch.randn(M, V, generator=g) * 2) / 2
    elif case == "flat":             # every logit equal
        x = torch.zeros(M, V)
    elif case == "few_finite":       # fewer than k finite logits
        x = torch.full((M, V), float("-inf"))
        x[:, ::5000] = torch.randn(M, x[:, ::5000].shape[1], generator=g)
    elif case == "many_kept":        # ties at the k-th largest that keep more than 64 tokens
        x = torch.randn(M, V, generator=g) - 10
        x[:, 100:200] = 5.0
    else:                            # 100 ties at the top inside one chunk, k = 50
        x = torch.randn(M, V, generator=g)
        x[:, 9000:9100] = 6.0
    x = x.to(torch.bfloat16).to(DEV)
    for top_p in (None, 0.9):
        _check(x, 1.0, 50, top_p, 99, 3, oracle=case != "few_finite")
