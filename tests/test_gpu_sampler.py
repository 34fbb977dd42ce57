"""GPU: the one-launch sampler (tinytron/inference/sampler.py:6-62) against
oracle/sampler.py.

* greedy (top_k = 1): the token is the first maximum, bit-exact, and its
  log-probability is -log(number of tied maxima kept);
* the full log_softmax of the filtered logits: the -inf pattern (which
  tokens survive temperature / top-k / top-p) equals the oracle's exactly,
  except on rows whose top-p cut sits within 1e-6 of a cumulative
  probability (the device sums fixed-point masses, the oracle float64, and
  the reference fp32: such rows are rounding-dependent in all three); the
  finite values agree within 2e-5 + 1e-5 |ref| (fp32 exp / log);
* the drawn token equals the oracle's inverse-CDF draw with the same
  SplitMix64 uniform, and the draws' frequencies follow softmax.
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import sampler as osm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _logits(M, V, dtype, seed, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, V, generator=g) * scale).to(dtype)
    return x


def _np(x: torch.Tensor) -> np.ndarray:
    return x.float().numpy()


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 32000), (torch.float32, 32000), (torch.bfloat16, 65536),
                                     (torch.float32, 32768), (torch.bfloat16, 1003), (torch.float32, 7),
                                     (torch.bfloat16, 1)])
def test_greedy_is_first_argmax(dtype, V):
    from tinytron_amd import ops

    x = _logits(64, V, dtype, seed=V)
    if V > 2:  # planted exact ties in some rows: the first index wins
        x[3, V // 3] = x[3, 2 * V // 3] = 100.0
        x[5, V - 1] = x[5, 1] = 50.0
    xd = x.to(DEV)
    tok, lp = ops.sample_tokens(xd, top_k=1, return_logprob=True)
    want = osm.greedy(_np(x))
    assert torch.equal(tok.cpu(), torch.from_numpy(want))
    ties = (x.float() == x.float().max(-1, keepdim=True).values).sum(-1)
    assert torch.allclose(lp.cpu(), -torch.log(ties.float()), atol=1e-6)


CASES = [
    # temperature, top_k, top_p
    (1.0, None, None),
    (0.7, None, None),
    (1.0, 5, None),
    (1.3, 100, None),
    (1.0, None, 0.9),
    (0.8, None, 0.3),
    (1.0, 50, 0.8),
    (1.0, 2, 0.99),
    (1.0, 1, 0.5),
]


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 32000), (torch.float32, 32000), (torch.bfloat16, 1003),
                                     (torch.float32, 64), (torch.bfloat16, 40000)])
@pytest.mark.parametrize("temperature,top_k,top_p", CASES)
def test_filtered_log_probs_and_draw_match_oracle(dtype, V, temperature, top_k, top_p):
    from tinytron_amd import ops

    M = 16
    x = _logits(M, V, dtype, seed=7 * V + (top_k or 0))
    xn = _np(x)
    seed, offset = 1234, 5
    tok, lp, full = ops.sample_tokens(x.to(DEV), temperature, top_k, top_p, seed, offset,
                                      return_logprob=True, return_logprobs=True)
    tok, lp, full = tok.cpu().numpy(), lp.cpu().numpy(), full.cpu().numpy()
    f = osm.filter_logits(xn, temperature, top_k, top_p)
    ref = osm.log_probs(f)
    if top_p is not None:
        margin = osm.top_p_margin(xn, temperature, top_k, top_p)
        rows = np.flatnonzero(margin > 1e-6)
        assert len(rows) >= M - 2
    else:
        rows = np.arange(M)
    want = osm.sample(xn, temperature, top_k, top_p, seed, offset)
    for r in rows:
        assert np.array_equal(np.isfinite(full[r]), np.isfinite(ref[r])), f"row {r}: kept set differs"
        fin = np.isfinite(ref[r])
        assert np.allclose(full[r][fin], ref[r][fin], rtol=1e-5, atol=2e-5), f"row {r}"
        assert tok[r] == want[r], f"row {r}: token {tok[r]} != oracle {want[r]}"
    for r in range(M):
        assert np.isfinite(full[r, tok[r]]), f"row {r}: drew a filtered token"
        assert lp[r] == full[r, tok[r]]


def test_top_p_equal_values_keep_first_in_index_order():
    from tinytron_amd import ops

    x = torch.full((2, 16), float("-inf"))
    x[:, :10] = 0.5
    _, full = ops.sample_tokens(x.to(DEV), top_p=0.35, return_logprobs=True)
    full = full.cpu()
    for r in range(2):
        assert torch.isfinite(full[r]).nonzero().flatten().tolist() == [0, 1, 2]
        assert torch.allclose(full[r, :3], torch.full((3,), -math.log(3.0)), atol=1e-6)


def test_top_k_counts_duplicates_and_keeps_ties():
    from tinytron_amd import ops

    # values 5, 4, 4, 4, 3, ...: top_k = 2 -> the 2nd largest is 4, all three 4s kept
    x = torch.tensor([[3.0, 4.0, 5.0, 4.0, 1.0, 4.0, 2.0, 0.0]])
    _, full = ops.sample_tokens(x.to(DEV), top_k=2, return_logprobs=True)
    assert torch.isfinite(full.cpu()[0]).nonzero().flatten().tolist() == [1, 2, 3, 5]
    # fewer finite values than k: every finite value kept
    y = torch.tensor([[1.0, float("-inf"), 2.0, float("-inf")]])
    _, full = ops.sample_tokens(y.to(DEV), top_k=3, return_logprobs=True)
    assert torch.isfinite(full.cpu()[0]).tolist() == [True, False, True, False]


def test_draw_frequencies_follow_softmax():
    from tinytron_amd import ops

    base = torch.tensor([2.0, 0.5, 1.0, -1.0, 0.0, 1.5, float("-inf"), 0.25])
    n = 20000
    x = base.expand(n, 8).contiguous().to(DEV)
    tok = ops.sample_tokens(x, seed=99, offset=0).cpu().numpy()
    counts = np.bincount(tok, minlength=8)
    p = torch.softmax(base.double(), 0).numpy()
    assert counts[6] == 0
    live = p > 0
    chi2 = float(((counts[live] - n * p[live]) ** 2 / (n * p[live])).sum())
    assert chi2 < 35.0  # df 6: p ~ 1e-5


def test_seed_and_offset_determine_the_draw():
    from tinytron_amd import ops

    x = _logits(32, 5000, torch.bfloat16, seed=3).to(DEV)
    a = ops.sample_tokens(x, seed=1, offset=0)
    b = ops.sample_tokens(x, seed=1, offset=0)
    c = ops.sample_tokens(x, seed=1, offset=1)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


def test_strided_rows_and_empty_batch():
    from tinytron_amd import ops

    x3 = _logits(8, 3 * 4000, torch.bfloat16, seed=4).view(8, 3, 4000).to(DEV)
    last = x3[:, -1, :]
    a, la = ops.sample_tokens(last, 0.9, 20, 0.95, 5, 6, return_logprobs=True)
    b, lb = ops.sample_tokens(last.contiguous(), 0.9, 20, 0.95, 5, 6, return_logprobs=True)
    assert torch.equal(a, b) and torch.equal(la, lb)
    # a row stride that is not a multiple of 8 elements takes the scalar loads
    x = _logits(4, 1001, torch.bfloat16, seed=5)
    wide = torch.zeros(4, 1003, dtype=torch.bfloat16)
    wide[:, :1001] = x
    a, la = ops.sample_tokens(wide.to(DEV)[:, :1001], top_k=7, seed=2, return_logprobs=True)
    b, lb = ops.sample_tokens(x.to(DEV), top_k=7, seed=2, return_logprobs=True)
    assert torch.equal(a, b) and torch.equal(la, lb)
    empty = ops.sample_tokens(torch.empty(0, 100, dtype=torch.bfloat16, device=DEV))
    assert empty.shape == (0,)


def test_errors():
    from tinytron_amd import ops

    x = torch.zeros(2, 10, device=DEV)
    with pytest.raises(ValueError, match="temperature must be > 0"):
        ops.sample_tokens(x, temperature=0.0)
    with pytest.raises(ValueError, match="vocab size"):
        ops.sample_tokens(torch.zeros(1, 32769, device=DEV))
    with pytest.raises(ValueError, match="vocab size"):
        ops.sample_tokens(torch.zeros(1, 65537, dtype=torch.bfloat16, device=DEV))


def test_engine_sampler_follows_torch_seed():
    from tinytron_amd import sampler

    x = _logits(8, 3000, torch.bfloat16, seed=6).to(DEV)
    torch.manual_seed(17)
    a = [sampler.sample_next_token(x, top_p=0.9) for _ in range(3)]
    torch.manual_seed(17)
    b = [sampler.sample_next_token(x, top_p=0.9) for _ in range(3)]
    assert all(torch.equal(u, v) for u, v in zip(a, b))
    tok, lp = sampler.sample_next_token_with_log_prob(x, temperature=0.5, top_k=10)
    assert tok.dtype == torch.int64 and lp.dtype == torch.float32 and bool(torch.all(lp <= 0))
    assert torch.equal(sampler.sample_next_token(x, top_k=1), torch.argmax(x.float(), -1))


def test_sampler_manual_seed_counts_calls():
    from tinytron_amd import ops, sampler

    x = _logits(8, 3000, torch.bfloat16, seed=8).to(DEV)
    sampler.manual_seed(5)
    a = [sampler.sample_next_token(x, top_k=50) for _ in range(2)]
    sampler.manual_seed(None)
    assert torch.equal(a[0], ops.sample_tokens(x, top_k=50, seed=5, offset=0))
    assert torch.equal(a[1], ops.sample_tokens(x, top_k=50, seed=5, offset=1))


@pytest.mark.parametrize("top_p", [None, 0.5, 0.1, 0.99])
def test_greedy_kernel_matches_full_sampler_on_ties(top_p):
    # top_k = 1 without full log-prob rows runs the greedy kernel; with them,
    # the general kernel: same token and token log-probability, ties included
    from tinytron_amd import ops

    x = _logits(8, 5000, torch.bfloat16, seed=11)
    x[:, 100] = x[:, 900] = x[:, 1300] = x[:, 4000] = x[:, 4999] = 60.0  # five tied maxima
    x[3, 2000] = 70.0  # a single maximum in row 3
    xd = x.to(DEV)
    t1, l1 = ops.sample_tokens(xd, top_k=1, top_p=top_p, return_logprob=True)
    t2, l2, full = ops.sample_tokens(xd, top_k=1, top_p=top_p, return_logprob=True, return_logprobs=True)
    assert torch.equal(t1, t2) and torch.equal(l1, l2)
    kept = 5 if top_p is None else max(1, int(top_p * 5))
    want = torch.full((8,), -math.log(kept))
    want[3] = 0.0
    assert torch.allclose(l1.cpu(), want, atol=1e-6)
    assert int(t1[0]) == 100 and int(t1[3]) == 2000


@pytest.mark.parametrize("temperature,top_k,top_p", CASES)
def test_filter_logits_matches_oracle(temperature, top_k, top_p):
    """tinytron_amd.sampler.filter_logits (the reference's exported function,
    sampler.py:6-36): -inf exactly where the oracle filters, logits / T elsewhere."""
    from tinytron_amd.sampler import filter_logits

    M, V = 16, 32000
    x = _logits(M, V, torch.bfloat16, seed=11 * V + (top_k or 0))
    xn = _np(x)
    got = filter_logits(x.to(DEV), temperature, top_k, top_p).cpu().numpy()
    want = osm.filter_logits(xn, temperature, top_k, top_p)
    rows = np.arange(M)
    if top_p is not None:
        rows = np.flatnonzero(osm.top_p_margin(xn, temperature, top_k, top_p) > 1e-6)
        assert len(rows) >= M - 2
    for r in rows:
        fin = np.isfinite(want[r])
        assert np.array_equal(np.isfinite(got[r]), fin), f"row {r}: kept set differs"
        # the kept values are the reference's own op, logits / temperature, run by
        # torch on the device (which multiplies by the reciprocal): within one fp32
        # ulp of the host's correctly rounded division, equal at temperature 1
        expect = (x[r].float() / temperature if temperature != 1.0 else x[r].float()).numpy()
        if temperature == 1.0:
            assert np.array_equal(got[r][fin], expect[fin]), f"row {r}: kept values differ"
        else:
            assert np.allclose(got[r][fin], expect[fin], rtol=2.4e-7, atol=0), f"row {r}: kept values differ"
    with pytest.raises(ValueError):
        filter_logits(x.to(DEV), temperature=0.0)
