"""GPU: a seeded sweep of sampler settings against oracle/sampler.py, beyond
the grid of test_gpu_sampler.py: vocabulary sizes from 1 to the limits (the
per-thread element counts 8-64), row strides, logit scales (peaked and flat
rows), temperatures, top-k from 1 to beyond V, top-p from tiny to near 1,
bf16 and fp32 logits. Same checks: the kept set (-inf pattern) and drawn token
equal the oracle's on rows whose top-p cut is not within 1e-6 of a cumulative
probability, log-probabilities within 2e-5 + 1e-5 |ref|, the token's
log-probability equal to its row entry.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import sampler as osm

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("i", range(30))
def test_sampler_sweep(i):
    from tinytron_amd import ops

    rng = np.random.default_rng(8000 + i)
    f32 = bool(rng.integers(0, 2))
    vmax = ops.SAMPLE_MAX_VOCAB[torch.float32 if f32 else torch.bfloat16]
    V = int(rng.choice([1, 2, 7, 100, 1000, 5003, 32000, vmax]))
    M = int(rng.integers(1, 40))
    scale = float(rng.choice([0.1, 1.0, 3.0, 20.0]))
    temperature = float(rng.choice([1.0, 0.5, 1.7]))
    top_k = [None, 1, 2, 10, 50, 1000, V + 5][int(rng.integers(0, 7))]
    top_p = [None, 0.05, 0.5, 0.9, 0.999][int(rng.integers(0, 5))]
    pad = int(rng.choice([0, 3, 8]))
    print(f"sweep case {i}: f32 {f32} V {V} M {M} scale {scale} T {temperature} k {top_k} p {top_p} pad {pad}",
          flush=True)
    dtype = torch.float32 if f32 else torch.bfloat16
    g = torch.Generator().manual_seed(i)
    wide = (torch.randn(M, V + pad, generator=g) * scale).to(dtype)
    x = wide[:, :V]
    xn = x.float().numpy()
    seed, offset = 77 + i, i
    tok, lp, full = ops.sample_tokens(wide.to(DEV)[:, :V], temperature, top_k, top_p, seed, offset,
                                      return_logprob=True, return_logprobs=True)
    tok, lp, full = tok.cpu().numpy(), lp.cpu().numpy(), full.cpu().numpy()
    f = osm.filter_logits(xn, temperature, top_k, top_p)
    ref = osm.log_probs(f)
    rows = np.arange(M)
    if top_p is not None:
        rows = np.flatnonzero(osm.top_p_margin(xn, temperature, top_k, top_p) > 1e-6)
    want = osm.sample(xn, temperature, top_k, top_p, seed, offset)
    for r in rows:
        assert np.array_equal(np.isfinite(full[r]), np.isfinite(ref[r])), f"row {r}: kept set differs"
        fin = np.isfinite(ref[r])
        assert np.allclose(full[r][fin], ref[r][fin], rtol=1e-5, atol=2e-5), f"row {r}"
        assert tok[r] == want[r], f"row {r}: token {tok[r]} != oracle {want[r]}"
    for r in range(M):
        assert np.isfinite(full[r, tok[r]]), f"row {r}: drew a filtered token"
        assert lp[r] == full[r, tok[r]]
