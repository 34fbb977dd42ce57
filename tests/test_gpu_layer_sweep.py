"""GPU: a seeded sweep of decode-step layer-operation shapes against fp64 /
torch references, beyond the hand-picked cases of test_gpu_layer_ops.py:
split-K GEMM partials (row counts across several 64-row tiles, widths on
and off the 128-column tile, every k_chunk, row-major and fragment-ordered
weights), residual add + RMSNorm over split-K partials (1-20 splits) and over
bf16 rows (strided), SwiGLU from partials and from bf16 rows. Same bounds as
test_gpu_layer_ops.py.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_layer_ops import _bf16_ulps, _seq_sum

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("i", range(20))
def test_linear_partials_sweep(i):
    from tinytron_amd import ops

    rng = np.random.default_rng(3000 + i)
    M = int(rng.choice([1, 3, 64, 65, 130, 200]))
    N = 64 * int(rng.integers(1, 49))
    kc = int(rng.choice([256, 512, 1024]))
    K = kc * int(rng.integers(1, 7))
    packed = bool(rng.integers(0, 2))
    print(f"sweep case {i}: M {M} N {N} K {K} kc {kc} packed {packed}", flush=True)
    g = torch.Generator().manual_seed(i)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    wd = w.to(DEV)
    P = ops.linear_partials(x.to(DEV), ops.PackedWeight(wd) if packed else wd, k_chunk=kc)
    got = P.double().sum(0).cpu()
    xd, wdd = x.double(), w.double()
    ref = xd @ wdd.T
    bound = 1e-5 * (xd.abs() @ wdd.abs().T) + 1e-30
    assert torch.all((got - ref).abs() <= bound), float(((got - ref).abs() / bound).max())


@pytest.mark.parametrize("i", range(12))
def test_add_rmsnorm_sweep(i):
    from tinytron_amd import ops

    rng = np.random.default_rng(3100 + i)
    C = 1024 * int(rng.integers(1, 9))
    M = int(rng.choice([1, 7, 64, 300]))
    S = int(rng.integers(0, 21))
    rows = bool(rng.integers(0, 2))
    print(f"sweep case {i}: C {C} M {M} S {S} rows {rows}", flush=True)
    g = torch.Generator().manual_seed(100 + i)
    eps = 1e-6
    x = torch.randn(M, C, generator=g) * 2
    w = torch.rand(C, generator=g) + 0.5
    xd = x.to(DEV)
    if rows:  # bf16 addend rows with a wider row stride
        wide = (torch.randn(M, C + 32, generator=g)).to(torch.bfloat16)
        a = wide[:, 16:16 + C]
        y = ops.add_rmsnorm_rows(xd, w.to(DEV), eps, addend=wide.to(DEV)[:, 16:16 + C]).cpu()
        x_ref = x + a.float()
    else:
        P = torch.randn(S, M, C, generator=g) if S else None
        y = ops.add_rmsnorm(xd, w.to(DEV), eps, partials=P.to(DEV) if S else None).cpu()
        x_ref = x + _seq_sum(P).to(torch.bfloat16).float() if S else x
    assert torch.equal(xd.cpu(), x_ref)
    xr = x_ref.double()
    y_ref = (w.double() * (xr / torch.sqrt((xr * xr).mean(-1, keepdim=True) + eps))).float().to(torch.bfloat16)
    assert _bf16_ulps(y, y_ref) <= 1


@pytest.mark.parametrize("i", range(10))
def test_silu_mul_sweep(i):
    from tinytron_amd import ops

    rng = np.random.default_rng(3200 + i)
    I = 4 * int(rng.integers(1, 2049))
    M = int(rng.choice([1, 5, 64, 257]))
    S = int(rng.integers(1, 13))
    rows = bool(rng.integers(0, 2))
    print(f"sweep case {i}: I {I} M {M} S {S} rows {rows}", flush=True)
    g = torch.Generator().manual_seed(200 + i)
    if rows:
        gu = (torch.randn(M, 2 * I, generator=g) * 2).to(torch.bfloat16)
        gud = gu.to(DEV)
        got = ops.silu_mul_rows(gud[:, :I], gud[:, I:]).cpu()
        gate, up = gu[:, :I], gu[:, I:]
    else:
        P = torch.randn(S, M, 2 * I, generator=g) * 2
        got = ops.silu_mul(P.to(DEV)).cpu()
        tot = _seq_sum(P)
        gate, up = tot[:, :I].to(torch.bfloat16), tot[:, I:].to(torch.bfloat16)
    ref = (torch.nn.functional.silu(gate.float()).to(torch.bfloat16).float() * up.float()).to(torch.bfloat16)
    assert _bf16_ulps(got, ref) <= 1
