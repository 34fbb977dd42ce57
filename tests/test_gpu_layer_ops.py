"""GPU: decode-step layer operations (skinny split-K GEMM, partial
reductions, residual add + RMSNorm, SwiGLU) against fp64 / torch CPU
references of the same math.

* linear_partials: the sum of the partials equals x @ W^T up to fp32
  accumulation error, bounded elementwise by 1e-5 * (|x| @ |W|^T) (K <= 6144
  terms, fp32 epsilon 6e-8).
* splitk_reduce_bf16 / the partial sums inside add_rmsnorm and silu_mul add
  the splits in order 0, 1, ..., S-1 in fp32; the references do the same, so
  those sums are compared bit for bit.
* RMSNorm and SiLU outputs agree within one bf16 ulp (the rsqrt / exp of the
  device and of the host may differ in the last fp32 bit).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _seq_sum(P: torch.Tensor) -> torch.Tensor:
    acc = P[0].clone()
    for s in range(1, P.shape[0]):
        acc = acc + P[s]
    return acc


def _bf16_ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    return int((ai - bi).abs().max())


@pytest.mark.parametrize("M,N,K,kc", [(1, 64, 512, 256), (7, 3072, 2048, 512), (64, 2048, 6144, 512),
                                      (100, 128, 1024, 256), (64, 12288, 2048, 512), (64, 3072, 2048, 1024), (37, 2048, 6144, 1024), (100, 128, 1024, 1024),
                                      (64, 12288, 2048, 1024), (3, 6144, 4096, 1024)])
def test_linear_partials(M, N, K, kc):
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(M + N + K)
    x_full = torch.randn(M, K + 8, generator=g).to(torch.bfloat16)
    x = x_full[:, :K]
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    x_dev = x_full.to(DEV)[:, :K]  # row stride K + 8
    assert x_dev.stride(0) == K + 8
    P = ops.linear_partials(x_dev, w.to(DEV), k_chunk=kc)
    torch.cuda.synchronize()
    assert P.shape == (K // kc, M, N)
    got = P.double().sum(0).cpu()
    xd, wd = x.double(), w.double()
    ref = xd @ wd.T
    bound = 1e-5 * (xd.abs() @ wd.abs().T) + 1e-30
    assert torch.all((got - ref).abs() <= bound), float(((got - ref).abs() / bound).max())
    # each split is the product over its own k chunk
    s = K // kc - 1
    ref_s = xd[:, s * kc:(s + 1) * kc] @ wd[:, s * kc:(s + 1) * kc].T
    bound_s = 1e-5 * (xd[:, s * kc:(s + 1) * kc].abs() @ wd[:, s * kc:(s + 1) * kc].abs().T) + 1e-30
    assert torch.all((P[s].double().cpu() - ref_s).abs() <= bound_s)


@pytest.mark.parametrize("kc", [256, 512, 1024])
def test_linear_partials_packed_equals_row_major(kc):
    """The fragment-ordered weight gives the row-major kernel's partials bit
    for bit (same fragments, same MFMA sequence), and packing round-trips."""
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(kc)
    M, N, K = 45, 192, 2048
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    pw = ops.PackedWeight(w)
    assert torch.equal(pw.unpack(), w)
    a = ops.linear_partials(x, w, k_chunk=kc).clone()
    b = ops.linear_partials(x, pw, k_chunk=kc)
    assert torch.equal(a, b)


def test_splitk_reduce_bit_exact():
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(3)
    P = torch.randn(5, 33, 192, generator=g) * 10
    got = ops.splitk_reduce_bf16(P.to(DEV)).cpu()
    ref = _seq_sum(P).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("C,with_partials,S", [(2048, True, 4), (1024, False, 0), (3072, True, 8), (2048, True, 12),
                                               (2048, True, 20), (4096, True, 6), (768, True, 3), (512, False, 0),
                                               (5120, True, 10), (772, True, 2)])
def test_add_rmsnorm(C, with_partials, S):
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(C + S)
    M, eps = 37, 1e-6
    x = torch.randn(M, C, generator=g) * 3
    w = torch.rand(C, generator=g) + 0.5
    P = torch.randn(S, M, C, generator=g) if with_partials else None
    xd = x.to(DEV)
    y = ops.add_rmsnorm(xd, w.to(DEV), eps, partials=P.to(DEV) if with_partials else None).cpu()
    x_ref = x + _seq_sum(P).to(torch.bfloat16).float() if with_partials else x
    assert torch.equal(xd.cpu(), x_ref)  # the residual update is exact
    xr = x_ref.double()
    y_ref = (w.double() * (xr / torch.sqrt((xr * xr).mean(-1, keepdim=True) + eps))).float().to(torch.bfloat16)
    assert _bf16_ulps(y, y_ref) <= 1


def test_silu_mul():
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(5)
    S, M, I = 3, 19, 6144
    P = torch.randn(S, M, 2 * I, generator=g) * 2
    got = ops.silu_mul(P.to(DEV)).cpu()
    tot = _seq_sum(P)
    gate = tot[:, :I].to(torch.bfloat16)
    up = tot[:, I:].to(torch.bfloat16)
    ref = (torch.nn.functional.silu(gate.float()).to(torch.bfloat16).float() * up.float()).to(torch.bfloat16)
    assert _bf16_ulps(got, ref) <= 1


def _swiglu_ref(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(silu(bf16 g)) * bf16 u) from fp64 / fp32 sums (torch CPU)."""
    gb = g.to(torch.bfloat16)
    ub = u.to(torch.bfloat16)
    return (torch.nn.functional.silu(gb.float()).to(torch.bfloat16).float() * ub.float()).to(torch.bfloat16)


@pytest.mark.parametrize("M,I,K", [(1, 24, 2048), (7, 6144, 2048), (64, 6144, 2048), (100, 240, 2048),
                                   (130, 6144, 2048), (1, 24, 1024), (64, 4096, 1024), (70, 240, 1024),
                                   (64, 8192, 2048), (33, 16, 1024), (64, 3072, 1024), (1, 24, 768),
                                   (64, 3072, 768), (45, 240, 768)])
def test_linear_swiglu(M, I, K):
    """Gate|up + SwiGLU in one launch (whole-K fp32 sums, interleaved packed
    weight) against the fp64 sums taken through the same bf16 chain. The
    device sums g, u differ from the fp64 ones by at most 2e-5 * (|x| @ |W|^T)
    (bg, bu); with the bf16 roundings of g, u, SiLU and the product, each
    output is within |d/dg| (bg + ulp g) + |d/du| (bu + ulp u) + 2 ulp of the
    reference (d/dg = silu'(g) u, d/du = silu(g), ulp = 2^-8 relative), and
    nearly all outputs are bit-equal to it and to the split-K partials path.
    Columns past I of a strided output stay untouched."""
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(M * 7 + I + (K if K != 2048 else 0))
    x_full = torch.randn(M, K + 8, generator=g).to(torch.bfloat16)
    wg = (torch.randn(I, K, generator=g) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(I, K, generator=g) * 0.05).to(torch.bfloat16)
    x = x_full.to(DEV)[:, :K]
    pw = ops.PackedWeight(ops.interleave_gate_up(wg, wu).to(DEV))
    out_full = torch.full((M, I + 8), float("nan"), dtype=torch.bfloat16, device=DEV)
    got = ops.linear_swiglu(x, pw, out=out_full[:, :I])
    torch.cuda.synchronize()
    assert torch.isnan(out_full[:, I:].float()).all()
    got = got.cpu()
    xd = x_full[:, :K].double()
    gd, ud = xd @ wg.double().T, xd @ wu.double().T
    # fp32 MFMA accumulation over K (at most 64 k steps of 2^-24 each per half, then the
    # halves' sum) stays below 1e-5 of sum |x w|; the bound is first order in the
    # bf16 roundings that follow, so 2e-5 leaves room for a rounding boundary crossed
    bg, bu = 2e-5 * (xd.abs() @ wg.double().abs().T), 2e-5 * (xd.abs() @ wu.double().abs().T)
    ref = _swiglu_ref(gd, ud)
    sig = torch.sigmoid(gd)
    silu, dsilu = gd * sig, sig * (1 + gd * (1 - sig))
    u2 = 2.0 ** -8
    tol = (dsilu * ud).abs() * (bg + u2 * gd.abs()) + silu.abs() * (bu + u2 * ud.abs()) + 2 * u2 * (silu * ud).abs()
    err = (got.double() - ref.double()).abs()
    assert torch.all(err <= tol + 1e-30), float((err / (tol + 1e-30)).max())
    assert float((got.view(torch.int16) == ref.view(torch.int16)).float().mean()) >= 0.95
    if (2 * I) % 64 == 0:  # the same projection through split-K partials + silu_mul
        P = ops.linear_partials(x, ops.PackedWeight(torch.cat([wg, wu]).to(DEV)), k_chunk=512 if K % 512 == 0 else 256)
        old = ops.silu_mul(P).cpu()
        assert float((old.view(torch.int16) == got.view(torch.int16)).float().mean()) >= 0.95
        assert torch.all((old.double() - ref.double()).abs() <= tol + 1e-30)


def test_linear_swiglu_rejects_unsupported():
    from tinytron_amd import ops

    assert ops.swiglu_supported(2048, 6144) and ops.swiglu_supported(1024, 4096) and ops.swiglu_supported(768, 3072)
    assert not ops.swiglu_supported(3072, 6144) and not ops.swiglu_supported(4096, 6144)
    assert not ops.swiglu_supported(1536, 6144) and not ops.swiglu_supported(512, 2048)
    assert not ops.swiglu_supported(2048, 100)
    x = torch.zeros(4, 3072, dtype=torch.bfloat16, device=DEV)
    w = ops.PackedWeight(torch.zeros(48, 3072, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        ops.linear_swiglu(x, w)  # K must be 768, 1024 or 2048
    x = torch.zeros(4, 2048, dtype=torch.bfloat16, device=DEV)
    w = ops.PackedWeight(torch.zeros(16, 2048, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        ops.linear_swiglu(x, w)  # I = 8 is a multiple of neither 16 nor 24


@pytest.mark.parametrize("C,with_addend", [(2048, True), (1024, False), (4096, True), (768, True), (516, False)])
def test_add_rmsnorm_rows(C, with_addend):
    """Prefill rows: x += float(bf16 addend) exactly (strided addend rows),
    y within one bf16 ulp of the fp64 RMSNorm."""
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(C + with_addend)
    M, eps = 3001, 1e-6
    x = torch.randn(M, C, generator=g) * 3
    w = torch.rand(C, generator=g) + 0.5
    wide = (torch.randn(M, C + 64, generator=g) * 2).to(torch.bfloat16)
    a = wide[:, 32:32 + C] if with_addend else None  # row stride C + 64
    xd = x.to(DEV)
    y = ops.add_rmsnorm_rows(xd, w.to(DEV), eps, addend=wide.to(DEV)[:, 32:32 + C] if with_addend else None).cpu()
    x_ref = x + a.float() if with_addend else x
    assert torch.equal(xd.cpu(), x_ref)  # the residual update is exact
    xr = x_ref.double()
    y_ref = (w.double() * (xr / torch.sqrt((xr * xr).mean(-1, keepdim=True) + eps))).float().to(torch.bfloat16)
    assert _bf16_ulps(y, y_ref) <= 1


def test_silu_mul_rows():
    """Prefill rows: bf16(bf16(silu(g)) * u) from bf16 gate / up outputs (a
    stacked gate|up buffer's two column halves), within one bf16 ulp of torch."""
    from tinytron_amd import ops

    g = torch.Generator().manual_seed(6)
    M, I = 1003, 6144
    gu = (torch.randn(M, 2 * I, generator=g) * 2).to(torch.bfloat16)
    gud = gu.to(DEV)
    got = ops.silu_mul_rows(gud[:, :I], gud[:, I:]).cpu()
    ref = (torch.nn.functional.silu(gu[:, :I].float()).to(torch.bfloat16).float() * gu[:, I:].float()).to(torch.bfloat16)
    assert _bf16_ulps(got, ref) <= 1
    sep = ops.silu_mul_rows(gud[:, :I].contiguous(), gud[:, I:].contiguous()).cpu()
    assert torch.equal(sep, got)


def test_layer_ops_reject_bad_shapes():
    from tinytron_amd import ops

    x = torch.zeros(4, 100, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 100, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.linear_partials(x, w, k_chunk=256)  # K not a multiple of the chunk
    with pytest.raises(ValueError):  # hidden size not a multiple of 4
        ops.add_rmsnorm(torch.zeros(2, 1002, device=DEV), torch.ones(1002, device=DEV), 1e-6)
    with pytest.raises(ValueError):  # hidden size past 8192
        ops.add_rmsnorm(torch.zeros(2, 8196, device=DEV), torch.ones(8196, device=DEV), 1e-6)
