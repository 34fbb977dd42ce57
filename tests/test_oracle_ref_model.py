"""Pins oracle/ref_model.py (the reference's block composition, gpt.py:33-115,
norm.py:14-19, mlp.py:44-45, attn.py:378-440) without the GPU model:

* closed forms in fp64 numpy: with every projection zero the logits are the
  tied head over the final norm of the embedding (residual passthrough,
  lnf, tied lm_head); with q = k = 0 the attention is the causal mean of V
  per KV head h // G (mask, GQA map, c_proj, residual order); RMSNorm of a
  constant row is weight * sign / sqrt(1 + eps / c^2);
* an invariant: prefill of T tokens equals prefill of T - 3 plus three
  one-token cached steps (cache append, position offsets, decode mask);
* the bf16 mode against the fp32 code run under torch.autocast on the CPU
  (torch's own autocast policy sets the rounding points), with a planted
  mistake (SiLU * up kept in fp32) that the comparison catches.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle.ref_model import RefGPT


def _state(L, C, hq, hkv, ffn, vocab, std=0.2, seed=0):
    g = torch.Generator().manual_seed(seed)
    D = C // hq
    sd = {"wte.weight": torch.randn(vocab, C, generator=g), "lnf.weight": 1 + 0.3 * torch.randn(C, generator=g)}
    for i in range(L):
        p = f"blocks.{i}."
        sd[p + "ln_1.weight"] = 1 + 0.3 * torch.randn(C, generator=g)
        sd[p + "ln_2.weight"] = 1 + 0.3 * torch.randn(C, generator=g)
        for name, shape in (("attn.q_proj", (hq * D, C)), ("attn.k_proj", (hkv * D, C)), ("attn.v_proj", (hkv * D, C)),
                            ("attn.c_proj", (C, C)), ("mlp.gate_proj", (ffn, C)), ("mlp.up_proj", (ffn, C)),
                            ("mlp.down_proj", (C, ffn))):
            sd[p + name + ".weight"] = std * torch.randn(*shape, generator=g)
    return sd


def _np_rms(x, w):
    return w * x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)


def _run(ref, idx):
    caches = ref.new_caches(idx.shape[0], idx.shape[1] + 8, page_size=4)
    with torch.no_grad():
        return ref.forward(idx, caches, 0)


def test_zero_projections_give_tied_head_over_final_norm():
    L, C, hq, hkv, ffn, V = 2, 32, 4, 2, 48, 40
    sd = _state(L, C, hq, hkv, ffn, V)
    for k in sd:
        if k.endswith("_proj.weight"):
            sd[k] = torch.zeros_like(sd[k])
    idx = torch.tensor([[3, 17, 0, 39, 3]])
    got = _run(RefGPT(sd, L, hq, hkv), idx)[0].double().numpy()
    e = sd["wte.weight"].double().numpy()[idx[0].numpy()]
    want = _np_rms(e, sd["lnf.weight"].double().numpy()) @ sd["wte.weight"].double().numpy().T
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_uniform_attention_is_causal_mean_of_v_per_kv_head():
    """q = k = 0: every score is 0, so head h at position t averages v_s of KV
    head h // G over s <= t; the MLP's down projection is zero."""
    L, C, hq, hkv, ffn, V = 1, 48, 6, 2, 32, 30
    D, G = C // hq, hq // hkv
    sd = _state(L, C, hq, hkv, ffn, V, seed=3)
    for k in ("blocks.0.attn.q_proj.weight", "blocks.0.attn.k_proj.weight", "blocks.0.mlp.down_proj.weight"):
        sd[k] = torch.zeros_like(sd[k])
    idx = torch.tensor([[5, 2, 29, 2, 11, 7]])
    got = _run(RefGPT(sd, L, hq, hkv), idx)[0].double().numpy()

    f = {k: v.double().numpy() for k, v in sd.items()}
    e = f["wte.weight"][idx[0].numpy()]                              # [T, C]
    n = _np_rms(e, f["blocks.0.ln_1.weight"])
    v = (n @ f["blocks.0.attn.v_proj.weight"].T).reshape(-1, hkv, D)  # [T, Hkv, D]
    T = e.shape[0]
    y = np.zeros((T, hq, D))
    for t in range(T):
        for h in range(hq):
            y[t, h] = v[:t + 1, h // G].mean(0)
    x = e + y.reshape(T, C) @ f["blocks.0.attn.c_proj.weight"].T
    want = _np_rms(x, f["lnf.weight"]) @ f["wte.weight"].T
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)

    # the other head map (h % H_kv) gives different logits: the check above is sensitive to it
    y2 = np.stack([np.stack([v[:t + 1, h % hkv].mean(0) for h in range(hq)]) for t in range(T)])
    x2 = e + y2.reshape(T, C) @ f["blocks.0.attn.c_proj.weight"].T
    assert np.abs(_np_rms(x2, f["lnf.weight"]) @ f["wte.weight"].T - want).max() > 1e-2


@pytest.mark.parametrize("c", [1e-3, 0.5, -2.0, 300.0])
def test_rmsnorm_of_constant_row(c):
    w = torch.linspace(-1, 2, 16)
    got = RefGPT._rms(torch.full((1, 16), c), w)[0].double().numpy()
    want = w.double().numpy() * np.sign(c) / np.sqrt(1 + 1e-6 / (c * c))
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)


def test_rmsnorm_is_scale_invariant():
    x = torch.randn(3, 64, generator=torch.Generator().manual_seed(1))
    w = torch.rand(64) + 0.5
    np.testing.assert_allclose(RefGPT._rms(x * 37.0, w).numpy(), RefGPT._rms(x, w).numpy(), rtol=1e-5, atol=1e-6)


def test_cached_steps_equal_full_prefill():
    L, C, hq, hkv, ffn, V = 2, 64, 4, 2, 96, 50
    ref = RefGPT(_state(L, C, hq, hkv, ffn, V, std=0.1, seed=5), L, hq, hkv)
    idx = torch.randint(0, V, (2, 12), generator=torch.Generator().manual_seed(2))
    full = _run(ref, idx)
    caches = ref.new_caches(2, 20, page_size=4)
    with torch.no_grad():
        ref.forward(idx[:, :9], caches, 0)
        for t in range(9, 12):
            step = ref.forward(idx[:, t:t + 1], caches, t)
            torch.testing.assert_close(step[:, 0], full[:, t], rtol=1e-5, atol=1e-5)


def test_tuple_cache_path_equals_paged_cache_path():
    """use_paged_kv_cache=False (past K/V concatenated each step) gives the
    paged cache's greedy tokens and logits."""
    L, C, hq, hkv, ffn, V = 2, 64, 4, 2, 96, 50
    ref = RefGPT(_state(L, C, hq, hkv, ffn, V, std=0.1, seed=6), L, hq, hkv)
    idx = torch.randint(0, V, (2, 10), generator=torch.Generator().manual_seed(3))
    t0, _, l0 = ref.generate_greedy(idx, 6, 32, page_size=4)
    t1, _, l1 = ref.generate_greedy(idx, 6, 32, tuple_cache=True)
    assert torch.equal(t0, t1)
    for a, b in zip(l0, l1):
        torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


class _UnroundedSwiGLU(RefGPT):
    """A planted mistake: SiLU(gate) * up computed from fp32 copies, so the
    product skips its bf16 rounding."""

    def forward(self, idx, caches, position_offset):
        import torch.nn.functional as F

        orig_silu = F.silu
        F.silu = lambda t: orig_silu(t.float())
        try:
            return super().forward(idx, caches, position_offset)
        finally:
            F.silu = orig_silu


def _sdpa_fp32_to_bf16(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False):
    """SDPA over the bf16 inputs in fp32, output rounded to bf16: the
    autocast op's input and output rounding, without the internal rounding a
    particular bf16 kernel adds (torch's CPU kernel rounds P; attention is a
    toleranced op in the parity contract, so its internals are not pinned here)."""
    with torch.autocast("cpu", enabled=False):
        y = _SDPA(q.to(torch.bfloat16).float(), k.to(torch.bfloat16).float(), v.to(torch.bfloat16).float(),
                  attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal)
    return y.to(torch.bfloat16)


_SDPA = torch.nn.functional.scaled_dot_product_attention


def _bf16_vs_autocast(cls, monkeypatch):
    L, C, hq, hkv, ffn, V = 2, 256, 4, 2, 512, 1000
    sd = _state(L, C, hq, hkv, ffn, V, std=0.02, seed=9)
    sd["wte.weight"] *= 0.1  # init_std-sized embedding, as the models are initialised
    idx = torch.randint(0, V, (2, 24), generator=torch.Generator().manual_seed(4))
    got = _run(cls(sd, L, hq, hkv, autocast_bf16=True), idx).float()
    exact = _run(RefGPT(sd, L, hq, hkv), idx).float()
    with monkeypatch.context() as m:
        m.setattr(torch.nn.functional, "scaled_dot_product_attention", _sdpa_fp32_to_bf16)
        with torch.autocast("cpu", dtype=torch.bfloat16):
            auto = _run(RefGPT(sd, L, hq, hkv), idx).float()
    return got, auto, exact


def test_bf16_mode_follows_torch_autocast(monkeypatch):
    got, auto, exact = _bf16_vs_autocast(RefGPT, monkeypatch)
    assert got.dtype == auto.dtype
    scale = exact.abs().max()
    d_auto = (got - auto).abs()
    d_exact = (got - exact).abs()
    # same rounding points: the two bf16 runs differ only where an fp32 summation
    # order flips a bf16 rounding (rare), far less than bf16 differs from fp32
    # (measured: 99.998 % of logits identical, largest difference 1e-6 of a 25.6 scale)
    assert d_auto.max() <= 2 ** -12 * scale
    assert d_auto.mean() <= 1e-4 * d_exact.mean()
    assert (d_auto == 0).float().mean() >= 0.999


def test_bf16_mode_catches_a_missing_rounding_point(monkeypatch):
    good, auto, exact = _bf16_vs_autocast(RefGPT, monkeypatch)
    bad, _, _ = _bf16_vs_autocast(_UnroundedSwiGLU, monkeypatch)
    # one missing rounding point moves the logits by a sizeable share of the bf16-vs-fp32 gap
    assert (bad - auto).abs().mean() > 0.1 * (good - exact).abs().mean()
    assert (bad - auto).abs().mean() > 1e3 * (good - auto).abs().mean()
