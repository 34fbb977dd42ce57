"""GPU: the bf16 model (module path and fused decode step) against the
reference's op sequence under bf16 autocast, restated on the CPU
(oracle.ref_model with autocast_bf16=True, whose rounding points are pinned
to torch's own CPU autocast in tests/test_oracle_ref_model.py).

* Every op in isolation (C1's model, module path): each op of every layer is
  fed the GPU's own inputs on the CPU and its output compared with the GPU's.
  With the same rounding points the outputs are bit-identical except where
  an fp32 summation order flips one bf16 rounding (a few in 10^4); a missing
  or extra rounding point would make most outputs differ.
* One layer, fused kernels (packed prefill, fused decode step): with one
  layer, flips have no room to compound, so the logits agree almost bit for
  bit.
* Several layers end to end: each flip perturbs every later value slightly
  and flips a few more, so after several layers the GPU is as far from the
  bf16 oracle as bf16 rounding itself is from fp32 (the bf16-fp32 "gap").
  The bound is stated against that gap, and greedy tokens must equal the
  oracle's argmax except at a near-tie (top-2 margin within the GPU-oracle
  noise).
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16

# several layers: |GPU - bf16 oracle| <= RATIO * |bf16 oracle - fp32 oracle| (mean and max over all logits)
RATIO = 1.5


def _config(**kw):
    from tinytron_amd.model import ModelConfig

    base = dict(num_layer=6, hidden_size=512, num_attention_heads=8, num_key_value_heads=2, vocab_size=32000,
                intermediate_size=2048, init_std=0.02, block_size=256, tied_lm_head=True)
    base.update(kw)
    return ModelConfig(**base)


def _oracles(model, cfg):
    from oracle.ref_model import RefGPT

    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    args = (sd, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads)
    return RefGPT(*args, autocast_bf16=True), RefGPT(*args)


def _oracle_steps(ref, prompt, forced, block):
    """Logits [steps + 1, V] of one sequence: the prompt's last position, then
    one cached step per forced token."""
    caches = ref.new_caches(1, block, page_size=16)
    out = []
    with torch.no_grad():
        out.append(ref.forward(prompt[None], caches, 0)[0, -1].float())
        for i, t in enumerate(forced):
            out.append(ref.forward(torch.tensor([[int(t)]]), caches, prompt.numel() + i)[0, -1].float())
    return torch.stack(out)


def compare_to_oracles(gpu, ob, of, what, ratio=RATIO):
    """gpu, ob (bf16 oracle), of (fp32 oracle): logits [steps, V]. Returns the
    largest |gpu - ob| (the noise level for near-tie decisions)."""
    d, gap, d32 = (gpu - ob).abs(), (ob - of).abs(), (gpu - of).abs()
    mean_r, max_r = float(d.mean() / gap.mean()), float(d.max() / gap.max())
    print(f"{what}: |gpu - bf16 oracle| mean {float(d.mean()):.3e} ({mean_r:.2f} x the bf16-fp32 gap), max "
          f"{float(d.max()):.3e} ({max_r:.2f} x); |gpu - fp32 oracle| mean {float(d32.mean()):.3e}; identical "
          f"{float((d == 0).float().mean()):.3f}", flush=True)
    assert mean_r <= ratio and max_r <= ratio, what
    # as far from fp32 as bf16 rounding is (an extra rounding point would add to it)
    assert float(d32.mean()) <= RATIO * float(gap.mean()), what
    return float(d.max())


def greedy_agrees(tokens, ob_logits, noise, what):
    """GPU greedy tokens vs the bf16 oracle's argmax row by row (teacher-forced on
    the GPU's tokens): a different token must be a near-tie in the oracle's
    row, within twice the GPU-oracle noise of the logits."""
    for s, t in enumerate(tokens):
        row = ob_logits[s]
        best = int(row.argmax())
        if int(t) != best:
            gap = float(row[best] - row[int(t)])
            assert gap <= 2 * noise, f"{what}: step {s} token {int(t)} vs oracle {best}, logit gap {gap:.3e}"


def _lin(x, w):
    import torch.nn.functional as F

    return F.linear(x.to(BF16).float(), w.to(BF16).float()).to(BF16)


def _rms(x, w):
    x32 = x.float()
    return w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + 1e-6))


def test_c1_bf16_each_op_matches_reference_autocast():
    """C1's model (6 L, d 512, 8/2 heads, V 32000) in bf16, prompt of 128
    tokens through the module path; every op checked with the GPU's inputs."""
    import torch.nn.functional as F

    from oracle import ref_path
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import GPT

    cfg = _config()
    model = GPT(cfg, device=DEV, dtype=BF16)
    cap, hooks = {}, []

    def hook(name):
        def f(mod, inp, out):
            cap[name] = (inp[0].detach().cpu(), (out[0] if isinstance(out, tuple) else out).detach().cpu())
        return f

    for i, blk in enumerate(model.blocks):
        for n in ("q_proj", "k_proj", "v_proj", "c_proj"):
            hooks.append(getattr(blk.attn, n).register_forward_hook(hook(f"{i}.{n}")))
        for n in ("gate_proj", "up_proj", "down_proj"):
            hooks.append(getattr(blk.mlp, n).register_forward_hook(hook(f"{i}.{n}")))
        for n in ("ln_1", "ln_2"):
            hooks.append(getattr(blk, n).register_forward_hook(hook(f"{i}.{n}")))
        hooks.append(blk.register_forward_hook(hook(f"{i}.block")))
    hooks.append(model.lnf.register_forward_hook(hook("lnf")))
    T = 128
    prompt = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(1337))
    cache = PagedKVCache.from_model_config(cfg, 1, 128, DEV, BF16)
    with torch.no_grad():
        logits, _ = model(prompt.to(DEV), use_cache=True, past_key_values=cache, position_offset=0)
    for h in hooks:
        h.remove()
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.hidden_size // cfg.num_attention_heads

    def same(name, got, want, min_identical, rel=0.0):
        got, want = got.float(), want.float()
        d = (got - want).abs()
        ident = float((d == 0).float().mean())
        worst = float(d.max() / want.abs().max())
        assert ident >= min_identical and worst <= max(rel, 2.0 ** -7), f"{name}: identical {ident:.5f}, max rel {worst:.2e}"

    for i in range(cfg.num_layer):
        p = f"blocks.{i}."
        x = cap[f"{i}.ln_1"][0]
        # RMSNorm is fp32 (its output rounds to bf16 only inside the next projection)
        torch.testing.assert_close(cap[f"{i}.ln_1"][1], _rms(x, sd[p + "ln_1.weight"]), rtol=1e-6, atol=1e-7)
        for n in ("q_proj", "k_proj", "v_proj"):
            assert cap[f"{i}.{n}"][1].dtype == BF16
            same(f"{i}.{n}", cap[f"{i}.{n}"][1], _lin(cap[f"{i}.{n}"][0], sd[p + f"attn.{n}.weight"]), 0.999)
        q = cap[f"{i}.q_proj"][1].view(1, T, H, D).transpose(1, 2)
        k = cap[f"{i}.k_proj"][1].view(1, T, Hkv, D).transpose(1, 2)
        v = cap[f"{i}.v_proj"][1].view(1, T, Hkv, D).transpose(1, 2)
        qr, kr = ref_path.rope_impl(q, k, torch.arange(T)[None])
        kr, vr = ref_path.gqa_impl(kr, v, Hkv, H)
        y = F.scaled_dot_product_attention(qr.float(), kr.float(), vr.float(), is_causal=True).to(BF16)
        same(f"{i} attention", cap[f"{i}.c_proj"][0], y.transpose(1, 2).reshape(1, T, H * D), 0.995)
        same(f"{i}.c_proj", cap[f"{i}.c_proj"][1], _lin(cap[f"{i}.c_proj"][0], sd[p + "attn.c_proj.weight"]), 0.999)
        mid = cap[f"{i}.ln_2"][0]
        assert mid.dtype == torch.float32 and torch.equal(mid, x + cap[f"{i}.c_proj"][1].float())  # fp32 residual
        torch.testing.assert_close(cap[f"{i}.ln_2"][1], _rms(mid, sd[p + "ln_2.weight"]), rtol=1e-6, atol=1e-7)
        for n in ("gate_proj", "up_proj"):
            same(f"{i}.{n}", cap[f"{i}.{n}"][1], _lin(cap[f"{i}.{n}"][0], sd[p + f"mlp.{n}.weight"]), 0.999)
        swiglu = F.silu(cap[f"{i}.gate_proj"][1]) * cap[f"{i}.up_proj"][1]   # bf16 SiLU, bf16 product
        same(f"{i} silu*up", cap[f"{i}.down_proj"][0], swiglu, 0.9999)
        same(f"{i}.down_proj", cap[f"{i}.down_proj"][1], _lin(cap[f"{i}.down_proj"][0], sd[p + "mlp.down_proj.weight"]),
             0.999)
        assert torch.equal(cap[f"{i}.block"][1], mid + cap[f"{i}.down_proj"][1].float())
    torch.testing.assert_close(cap["lnf"][1], _rms(cap["lnf"][0], sd["lnf.weight"]), rtol=1e-6, atol=1e-7)
    same("lm_head", logits.cpu(), _lin(cap["lnf"][1], sd["wte.weight"]), 0.999)


def _run_gpu(model, cfg, prompt, lens, steps, paged):
    """Prefill (ragged, logits at each prompt's end) then greedy steps; returns
    logits [B, steps + 1, V] and the greedy tokens [B, steps]."""
    from tinytron_amd.cache import PagedKVCache

    B = len(lens)
    cache = PagedKVCache.from_model_config(cfg, B, 16 if paged else 128, DEV, BF16, paged_pool=paged,
                                           seq_capacity=[n + steps + 1 for n in lens])
    logits, toks = [], []
    with torch.no_grad():
        cache.set_pending_new_lens(lens)
        out, _ = model(prompt.to(DEV), use_cache=True, past_key_values=cache, position_offset=0,
                       logits_index=torch.tensor(lens, device=DEV) - 1)
        cache.set_pending_new_lens(None)
        row = out[:, -1].float()
        for s in range(steps):
            logits.append(row.cpu())
            t = row.argmax(-1)
            toks.append(t.cpu())
            pos = lens[0] + s if len(set(lens)) == 1 else 0  # checked against the cache only when uniform
            out, _ = model(t.view(B, 1), use_cache=True, past_key_values=cache, position_offset=pos)
            row = out[:, -1].float()
        logits.append(row.cpu())
    return torch.stack(logits, 1), torch.stack(toks, 1)


@pytest.mark.parametrize("shape", ["d1024", "preset_0.1b", "preset_0.25b", "preset_13b"])
def test_one_layer_fused_path_matches_reference_autocast(shape):
    """One layer through the packed prefill and the fused decode step
    (split-K GEMMs, RoPE + append with the attention, fused add + RMSNorm,
    SwiGLU) against the oracle, per sequence of a ragged batch, at d 1024
    (16/4 heads, D 64) and at the reference presets' layer shapes
    (scripts/debug/inference.sh:71-77, 52-57, 101-107): 0.1B d 768 (16/4
    heads, D 48, ffn 3072: gate|up + SwiGLU in one K = 768 launch), 0.25B
    d 1024 (32/4 heads, D 32, ffn 4096: one K = 1024 launch), 13B d 5120
    (40/8 heads: G 5, D 128, ffn 13824: split-K gate|up and silu_mul). The
    fused decode step runs every step (asserted), with the one-launch SwiGLU
    wherever the kernel takes the shape (asserted)."""
    from tinytron_amd.model import GPT

    dims = {"d1024": (1024, 16, 4, 2048), "preset_0.1b": (768, 16, 4, 3072), "preset_0.25b": (1024, 32, 4, 4096),
            "preset_13b": (5120, 40, 8, 13824)}[shape]
    cfg = _config(num_layer=1, hidden_size=dims[0], num_attention_heads=dims[1], num_key_value_heads=dims[2],
                  intermediate_size=dims[3], vocab_size=8192, block_size=256)
    model = GPT(cfg, device=DEV, dtype=BF16)
    assert model._swiglu_fused() == (shape != "preset_13b")
    calls = []
    fused = model._decode_step_fused
    model._decode_step_fused = lambda *a, **k: (calls.append(1), fused(*a, **k))[1]
    ob, of = _oracles(model, cfg)
    lens, steps = [70, 9, 33], 8
    prompt = torch.randint(0, cfg.vocab_size, (len(lens), max(lens)), generator=torch.Generator().manual_seed(31))
    gpu, toks = _run_gpu(model, cfg, prompt, lens, steps, paged=True)
    assert len(calls) == steps, f"fused decode step ran {len(calls)} of {steps} steps"
    for b, n in enumerate(lens):
        lb = _oracle_steps(ob, prompt[b, :n], toks[b].tolist(), 128)
        lf = _oracle_steps(of, prompt[b, :n], toks[b].tolist(), 128)
        noise = compare_to_oracles(gpu[b], lb, lf, f"1-layer fused, sequence {b}", ratio=1.0)
        # One flip upstream (a residual element one bf16 ulp off) moves the final
        # RMSNorm's scale and the lm_head input, and so every logit by a small
        # amount, which flips many logits' own bf16 rounding at once: every logit
        # stays within two bf16 ulps of its row's largest logit (measured: one).
        top = torch.maximum(gpu[b].abs(), lb.abs()).amax(-1, keepdim=True)
        ulp = torch.ldexp(torch.ones(()), torch.frexp(top)[1] - 8)
        worst = float(((gpu[b] - lb).abs() / ulp).max())
        assert worst <= 2.0, f"sequence {b}: a logit is {worst:.2f} bf16 ulps (of its row's largest) from the oracle"
        greedy_agrees(toks[b].tolist(), lb, noise, f"1-layer fused, sequence {b}")


@pytest.mark.parametrize("name", ["c1_module", "d1024_fused", "d2048_fused", "default_0.25b"])
def test_several_layers_match_reference_autocast(name):
    """C1's model through the module path (contiguous cache, prompt 128, 64
    greedy steps), a 4-layer d 1024 model through the packed prefill and the
    fused decode step (paged pool, ragged batch, 12 steps), a 2-layer
    model of C5's width (d 2048, ffn 6144: gate|up + SwiGLU as one whole-K
    launch) the same way, and the reference's default 0.25B model
    (scripts/debug/inference.sh:52-57: 12 layers, d 1024, 32 / 4 heads, so
    head_dim 32, ffn 4096) through the same fused paths."""
    from tinytron_amd.model import GPT

    if name == "c1_module":
        cfg = _config()
        lens, steps, paged, seed = [128], 64, False, 1337
    elif name == "default_0.25b":
        cfg = _config(num_layer=12, hidden_size=1024, num_attention_heads=32, num_key_value_heads=4,
                      intermediate_size=4096, vocab_size=32000, block_size=256)
        lens, steps, paged, seed = [70, 9, 33], 8, True, 53
    elif name == "d2048_fused":
        cfg = _config(num_layer=2, hidden_size=2048, num_attention_heads=32, num_key_value_heads=8,
                      intermediate_size=6144, vocab_size=8192, block_size=256)
        lens, steps, paged, seed = [70, 9, 33], 8, True, 41
    else:
        cfg = _config(num_layer=4, hidden_size=1024, num_attention_heads=16, num_key_value_heads=4,
                      intermediate_size=2048, vocab_size=8192, block_size=256)
        lens, steps, paged, seed = [70, 9, 33], 12, True, 29
    model = GPT(cfg, device=DEV, dtype=BF16)
    ob, of = _oracles(model, cfg)
    prompt = torch.randint(0, cfg.vocab_size, (len(lens), max(lens)), generator=torch.Generator().manual_seed(seed))
    gpu, toks = _run_gpu(model, cfg, prompt, lens, steps, paged)
    for b, n in enumerate(lens):
        lb = _oracle_steps(ob, prompt[b, :n], toks[b].tolist(), 256)
        lf = _oracle_steps(of, prompt[b, :n], toks[b].tolist(), 256)
        noise = compare_to_oracles(gpu[b], lb, lf, f"{name}, sequence {b}")
        greedy_agrees(toks[b].tolist(), lb, noise, f"{name}, sequence {b}")
