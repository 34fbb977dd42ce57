"""GPU: config C5 run as a workload (the 1.3B-class dense GQA model of the
end-to-end benchmark: 24 layers, d 2048, 32/8 heads, D 64, ffn 6144, V 32000,
bf16 random-init weights; batch 64 with prompts U[64, 2048] drawn from seed
1337 exactly as bench.py draws them; paged pool, page size 16).

* Ragged batch == batch 1: four sequences of the 64 (the shortest, the
  longest, two seeded others) generate the same greedy tokens alone as in
  the batch until a near-tie: where the runs first differ, the two tokens'
  logits (one batch-1 pass over the shared prefix) are within the bf16 noise
  of the 24-layer step (bf16 GEMMs of different batch shapes round
  differently, and the difference compounds over the layers).
* Fused decode step == module path: teacher-forced steps from identical
  caches; logits within a bf16 bound, greedy tokens equal barring near-ties.
* fp8-e4m3 KV cache vs bf16 KV cache: the logits of the first decode steps
  within a stated bound, and top-1 agreement.
* The shortest sequence's logits (prefill and decode steps) against the
  reference's op sequence under bf16 autocast restated on the CPU
  (oracle.ref_model), within the bound of tests/test_gpu_model_bf16.py.
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"
SEED = 1337
B, LO, HI, V, P = 64, 64, 2048, 32000, 16
# Two bf16 implementations of the 24-layer step (different GEMM shapes or
# kernels) differ by up to ~5e-2 per logit (measured: fused vs module path,
# max 5.5e-2 at a logit scale of 4.9); two tokens closer than this are a tie.
NEAR_TIE = 0.1


def _inputs():
    g = torch.Generator().manual_seed(SEED)
    lens = torch.randint(LO, HI + 1, (B,), generator=g).tolist()
    prompt = torch.randint(0, V, (B, max(lens)), generator=g)
    return lens, prompt


@pytest.fixture(scope="module")
def c5():
    from tinytron_amd.model import GPT, ModelConfig

    lens, prompt = _inputs()
    cfg = ModelConfig(num_layer=24, hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, vocab_size=V,
                      intermediate_size=6144, init_std=0.02, block_size=max(lens) + 32, seed=SEED)
    print(f"\nC5 model: 24 layers, d 2048, B {B}, prompts {min(lens)}..{max(lens)}", flush=True)
    model = GPT(cfg, device=DEV, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    return cfg, model, lens, prompt


def _prefill(model, cfg, lens, prompt, steps, kv_dtype=None):
    from tinytron_amd.cache import PagedKVCache

    n = len(lens)
    cache = PagedKVCache.from_model_config(cfg, n, P, DEV, torch.bfloat16, kv_cache_dtype=kv_dtype, paged_pool=True,
                                           seq_capacity=[x + steps + 1 for x in lens])
    cache.set_pending_new_lens(lens)
    out, _ = model(prompt[:, :max(lens)].to(DEV), use_cache=True, past_key_values=cache, position_offset=0,
                   logits_index=torch.tensor(lens, device=DEV) - 1)
    cache.set_pending_new_lens(None)
    return cache, out[:, -1].float()


def _forced_steps(model, cache, first, tokens):
    """Logits [steps + 1, n, V]: `first`, then one step per column of tokens [n, steps]."""
    rows = [first]
    for s in range(tokens.shape[1]):
        out, _ = model(tokens[:, s:s + 1].to(DEV), use_cache=True, past_key_values=cache, position_offset=0)
        rows.append(out[:, -1].float())
    return torch.stack(rows)


@torch.no_grad()
def test_c5_ragged_batch_equals_batch_one(c5):
    from tinytron_amd.engine import InferenceEngine

    cfg, model, lens, prompt = c5
    steps = 16
    eng = InferenceEngine(cfg, device=DEV, dtype=torch.bfloat16, kv_cache_page_size=P, paged_pool=True, model=model)
    batch, stats = eng.generate(prompt, steps, top_k=1, prompt_lens=lens, return_stats=True)
    assert stats["lengths"] == [n + steps for n in lens]
    order = sorted(range(B), key=lambda b: lens[b])
    g = torch.Generator().manual_seed(SEED + 1)
    picks = [order[0], order[-1]] + [int(i) for i in torch.randperm(B, generator=g)[:2]]
    for b in picks:
        n = lens[b]
        single = eng.generate(prompt[b:b + 1, :n], steps, top_k=1)
        got, alone = batch[b, :n + steps].cpu(), single[0, :n + steps].cpu()
        assert torch.equal(got[:n], prompt[b, :n])
        diff = (got != alone).nonzero()
        if len(diff) == 0:
            print(f"sequence {b} (prompt {n}): batch == batch-1 for all {steps} steps", flush=True)
            continue
        # first divergence: both runs share the prefix, so one batch-1 pass over it gives the
        # logits both chose from; the two tokens must be a near-tie there
        s = int(diff[0])
        cache, first = _prefill(model, cfg, [s], got[None, :s], 0)
        row = first[0].cpu()
        tie = float((row[int(got[s])] - row[int(alone[s])]).abs())
        print(f"sequence {b} (prompt {n}): diverges at step {s - n}, logit gap of the two tokens {tie:.3e}",
              flush=True)
        assert tie <= NEAR_TIE, f"sequence {b}: tokens {int(got[s])} / {int(alone[s])} are not a near-tie"
        del cache


@torch.no_grad()
def test_c5_fused_step_matches_module_path(c5):
    cfg, model, lens, prompt = c5
    steps = 4
    g = torch.Generator().manual_seed(SEED + 2)
    forced = torch.randint(0, V, (B, steps), generator=g)
    runs = []
    for fused in (True, False):
        model.fused_decode = fused
        cache, first = _prefill(model, cfg, lens, prompt, steps)
        runs.append(_forced_steps(model, cache, first, forced).cpu())
        del cache
    model.fused_decode = True
    a, b = runs
    assert torch.equal(a[0], b[0])  # same prefill
    d = (a[1:] - b[1:]).abs()
    scale = float(a[1:].abs().max())
    rel = (d.norm(dim=-1) / a[1:].norm(dim=-1)).max()
    print(f"fused vs module: max |d| {float(d.max()):.3e} of logit scale {scale:.2f}, mean {float(d.mean()):.3e}, "
          f"largest row-relative L2 {float(rel):.3e}", flush=True)
    # bf16 outputs of two GEMM implementations (skinny split-K vs hipBLASLt) and two
    # summation orders of the norms, compounded over 24 layers (measured 1.4e-2)
    assert float(rel) <= 2.5e-2
    assert float(d.max()) <= NEAR_TIE
    top_a, top_b = a[1:].argmax(-1), b[1:].argmax(-1)
    for s, r in (top_a != top_b).nonzero().tolist():
        row = a[1 + s, r]
        assert float(row[top_a[s, r]] - row[top_b[s, r]]) <= NEAR_TIE, f"step {s} row {r}: argmax differs, no near-tie"


@torch.no_grad()
def test_c5_fp8_kv_cache_stays_close_to_bf16(c5):
    cfg, model, lens, prompt = c5
    steps = 4
    g = torch.Generator().manual_seed(SEED + 3)
    forced = torch.randint(0, V, (B, steps), generator=g)
    runs = []
    for kvd in (None, torch.float8_e4m3fn):
        cache, first = _prefill(model, cfg, lens, prompt, steps, kv_dtype=kvd)
        runs.append(_forced_steps(model, cache, first, forced).cpu())
        del cache
    a, b = runs
    rel = (a - b).norm(dim=-1) / a.norm(dim=-1)      # [steps + 1, B]
    top1 = a.argmax(-1) == b.argmax(-1)
    agree = float(top1.float().mean())
    first = float(top1[0].float().mean())  # the prefill's logits: the first generated token
    print(f"fp8 vs bf16 KV: row-relative L2 mean {float(rel.mean()):.3e} max {float(rel.max()):.3e}, "
          f"top-1 agreement {agree:.3f} (first token {first:.3f})", flush=True)
    # e4m3 keeps 3 mantissa bits (|error| <= 1/16 of the value, ~2 % rms) per K/V
    # element; through 24 layers the logits move by a few percent of their norm.
    # Bounds set from the measured distribution of this seeded batch (mean 3.4e-2,
    # max 0.17, top-1 93 %, first token 96.9 %), so that an fp8 accuracy
    # regression of even 1.5x fails.
    assert float(rel.mean()) <= 0.05 and float(rel.max()) <= 0.22
    assert agree >= 0.9 and first >= 0.95


@torch.no_grad()
def test_c5_shortest_sequence_matches_reference_autocast(c5):
    from oracle.ref_model import RefGPT

    from tests.test_gpu_model_bf16 import compare_to_oracles, greedy_agrees

    cfg, model, lens, prompt = c5
    steps = 3
    b = min(range(B), key=lambda i: lens[i])
    n = lens[b]
    cache, first = _prefill(model, cfg, [n], prompt[b:b + 1, :n], steps)
    toks = [int(first[0].argmax())]
    rows = [first[0].cpu()]
    for s in range(steps):
        out, _ = model(torch.tensor([[toks[-1]]], device=DEV), use_cache=True, past_key_values=cache,
                       position_offset=n + s)
        rows.append(out[0, -1].float().cpu())
        toks.append(int(rows[-1].argmax()))
    gpu = torch.stack(rows)
    print(f"oracle run on the CPU: sequence {b}, prompt {n}, {steps} steps", flush=True)
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    res = []
    for bf in (True, False):
        ref = RefGPT(sd, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads, autocast_bf16=bf)
        caches = ref.new_caches(1, n + steps + 1, page_size=P)
        out = [ref.forward(prompt[b:b + 1, :n], caches, 0)[0, -1].float()]
        for s in range(steps):
            out.append(ref.forward(torch.tensor([[toks[s]]]), caches, n + s)[0, -1].float())
        res.append(torch.stack(out))
        del ref
    ob, of = res
    noise = compare_to_oracles(gpu, ob, of, f"C5 sequence {b}")
    greedy_agrees(toks, ob, noise, f"C5 sequence {b}")
