"""GPU: the reference's non-paged paths on the library's kernels.

* use_paged_kv_cache=False (engine.py:168-178, attn.py:174-186): per-layer
  (k, v) tuples of GQA-expanded heads grown by concatenation. C1 (fp32) greedy
  tokens equal the reference op sequence's with the same tuple cache
  (oracle.ref_model, tuple_cache=True), barring a near-tie; a bf16 model's
  logits through the tuples equal the paged cache's (prefill and
  teacher-forced decode steps) to a few bf16 ulps.
* The tuples keep the reference's shapes and values: [B, H_q, T, D], every
  call extends the newest tuple, and continuing an older tuple (a branch)
  leaves the tuples already handed out unchanged.
* The uncached forward (past_key_values None, use_cache False) gives the
  logits of the reference op sequence (fp32) and of the paged prefill (bf16).
"""
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_engine import _c1_config, _first_divergence

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_c1_tuple_cache_greedy_tokens_match_reference_cpu_path():
    from oracle.ref_model import RefGPT
    from tinytron_amd.engine import InferenceEngine
    from tinytron_amd.model import GPT

    cfg = _c1_config()
    model = GPT(cfg, device="cpu", dtype=torch.float32)
    state = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    eng = InferenceEngine(cfg, device=DEV, dtype=torch.float32, use_paged_kv_cache=False, model=model)
    g = torch.Generator().manual_seed(1337)
    prompt = torch.randint(0, cfg.vocab_size, (1, 128), generator=g)
    tokens, stats = eng.generate(prompt, 64, temperature=1.0, top_k=1, return_stats=True)
    ref = RefGPT(state, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads)
    ref_tokens, _, ref_logits = ref.generate_greedy(prompt, 64, cfg.block_size, tuple_cache=True)
    got = tokens.cpu()
    assert got.shape == ref_tokens.shape == (1, 192)
    div = _first_divergence(got, ref_tokens)
    if div is not None:
        step = div[1] - 128
        top2 = torch.topk(ref_logits[step][0].float(), 2).values
        assert float(top2[0] - top2[1]) < 1e-4, f"tokens diverge at step {step} without a near-tie"
    assert stats["decode_tokens_per_sec"] > 0


@pytest.mark.parametrize("hidden,heads,kv_heads", [(1024, 16, 4), (768, 16, 4)])
def test_bf16_tuple_cache_equals_paged_cache(hidden, heads, kv_heads):
    """bf16, D 64 (the MFMA decode / prefill kernels over the expanded store)
    and D 48 (a padded tile): prefill and 8 teacher-forced decode steps through
    the tuple cache give the paged cache's logits to a few bf16 ulps of each
    row's largest logit (the two caches split the attention work differently,
    so the fp32 merge order, and at most the last bits, differ)."""
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _ulps_of_row_max

    cfg = _c1_config(num_layer=2, hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv_heads,
                     block_size=128)
    model = GPT(cfg, device=DEV, dtype=torch.bfloat16)
    B, T = 3, 40
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(5)).to(DEV)
    with torch.no_grad():
        paged = PagedKVCache.from_model_config(cfg, B, 16, DEV, torch.bfloat16)
        lp, paged = model(prompt, past_key_values=paged, use_cache=True)
        lt, past = model(prompt, past_key_values=None, use_cache=True)
        assert len(past) == 2 and past[0][0].shape == (B, heads, T, hidden // heads)
        assert _ulps_of_row_max(lp.float().cpu(), lt.float().cpu()) <= 4
        tok = lp[:, -1].argmax(-1, keepdim=True)
        for step in range(8):
            lp, paged = model(tok, past_key_values=paged, use_cache=True, position_offset=T + step)
            lt, past = model(tok, past_key_values=past, use_cache=True, position_offset=T + step)
            assert _ulps_of_row_max(lp.float().cpu(), lt.float().cpu()) <= 4, f"step {step}"
            tok = lp[:, -1].argmax(-1, keepdim=True)


def test_tuple_semantics_shapes_and_branches():
    """Shapes [B, H_q, T, D]; a call continuing the newest tuple extends it; a
    call continuing an older tuple gives what a fresh store holding that tuple
    gives, and the tuples handed out before keep their values."""
    from tinytron_amd.model import Attention

    cfg = _c1_config(num_layer=1, hidden_size=512, num_attention_heads=8, num_key_value_heads=2, block_size=64)
    attn = Attention(cfg, 0, device=DEV, dtype=torch.bfloat16)
    other = Attention(cfg, 0, device=DEV, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(9)
    x0 = torch.randn(2, 10, 512, generator=g).to(DEV, torch.bfloat16)
    x1 = torch.randn(2, 1, 512, generator=g).to(DEV, torch.bfloat16)
    x2 = torch.randn(2, 1, 512, generator=g).to(DEV, torch.bfloat16)
    with torch.no_grad():
        _, t0 = attn(x0, past_kv=None, use_cache=True, position_offset=0)
        assert t0[0].shape == t0[1].shape == (2, 8, 10, 64)
        y1, t1 = attn(x1, past_kv=t0, use_cache=True, position_offset=10)
        assert t1[0].shape == (2, 8, 11, 64)
        assert torch.equal(t1[0][:, :, :10], t0[0]) and torch.equal(t1[1][:, :, :10], t0[1])
        t1_copy = (t1[0].clone(), t1[1].clone())
        y2, t2 = attn(x2, past_kv=t0, use_cache=True, position_offset=10)          # a branch from t0
        assert torch.equal(t1[0], t1_copy[0]) and torch.equal(t1[1], t1_copy[1])    # t1 unchanged
        y2_fresh, t2_fresh = other(x2, past_kv=(t0[0].clone(), t0[1].clone()), use_cache=True, position_offset=10)
        assert torch.equal(y2, y2_fresh) and torch.equal(t2[0], t2_fresh[0]) and torch.equal(t2[1], t2_fresh[1])
        y1_again, _ = other(x1, past_kv=(t0[0].clone(), t0[1].clone()), use_cache=True, position_offset=10)
        assert torch.equal(y1, y1_again)
        with pytest.raises(ValueError, match="position_offset"):
            attn(x1, past_kv=t2, use_cache=True, position_offset=3)


def test_uncached_forward_fp32_matches_reference_op_sequence():
    from oracle.ref_model import RefGPT
    from tinytron_amd.model import GPT

    cfg = _c1_config(num_layer=2, block_size=128)
    model = GPT(cfg, device="cpu", dtype=torch.float32)
    state = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    idx = torch.randint(0, cfg.vocab_size, (2, 37), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        got = model(idx.to(DEV)).float().cpu()
    ref = RefGPT(state, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads)
    want = ref.forward(idx, ref.new_caches(2, cfg.block_size, tuple_cache=True), 0)
    torch.testing.assert_close(got, want.float(), rtol=1e-3, atol=1e-3)


def test_uncached_forward_bf16_matches_paged_prefill():
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import GPT

    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=4, block_size=128)
    model = GPT(cfg, device=DEV, dtype=torch.bfloat16)
    idx = torch.randint(0, cfg.vocab_size, (2, 33), generator=torch.Generator().manual_seed(4)).to(DEV)
    with torch.no_grad():
        plain = model(idx).float()
        cache = PagedKVCache.from_model_config(cfg, 2, 16, DEV, torch.bfloat16)
        paged, _ = model(idx, past_key_values=cache, use_cache=True)
    from tests.test_gpu_engine import _ulps_of_row_max

    assert plain.shape == (2, 33, cfg.vocab_size)
    assert _ulps_of_row_max(plain.cpu(), paged.float().cpu()) <= 4
