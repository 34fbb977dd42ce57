"""GPU: the fused decode step issued by the library in one call
(tt_decode_layers_bf16, GPT.native_decode_step) against the same step issued
op by op from Python (GPT.native_decode_step = False). Both run the same
kernels with the same arguments, so the logits and the caches they leave
must agree bit for bit, step after step, for every attention partition
(balanced, per-segment, paired with and without the host rank order), bf16
and fp8 caches, the paged pool and the contiguous store, and both gate|up
forms (one-launch SwiGLU, split-K partials + silu_mul). The op-by-op path is
itself pinned to the reference's op sequence by test_gpu_model_bf16.py.
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


def _model(hidden, heads, kv_heads, inter, layers=2, seed=7):
    from tinytron_amd.model import GPT, ModelConfig

    cfg = ModelConfig(num_layer=layers, hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv_heads,
                      vocab_size=4096, intermediate_size=inter, init_std=0.02, block_size=512, tied_lm_head=True)
    torch.manual_seed(seed)
    return GPT(cfg, device=DEV, dtype=BF16), cfg


def _prefilled(model, cfg, lens, steps, paged, kv_dtype, seed):
    from tinytron_amd.cache import PagedKVCache

    B = len(lens)
    cache = PagedKVCache.from_model_config(cfg, B, 16 if paged else 128, DEV, kv_dtype, paged_pool=paged,
                                           seq_capacity=[n + steps + 1 for n in lens])
    prompt = torch.randint(0, cfg.vocab_size, (B, max(lens)), generator=torch.Generator().manual_seed(seed))
    with torch.no_grad():
        cache.set_pending_new_lens(lens)
        out, _ = model(prompt.to(DEV), use_cache=True, past_key_values=cache, position_offset=0,
                       logits_index=torch.tensor(lens, device=DEV) - 1)
        cache.set_pending_new_lens(None)
    return cache, out[:, -1]


def _steps(model, cache, first, lens, steps, native, split=None):
    """Greedy steps from the prefill's logits; returns every step's logits.
    ``split`` forces every layer's attention partition after the prefill."""
    model.native_decode_step = native
    if split is not None:
        for i in range(len(model.blocks)):
            cache.get_layer_cache(i)._split = split
    row, out = first, []
    with torch.no_grad():
        for s in range(steps):
            t = row.float().argmax(-1)
            pos = lens[0] + s if len(set(lens)) == 1 else 0
            logits, _ = model(t.view(-1, 1), use_cache=True, past_key_values=cache, position_offset=pos)
            row = logits[:, -1]
            out.append(row.clone())
    return out


def _cache_rows(cache, lens, steps, layers):
    """Each sequence's cached K / V (dequantized for fp8) after the steps."""
    rows = []
    for i in range(layers):
        layer = cache.get_layer_cache(i)
        for b, n in enumerate(lens):
            k, v = layer.gather(b, n + steps)
            rows += [k.float(), v.float()]
    return rows


CASES = {
    # name: (hidden, heads, kv heads, ffn, lens, paged, kv dtype, forced split)
    "balanced_ragged": (1024, 16, 4, 2048, [70, 9, 33], True, BF16, None),
    "per_segment_uniform": (1024, 16, 8, 2048, [40] * 64, True, BF16, None),
    "paired_host_order": (1024, 16, 8, 2048, [100 + 3 * b for b in range(64)], True, BF16, None),
    "paired_device_rank": (1024, 16, 4, 2048, [70, 9, 33, 120, 5], True, BF16, -2),
    "fp8_paged": (1024, 16, 4, 2048, [70, 9, 33], True, torch.float8_e4m3fn, None),
    "fp8_paired": (1024, 16, 8, 2048, [100 + 3 * b for b in range(64)], True, torch.float8_e4m3fn, None),
    "contiguous_store": (1024, 16, 4, 2048, [70, 9, 33], False, BF16, None),
    "splitk_gate_up": (512, 8, 2, 1024, [70, 9, 33], True, BF16, None),
    "head_dim_128": (2048, 16, 4, 2048, [70, 9, 33, 17], True, BF16, None),
}


@pytest.mark.parametrize("name", list(CASES))
def test_one_call_step_equals_op_by_op(name):
    from tinytron_amd import ops

    hidden, heads, kvh, inter, lens, paged, kv_dtype, split = CASES[name]
    model, cfg = _model(hidden, heads, kvh, inter)
    assert model._swiglu_fused() == (name != "splitk_gate_up")
    steps = 5
    print(f"case {name}: B {len(lens)}", flush=True)
    runs = {}
    for native in (True, False):
        cache, first = _prefilled(model, cfg, lens, steps, paged, kv_dtype, seed=11)
        calls = []
        fn = model._decode_step_native
        model._decode_step_native = lambda *a, **k: (calls.append(1), fn(*a, **k))[1]
        try:
            logits = _steps(model, cache, first, lens, steps, native, split)
        finally:
            del model._decode_step_native
        assert len(calls) == (steps if native else 0), f"the one-call step ran {len(calls)} times"
        picked = cache.get_layer_cache(0)._split
        runs[native] = (logits, _cache_rows(cache, lens, steps, cfg.num_layer), picked)
    if name.startswith("paired"):
        assert runs[True][2] == ops.SPLIT_PAIRED
    elif name == "per_segment_uniform":
        assert runs[True][2] == ops.SPLIT_PER_SEGMENT
    elif name == "balanced_ragged":
        assert runs[True][2] == 0
    for s, (a, b) in enumerate(zip(runs[True][0], runs[False][0])):
        assert torch.equal(a, b), f"{name}: step {s} logits differ (max {float((a.float() - b.float()).abs().max())})"
    for j, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        assert torch.equal(a, b), f"{name}: cached row set {j} differs"


def test_one_call_step_refuses_a_bad_layer_and_names_it():
    """A layer whose k_chunk is not positive is refused before anything of
    it is launched, with its index in the message; no layers is a no-op."""
    import ctypes

    from tinytron_amd import _lib, ops

    model, cfg = _model(1024, 16, 4, 2048)
    lens = [70, 9, 33]
    cache, first = _prefilled(model, cfg, lens, 2, True, BF16, seed=3)
    _steps(model, cache, first, lens, 1, True)
    plan = next(iter(model._native_plans.values()))
    arr = (_lib.DecodeLayer * 2)()
    ctypes.memmove(arr, plan[3], ctypes.sizeof(arr))
    arr[0].kc_down = 0
    lib, stream = _lib.load(), ops._stream(torch.device(DEV))
    assert lib.tt_decode_layers_bf16(ctypes.addressof(arr), 0, 1, stream) == _lib.TT_OK
    with pytest.raises(ValueError, match="layer 0: bad k_chunk"):
        _lib.check(lib.tt_decode_layers_bf16(ctypes.addressof(arr), 2, 128, stream), "decode step")
    torch.cuda.synchronize()


def test_plan_follows_alternating_caches():
    """Two caches of different batches and partitions stepped in turn on one
    model: the argument array is rebuilt for each switch (its signature names
    the cache's layouts and length buffers), and every step equals the
    op-by-op path's."""
    model, cfg = _model(1024, 16, 8, 2048)
    cases = [([100 + 3 * b for b in range(64)], 21), ([70, 9, 33], 22)]
    out = {}
    for native in (True, False):
        model.native_decode_step = native
        runs = [list(_prefilled(model, cfg, lens, 4, True, BF16, seed)) for lens, seed in cases]
        got = []
        with torch.no_grad():
            for s in range(4):
                for k, (lens, _) in enumerate(cases):
                    cache, row = runs[k]
                    t = row.float().argmax(-1)
                    logits, _ = model(t.view(-1, 1), use_cache=True, past_key_values=cache, position_offset=0)
                    runs[k][1] = logits[:, -1]
                    got.append(logits[:, -1].clone())
        out[native] = got
    for i, (a, b) in enumerate(zip(out[True], out[False])):
        assert torch.equal(a, b), f"step {i // 2} of cache {i % 2} differs"


def test_plan_does_not_keep_a_finished_cache_alive():
    """The model's argument array holds the cache's objects weakly: a cache
    dropped by its caller is freed (its K pool with it)."""
    import gc
    import weakref

    model, cfg = _model(1024, 16, 4, 2048)
    lens = [70, 9, 33]
    cache, first = _prefilled(model, cfg, lens, 2, True, BF16, seed=5)
    _steps(model, cache, first, lens, 2, True)
    assert model._native_plans
    pool = weakref.ref(cache.get_layer_cache(0).layout.k)
    del cache, first
    gc.collect()
    assert pool() is None
