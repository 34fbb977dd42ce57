"""GPU parity: the paired partition of decode attention
(split_tokens = SPLIT_PAIRED: the sequences ranked by length, one workgroup
per (rank pair (p, B - 1 - p), KV head), its waves on equal shares of the two
segments' tiles, merged in LDS, one launch, no workspace; B <= 256).

* Against the fp64 oracle, with the tolerance of test_gpu_decode_attention.py
  (|out - ref| <= 2e-3 + 2e-2 |ref|): ragged and uniform lengths, odd batches
  (the middle rank alone), ties in length (ranked by index), sequences shorter
  than the workgroup's waves (waves with no tiles, or with tiles of only one
  of the two segments), zero-length sequences (zeros), G 1-16, head dims on
  every tile width (32, 64, 128 and the padded 24 / 48 / 96), bf16 / fp8
  caches, paged / contiguous stores, one sequence and 256 sequences. fp32
  caches run the VALU kernel, which takes -2 as 0.
* The fused decode step in this partition against the two-launch path in the
  same partition, bit for bit (output, cache bytes, fp8 scales, lengths).
* With the caller's length order (length_order, the order the device ranks)
  the outputs equal the device-ranked ones bit for bit (same pairs, same
  arithmetic), for the two-launch and the fused step; any other permutation
  pairs differently and stays within the oracle tolerance.
* More than 256 sequences are refused.
* The KV cache picks the partition from its host lengths (ragged, B <= 256,
  rank pairs filling the CUs evenly: tt_decode_pick_split); a model's decode
  steps through it agree with the balanced partition's to a few bf16 ulps of
  each row's largest logit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_decode_attention import assert_close, run_case
from tests.test_gpu_decode_fused import _run_both, _setup

pytestmark = pytest.mark.gpu
PAIRED = -2

CASES = [
    # lengths, Hq, Hkv, D, P, paged, fp8
    ([300, 1, 2000, 65, 640, 33, 900], 32, 8, 128, 16, True, False),
    ([1, 2, 31, 33, 64, 65, 97, 129, 700], 8, 2, 64, 16, False, False),
    ([257, 257, 257, 1000], 16, 1, 128, 32, True, True),
    ([5, 40, 96, 200, 513], 6, 2, 48, 16, True, False),
    ([3, 17, 80, 150], 10, 2, 24, 48, False, False),
    ([33, 64, 100], 4, 4, 32, 16, True, False),
    ([1, 90, 400, 1025, 7, 7], 64, 8, 64, 64, True, True),
    ([500] * 5, 15, 3, 96, 16, False, True),
    ([2048, 1, 700], 64, 4, 128, 16, True, False),   # G 16 at D 128
    ([4000], 8, 2, 64, 16, True, False),             # one sequence: one rank, no pair
    ([100, 100, 100, 100, 3000, 3000], 16, 1, 64, 16, False, False),  # ties
]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_paired_vs_oracle(i):
    lengths, Hq, Hkv, D, P, paged, fp8 = CASES[i]
    print(f"paired case {i}: {CASES[i]}", flush=True)
    got, ref, _ = run_case(lengths, Hq=Hq, Hkv=Hkv, D=D, P=P, paged=paged, fp8=fp8, seed=170 + i, split_tokens=PAIRED)
    assert_close(got, ref)


@pytest.mark.parametrize("fp8", [False, True])
def test_paired_full_batch(fp8):
    """256 sequences (the most the partition takes), lengths U[1, 1200]."""
    rng = np.random.default_rng(11 + fp8)
    lengths = [int(x) for x in rng.integers(1, 1201, size=256)]
    print(f"paired full batch fp8 {fp8}", flush=True)
    got, ref, _ = run_case(lengths, Hq=8, Hkv=2, D=64, paged=True, fp8=fp8, seed=33, split_tokens=PAIRED)
    assert_close(got, ref)


def test_paired_zero_length_gives_zeros():
    got, ref, _ = run_case([5, 9, 33, 70, 11], Hq=8, Hkv=2, D=64, seed=3, zero_first=True, split_tokens=PAIRED)
    assert np.all(got[0] == 0.0)
    assert_close(got[1:], ref[1:])


def test_paired_f32_takes_the_valu_kernel():
    got, ref, _ = run_case([1, 17, 100, 333], Hq=8, Hkv=2, D=64, f32=True, seed=5, split_tokens=PAIRED)
    assert_close(got, ref, rtol=1e-4, atol=1e-5)


def test_paired_refuses_more_than_256_sequences():
    from tinytron_amd import _lib

    B, Hq, Hkv, D, cap = 257, 4, 1, 64, 32
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(B * Hkv * cap * D, dtype=torch.bfloat16, device="cuda")
    lens = torch.full((B,), 8, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    st = _lib.load().tt_gqa_decode_attn_bf16(
        q.data_ptr(), _lib.strides(*q.stride()[:2]), k.data_ptr(), k.data_ptr(),
        _lib.strides(Hkv * cap * D, 16 * D, cap * D), lens.data_ptr(), 8, None, 0, 0,
        out.data_ptr(), _lib.strides(*out.stride()[:2]), B, Hq, Hkv, D, 16, 0.125, PAIRED, None, None, 0, None)
    assert st == _lib.TT_ERR_UNSUPPORTED
    assert "256" in _lib.load().tt_last_error_string().decode()


@pytest.mark.parametrize("kv,paged,D,G,Hkv,from_partials", [
    ("bf16", True, 128, 4, 8, True),
    ("bf16", False, 64, 4, 4, False),
    ("fp8", True, 64, 8, 2, True),
    ("fp8", False, 128, 2, 4, False),
    ("bf16", True, 32, 16, 1, False),
    ("bf16", False, 48, 3, 2, True),
])
def test_fused_paired_step_equals_two_launches(kv, paged, D, G, Hkv, from_partials):
    """The fused step in the paired partition writes the two-launch path's
    cache bytes and gives its output bit for bit (both in that partition),
    with ragged lengths (odd and even batches) and uniform ones."""
    for lens in ([1, 31, 32, 33, 500], [7, 300, 64, 1000, 2, 129], [77] * 4):
        print(f"fused paired: {kv} paged {paged} D {D} G {G} Hkv {Hkv} partials {from_partials} lens {lens}",
              flush=True)
        layer, table, g = _setup(kv, paged, D, G * Hkv, Hkv, lens, seed=D + G + 1)
        _run_both(layer, table, g, G * Hkv, from_partials=from_partials, S=3, split_tokens=PAIRED)


def test_cache_picks_paired_for_ragged_lengths_and_matches_balanced():
    """A ragged batch whose rank pairs carry equal work (lengths 16, 32, ...,
    16 B) and fill one round of the GPU's CUs takes the
    paired partition (asserted); a bf16 model's teacher-forced decode steps
    through it give the balanced partition's logits to a few bf16 ulps of each
    row's largest logit. One pair far heavier than the mean keeps the balanced
    partition."""
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _c1_config, _ulps_of_row_max

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Hkv, D = 8, 64
    B = 2 * cus // Hkv  # (B / 2) * H_kv workgroups: one per CU
    lens = [16 * (i + 1) for i in range(B)]  # ranks p and B - 1 - p: (B + 2) / 2 tiles together
    assert ops.pick_split(lens, Hkv, D, "bf16") == PAIRED
    assert ops.pick_split(lens[:-1] + [lens[-1] + 40 * 32], Hkv, D, "bf16") == 0
    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=Hkv,
                     block_size=max(lens) + 16)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(12)
    prompt = torch.randint(0, cfg.vocab_size, (B, max(lens)), generator=g).cuda()
    steps = torch.randint(0, cfg.vocab_size, (B, 4), generator=g).cuda()
    last = torch.tensor(lens, device="cuda") - 1
    logits = {}
    with torch.no_grad():
        for name in ("paired", "balanced"):
            cache = PagedKVCache.from_model_config(cfg, B, 16, "cuda", torch.bfloat16,
                                                   seq_capacity=[n + 8 for n in lens])
            cache.set_pending_new_lens(lens)
            out, cache = model(prompt, past_key_values=cache, use_cache=True, logits_index=last)
            cache.set_pending_new_lens(None)
            if name == "balanced":
                for i in range(cfg.num_layer):
                    cache.get_layer_cache(i)._split = 0  # force the balanced partition
            assert cache.get_layer_cache(0)._attention_split() == (PAIRED if name == "paired" else 0)
            if name == "paired":  # the host's length order, uploaded once for the decode loop
                order = cache.get_layer_cache(0)._order
                assert order is not None and order.tolist() == ops.length_order(lens)
            rows = []
            for s in range(steps.shape[1]):
                out, cache = model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
                rows.append(out[:, -1].float().cpu())
            logits[name] = torch.stack(rows)
    assert _ulps_of_row_max(logits["paired"], logits["balanced"]) <= 4


@pytest.mark.parametrize("i", [0, 1, 6, 9, 10])
def test_paired_host_order_equals_device_ranking(i):
    lengths, Hq, Hkv, D, P, paged, fp8 = CASES[i]
    print(f"paired order case {i}: {CASES[i]}", flush=True)
    dev, ref, _ = run_case(lengths, Hq=Hq, Hkv=Hkv, D=D, P=P, paged=paged, fp8=fp8, seed=170 + i, split_tokens=PAIRED)
    host, _, _ = run_case(lengths, Hq=Hq, Hkv=Hkv, D=D, P=P, paged=paged, fp8=fp8, seed=170 + i, split_tokens=PAIRED,
                          length_order="sorted")
    assert np.array_equal(dev.view(np.uint32), host.view(np.uint32))
    assert_close(host, ref)


def test_paired_other_permutation_stays_correct():
    lengths = [300, 1, 2000, 65, 640, 33, 900, 12]
    perm = [3, 0, 7, 5, 1, 6, 2, 4]  # not the length order: other pairs, same coverage
    got, ref, _ = run_case(lengths, Hq=16, Hkv=4, D=64, paged=True, seed=9, split_tokens=PAIRED, length_order=perm)
    assert_close(got, ref)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_fused_paired_step_host_order_equals_device_ranking(kv):
    """The fused step with the caller's order writes the same cache bytes and
    outputs as with the device's ranking (the order of positions + 1), from
    the same cache state."""
    from tinytron_amd import ops
    from tests.test_gpu_decode_fused import _restore, _snapshot

    lens = [7, 300, 64, 1000, 2, 129, 129]
    layer, table, g = _setup(kv, True, 64, 16, 4, lens, seed=31)
    lay = layer.layout
    pos = layer._lens_dev[layer._cur].clone()
    B = pos.shape[0]
    q1 = torch.randn(B, 16, 64, generator=g).to(torch.bfloat16).cuda()
    k1 = torch.randn(B, 4, 64, generator=g).to(torch.bfloat16).cuda()
    v1 = torch.randn(B, 4, 64, generator=g).to(torch.bfloat16).cuda()
    snap = _snapshot(lay)
    runs = []
    for use_order in (False, True):
        _restore(lay, snap)
        order = torch.tensor(ops.length_order(lens), dtype=torch.int32, device="cuda") if use_order else None
        out = ops.decode_attention_append(table, pos, lay, max(lens) + 1, q=q1, k=k1, v=v1, split_tokens=PAIRED,
                                          length_order=order)
        torch.cuda.synchronize()
        runs.append([out.clone()] + _snapshot(lay))
    for x, y in zip(runs[0], runs[1]):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))


def test_engine_paired_graphs_equal_eager():
    """A ragged batch that picks the paired partition (asserted) decodes the
    same tokens and log-probabilities bit for bit with the step replayed from
    captured graphs as eagerly. Regression: capture restores the caches' host
    lengths, which re-picks the partition; the length order must stay in the
    buffer the graphs captured (a fresh tensor each pick left the graphs
    reading freed memory and pairing wrongly)."""
    from tinytron_amd import ops
    from tinytron_amd.engine import InferenceEngine
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _c1_config

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Hkv = 8
    B = 2 * cus // Hkv
    lens = [16 * (i + 1) for i in range(B)]
    assert ops.pick_split(lens, Hkv, 64, "bf16") == PAIRED
    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=Hkv,
                     vocab_size=4096, block_size=max(lens) + 32)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    prompt = torch.randint(0, cfg.vocab_size, (B, max(lens)), generator=torch.Generator().manual_seed(23))
    runs = {}
    for name, use_graphs in (("eager", False), ("graphs", True)):
        eng = InferenceEngine(cfg, device="cuda", dtype=torch.bfloat16, kv_cache_page_size=16, paged_pool=True,
                              model=model, use_graphs=use_graphs)
        toks, extra = eng.generate(prompt, 24, top_k=1, prompt_lens=lens, return_stats=True, return_logprobs=True)
        runs[name] = (toks.cpu(), extra["token_log_probs"].float().cpu())
    assert torch.equal(runs["eager"][0], runs["graphs"][0])
    assert torch.equal(runs["eager"][1], runs["graphs"][1])


def test_graph_captured_before_the_first_pick_ranks_on_the_device():
    """A decode step captured before the cache has picked its partition picks
    the paired one under capture, where no host copy can be recorded: the
    graph ranks the lengths on the device (no order uploaded) and its replay
    gives the logits of an eager step that uses the host's order, bit for
    bit (the same pairs)."""
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.engine import DecodeGraphs
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _c1_config

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Hkv = 8
    B = 2 * cus // Hkv
    lens = [16 * (i + 1) for i in range(B)]
    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=Hkv,
                     block_size=max(lens) + 16)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(41)
    prompt = torch.randint(0, cfg.vocab_size, (B, max(lens)), generator=g).cuda()
    tok = torch.randint(0, cfg.vocab_size, (B, 1), generator=g).cuda()
    last = torch.tensor(lens, device="cuda") - 1
    outs = {}
    with torch.no_grad():
        for name in ("graph", "eager"):
            cache = PagedKVCache.from_model_config(cfg, B, 16, "cuda", torch.bfloat16,
                                                   seq_capacity=[n + 8 for n in lens])
            cache.set_pending_new_lens(lens)
            model(prompt, past_key_values=cache, use_cache=True, logits_index=last)
            cache.set_pending_new_lens(None)
            if name == "graph":
                graphs = DecodeGraphs(model, cache, B, 0, False, torch.device("cuda"))
                assert cache.get_layer_cache(0)._order is None  # nothing uploaded under capture
                outs[name] = graphs.step(tok)[:, -1].float().cpu()
            else:
                out, cache = model(tok, past_key_values=cache, use_cache=True)
                assert cache.get_layer_cache(0)._attention_split() == PAIRED
                assert cache.get_layer_cache(0)._order is not None
                outs[name] = out[:, -1].float().cpu()
    assert torch.equal(outs["graph"], outs["eager"])
