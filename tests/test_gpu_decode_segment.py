"""GPU parity: the per-segment partition of decode attention
(split_tokens = SPLIT_PER_SEGMENT: one workgroup per (sequence, KV head),
its 4 waves on equal quarters of the tiles, merged in LDS, one launch).

* Against the fp64 oracle, with the tolerance of test_gpu_decode_attention.py
  (|out - ref| <= 2e-3 + 2e-2 |ref|): uniform and ragged lengths (the
  partition is correct for any lengths; it is only balanced for equal ones),
  sequences shorter than four tiles (waves with no tiles), a zero-length
  sequence (zeros), G 1-16, head dims on every tile width (32, 64, 128 and the
  padded 24 / 48 / 96), bf16 / fp8 caches, paged / contiguous stores. fp32
  caches run the VALU kernel, which takes -1 as 0.
* The fused decode step in this partition against the two-launch path in the
  same partition, bit for bit (output, cache bytes, fp8 scales, lengths).
* The KV cache picks the partition from its host lengths: equal lengths with
  B * H_kv a multiple of the resident round (tt_decode_pick_split), else the
  balanced one; a model's decode steps agree with the balanced partition's to
  a few bf16 ulps of each row's largest logit; the engine's graph-replayed
  steps in this partition equal its eager steps bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_decode_attention import assert_close, run_case
from tests.test_gpu_decode_fused import _run_both, _setup

pytestmark = pytest.mark.gpu
SEG = -1

CASES = [
    # lengths, Hq, Hkv, D, P, paged, fp8
    ([300] * 6, 32, 8, 128, 16, True, False),
    ([1, 2, 31, 33, 64, 65, 97, 129, 700], 8, 2, 64, 16, False, False),
    ([257, 257, 257, 1000], 16, 1, 128, 32, True, True),
    ([5, 40, 96, 200, 513], 6, 2, 48, 16, True, False),
    ([3, 17, 80, 150], 10, 2, 24, 48, False, False),
    ([33, 64, 100], 4, 4, 32, 16, True, False),
    ([1, 90, 400, 1025], 64, 8, 64, 64, True, True),
    ([500] * 5, 15, 3, 96, 16, False, True),
    ([2048, 1, 700], 40, 8, 128, 16, True, False),
]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_segment_vs_oracle(i):
    lengths, Hq, Hkv, D, P, paged, fp8 = CASES[i]
    print(f"segment case {i}: {CASES[i]}", flush=True)
    got, ref, _ = run_case(lengths, Hq=Hq, Hkv=Hkv, D=D, P=P, paged=paged, fp8=fp8, seed=70 + i, split_tokens=SEG)
    assert_close(got, ref)


def test_segment_zero_length_gives_zeros():
    got, ref, _ = run_case([5, 9, 33, 70], Hq=8, Hkv=2, D=64, seed=3, zero_first=True, split_tokens=SEG)
    assert np.all(got[0] == 0.0)
    assert_close(got[1:], ref[1:])


def test_segment_f32_takes_the_valu_kernel():
    got, ref, _ = run_case([1, 17, 100, 333], Hq=8, Hkv=2, D=64, f32=True, seed=5, split_tokens=SEG)
    assert_close(got, ref, rtol=1e-4, atol=1e-5)


def test_segment_without_workspace():
    """The MFMA per-segment path needs no workspace: a NULL workspace is accepted."""
    from tinytron_amd import _lib, ops

    lengths = [40, 40, 40]
    got, ref, _ = run_case(lengths, Hq=8, Hkv=2, D=64, seed=6, split_tokens=SEG)
    assert_close(got, ref)
    assert _lib.load().tt_decode_workspace_bytes(3, 8, 2, 64, 40, SEG) > 0  # what the VALU fallback would need
    # the bf16 entry point itself, with workspace NULL and 0 bytes
    q = torch.randn(3, 8, 64, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    k = torch.randn(3 * 2 * 48 * 64, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    v = torch.randn_like(k)
    lens = torch.full((3,), 40, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    st = _lib.load().tt_gqa_decode_attn_bf16(
        q.data_ptr(), _lib.strides(*q.stride()[:2]), k.data_ptr(), v.data_ptr(),
        _lib.strides(2 * 48 * 64, 16 * 64, 48 * 64), lens.data_ptr(), 40, None, 0, 0,
        out.data_ptr(), _lib.strides(*out.stride()[:2]), 3, 8, 2, 64, 16, 0.125, SEG, None, None, 0, None)
    assert st == _lib.TT_OK, _lib.load().tt_last_error_string()
    ref_out = ops.decode_attention(q, ops.KVLayout(k=k, v=v, strides=(2 * 48 * 64, 16 * 64, 48 * 64), num_heads=2,
                                                   head_dim=64, page_size=16, capacity=48, kind="bf16"),
                                   lens, 40, sm_scale=0.125)
    torch.cuda.synchronize()
    assert torch.allclose(out.float(), ref_out.float(), atol=2e-3, rtol=2e-2)


@pytest.mark.parametrize("kv,paged,D,G,Hkv,from_partials", [
    ("bf16", True, 128, 4, 8, True),
    ("bf16", False, 64, 4, 4, False),
    ("fp8", True, 64, 8, 2, True),
    ("fp8", False, 128, 2, 4, False),
    ("bf16", True, 32, 16, 1, False),
    ("bf16", False, 48, 3, 2, True),
])
def test_fused_segment_step_equals_two_launches(kv, paged, D, G, Hkv, from_partials):
    """The fused step in the per-segment partition writes the two-launch
    path's cache bytes and gives its output bit for bit (both in that
    partition), with uniform lengths and with ragged ones (a sequence of one
    token: three waves without tiles)."""
    for lens in ([77] * 5, [1, 31, 32, 33, 500]):
        print(f"fused segment: {kv} paged {paged} D {D} G {G} Hkv {Hkv} partials {from_partials} lens {lens}",
              flush=True)
        layer, table, g = _setup(kv, paged, D, G * Hkv, Hkv, lens, seed=D + G)
        _run_both(layer, table, g, G * Hkv, from_partials=from_partials, S=3, split_tokens=SEG)


def test_cache_picks_the_partition_and_matches_balanced():
    """Uniform lengths with B * H_kv a multiple of the resident round take the
    per-segment partition (asserted); a bf16 model's teacher-forced decode
    steps through it give the balanced partition's logits to a few bf16 ulps
    of each row's largest logit."""
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _c1_config, _ulps_of_row_max

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Hkv, D = 8, 64
    B = 2 * cus // Hkv  # one round of two workgroups per CU at head_dim 64
    assert ops.pick_split([100] * B, Hkv, D, "bf16") == SEG
    assert ops.pick_split([100] * (B - 1) + [101], Hkv, D, "bf16") != SEG
    assert ops.pick_split([100] * B, Hkv, D, "f32") == 0
    assert ops.pick_split([100] * (B + 1), Hkv, D, "bf16") == 0
    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=Hkv, block_size=96)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    prompt = torch.randint(0, cfg.vocab_size, (B, 24), generator=torch.Generator().manual_seed(8)).cuda()
    with torch.no_grad():
        seg = PagedKVCache.from_model_config(cfg, B, 16, "cuda", torch.bfloat16)
        bal = PagedKVCache.from_model_config(cfg, B, 16, "cuda", torch.bfloat16)
        ls, seg = model(prompt, past_key_values=seg, use_cache=True)
        lb, bal = model(prompt, past_key_values=bal, use_cache=True)
        for i in range(cfg.num_layer):
            bal.get_layer_cache(i)._split = 0  # force the balanced partition (decode steps keep the pick)
        assert seg.get_layer_cache(0)._attention_split() == SEG
        assert bal.get_layer_cache(0)._attention_split() == 0
        tok = ls[:, -1].argmax(-1, keepdim=True)
        for step in range(4):
            ls, seg = model(tok, past_key_values=seg, use_cache=True, position_offset=24 + step)
            lb, bal = model(tok, past_key_values=bal, use_cache=True, position_offset=24 + step)
            assert _ulps_of_row_max(ls.float().cpu(), lb.float().cpu()) <= 4, f"step {step}"
            tok = ls[:, -1].argmax(-1, keepdim=True)


@pytest.mark.parametrize("kv_dtype", [None, "fp8"])
def test_engine_uniform_batch_segment_graphs_equal_eager(kv_dtype):
    """The reference's own kind of batch (every prompt the same length) with
    B * H_kv filling one round of the GPU: the engine's caches pick the
    per-segment partition (asserted through the pick), and decode steps
    replayed from the captured graphs give the eager steps' tokens and
    log-probabilities bit for bit (the partition's agreement with the balanced
    one is checked on teacher-forced logits above, where greedy near-ties of a
    random-init model cannot move the comparison)."""
    from tinytron_amd import ops
    from tinytron_amd.engine import InferenceEngine
    from tinytron_amd.model import GPT
    from tests.test_gpu_engine import _c1_config

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    Hkv = 8
    B = 2 * cus // Hkv
    cfg = _c1_config(num_layer=2, hidden_size=1024, num_attention_heads=16, num_key_value_heads=Hkv,
                     vocab_size=4096, block_size=160)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    kvd = torch.float8_e4m3fn if kv_dtype == "fp8" else None
    kind = "fp8" if kv_dtype else "bf16"
    assert ops.pick_split([48] * B, Hkv, 64, kind) == SEG
    prompt = torch.randint(0, cfg.vocab_size, (B, 48), generator=torch.Generator().manual_seed(17))
    runs = {}
    for name, use_graphs in (("eager", False), ("graphs", True)):
        eng = InferenceEngine(cfg, device="cuda", dtype=torch.bfloat16, kv_cache_page_size=16, paged_pool=True,
                              kv_cache_dtype=kvd, model=model, use_graphs=use_graphs)
        toks, extra = eng.generate(prompt, 24, top_k=1, return_stats=True, return_logprobs=True)
        runs[name] = (toks.cpu(), extra["token_log_probs"].float().cpu())
    assert torch.equal(runs["eager"][0], runs["graphs"][0])
    assert torch.equal(runs["eager"][1], runs["graphs"][1])
