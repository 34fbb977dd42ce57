"""GPU: the fused decode step (tt_decode_attn_append_*) against the two-launch
path it replaces (rope_append, then decode_attention over positions + 1).

Both paths rotate q and k with the same arithmetic, write the same cache
slot and run the same partition (balanced, or per segment when the test
asks for it) over the same lengths, so the
comparison is bit for bit: attention output, every cache byte (and fp8
scale) and the lengths after the step. The two-launch path is itself pinned
to the oracle by test_gpu_rope_append.py and test_gpu_decode_attention.py.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(kv, paged, D, Hq, Hkv, lens, page=16, seed=0):
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import ModelConfig

    B = len(lens)
    cap = int(max(lens)) + 40
    cfg = ModelConfig(num_layer=1, hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      block_size=cap)
    kvd = torch.float8_e4m3fn if kv == "fp8" else None
    cache = PagedKVCache.from_model_config(cfg, B, page, DEV, torch.bfloat16, kv_cache_dtype=kvd, paged_pool=paged,
                                           seq_capacity=[cap] * B)
    layer = cache.get_layer_cache(0)
    table = ops.build_rope_table(cap, D, device=DEV)
    g = torch.Generator().manual_seed(seed)
    T = int(max(lens))
    q0 = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16).to(DEV)
    k0 = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    v0 = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).to(DEV)
    layer.rope_append(q0, k0, v0, table, new_lens=list(lens))
    return layer, table, g


def _snapshot(layout):
    ts = [layout.k, layout.v] + ([layout.k_scale, layout.v_scale] if layout.kind == "fp8" else [])
    return [t.clone() for t in ts]


def _restore(layout, snap):
    ts = [layout.k, layout.v] + ([layout.k_scale, layout.v_scale] if layout.kind == "fp8" else [])
    for t, s in zip(ts, snap):
        t.copy_(s)


def _run_both(layer, table, g, Hq, from_partials, S=4, split_tokens=0, sorted_order=False):
    from tinytron_amd import ops

    lay = layer.layout
    Hkv, D = lay.num_heads, lay.head_dim
    pos = layer._lens_dev[layer._cur].clone()
    B = pos.shape[0]
    max_len = int(pos.max().item()) + 1
    snap = _snapshot(lay)
    N = (Hq + 2 * Hkv) * D
    order = torch.tensor(ops.length_order(pos.tolist()), dtype=torch.int32, device=DEV) if sorted_order else None
    if from_partials:
        parts = (torch.randn(S, B, N, generator=g) * 0.5).to(DEV)
    else:
        q1 = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        k1 = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        v1 = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)

    lens_a = torch.full_like(pos, -1)
    ws = ops.Workspace(DEV)
    if from_partials:
        q_rot = ops.rope_append_partials(parts, Hq, table, pos, lay, lens_out=lens_a)
    else:
        q_rot = ops.rope_append(q1, k1, v1, table, pos, lay, lens_out=lens_a)
    out_a = ops.decode_attention(q_rot.view(B, Hq, D), lay, lens_a, max_len, workspace=ws, split_tokens=split_tokens,
                                 length_order=order)
    torch.cuda.synchronize()
    after_a = _snapshot(lay)

    _restore(lay, snap)
    lens_b = torch.full_like(pos, -1)
    ws_b = ops.Workspace(DEV)
    if from_partials:
        out_b = ops.decode_attention_append(table, pos, lay, max_len, partials=parts, num_q_heads=Hq,
                                            lens_out=lens_b, workspace=ws_b, split_tokens=split_tokens,
                                            length_order=order)
    else:
        out_b = ops.decode_attention_append(table, pos, lay, max_len, q=q1[:, :, 0], k=k1[:, :, 0], v=v1[:, :, 0],
                                            lens_out=lens_b, workspace=ws_b, split_tokens=split_tokens,
                                            length_order=order)
    torch.cuda.synchronize()
    after_b = _snapshot(lay)
    assert torch.equal(lens_a, lens_b)
    assert torch.equal(lens_b, pos + 1)
    for x, y in zip(after_a, after_b):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), "cache bytes differ"
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), \
        f"outputs differ: max |diff| {(out_a.float() - out_b.float()).abs().max().item()}"


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("paged", [True, False])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("from_partials", [False, True])
def test_fused_step_equals_two_launches(kv, paged, D, from_partials):
    rng = np.random.default_rng(D + 7 * paged)
    lens = rng.integers(1, 300, size=9).tolist()
    lens[0] = 31  # the new token opens a tile
    lens[1] = 32  # ... and a page
    Hq, Hkv = 8, 2
    layer, table, g = _setup(kv, paged, D, Hq, Hkv, lens)
    _run_both(layer, table, g, Hq, from_partials)


@pytest.mark.parametrize("G,Hkv", [(1, 4), (4, 8), (8, 2), (16, 1)])
def test_fused_step_group_sizes(G, Hkv):
    lens = [5, 200, 63, 64, 1, 1000]
    layer, table, g = _setup("bf16", True, 128, G * Hkv, Hkv, lens)
    _run_both(layer, table, g, G * Hkv, from_partials=True)


def test_fused_step_long_segments_split_over_waves():
    # a few long sequences: each segment spans many waves, only the wave
    # holding its last tile appends
    lens = [9000, 4000, 7777, 1]
    layer, table, g = _setup("bf16", True, 128, 32, 8, lens)
    _run_both(layer, table, g, 32, from_partials=False)
    _run_both(layer, table, g, 32, from_partials=True)


def test_fused_step_consecutive_steps():
    # three fused steps in a row equal three two-launch steps
    from tinytron_amd import ops

    lens = [17, 250, 96, 3]
    la, table, ga = _setup("fp8", True, 64, 16, 4, lens, seed=5)
    lb, _, gb = _setup("fp8", True, 64, 16, 4, lens, seed=5)
    _restore(lb.layout, _snapshot(la.layout))  # identical bytes in the never-written slots too
    B, Hq, D = len(lens), 16, 64
    N = (Hq + 8) * D
    ws_a, ws_b = ops.Workspace(DEV), ops.Workspace(DEV)
    for step in range(3):
        parts = (torch.randn(4, B, N, generator=ga) * 0.5).to(DEV)
        max_len = max(lens) + step + 1
        nxt = 1 - la._cur
        q_rot = ops.rope_append_partials(parts, Hq, table, la._lens_dev[la._cur], la.layout,
                                         lens_out=la._lens_dev[nxt])
        out_a = ops.decode_attention(q_rot.view(B, Hq, D), la.layout, la._lens_dev[nxt], max_len, workspace=ws_a)
        la._cur = nxt
        nxt = 1 - lb._cur
        out_b = ops.decode_attention_append(table, lb._lens_dev[lb._cur], lb.layout, max_len, partials=parts,
                                            num_q_heads=Hq, lens_out=lb._lens_dev[nxt], workspace=ws_b)
        lb._cur = nxt
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)), f"step {step}"
    torch.cuda.synchronize()
    assert torch.equal(la.layout.k, lb.layout.k) and torch.equal(la.layout.v, lb.layout.v)
    assert torch.equal(la.layout.k_scale, lb.layout.k_scale)


def test_fused_step_rejects_bad_bounds():
    from tinytron_amd import ops

    layer, table, g = _setup("bf16", True, 64, 8, 2, [10, 20])
    pos = layer._lens_dev[layer._cur]
    q = torch.zeros(2, 8, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(2, 2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="max_seq_len"):
        ops.decode_attention_append(table, pos, layer.layout, 0, q=q, k=k, v=k)
    with pytest.raises(ValueError, match="max_seq_len"):
        ops.decode_attention_append(table, pos, layer.layout, layer.layout.capacity + 1, q=q, k=k, v=k)
