"""GPU: the allocation-free decode step (tt_decode_attn_append_bf16_noalloc,
whose attention workspace is the library's own per-GPU scratch) against the
entry point it varies (tt_decode_attn_append_bf16 with a caller workspace).

Both run the same kernels over the same inputs, so the comparison is bit for
bit: attention output, every cache byte and the lengths after the step. Two
allocation-free calls run back to back, the second on a smaller batch: the
scratch keeps the first call's contents, and nothing in it may need to start
at zero. A call whose workspace would exceed the scratch is refused before
any launch. tt_decode_attn_append_bf16 itself is pinned to the oracle by the
fused-step and decode-attention parity tests.
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(paged, D, Hq, Hkv, lens, seed, page=16):
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import ModelConfig

    B = len(lens)
    cap = int(max(lens)) + 8
    cfg = ModelConfig(num_layer=1, hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      block_size=cap)
    cache = PagedKVCache.from_model_config(cfg, B, page, DEV, torch.bfloat16, paged_pool=paged,
                                           seq_capacity=[cap] * B)
    layer = cache.get_layer_cache(0)
    table = ops.build_rope_table(cap + 1, D, device=DEV)
    g = torch.Generator().manual_seed(seed)
    gd = torch.Generator(device=DEV).manual_seed(seed)
    T = int(max(lens))
    q0 = torch.randn(B, Hq, T, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    k0 = torch.randn(B, Hkv, T, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    v0 = torch.randn(B, Hkv, T, D, generator=gd, device=DEV, dtype=torch.bfloat16)
    layer.rope_append(q0, k0, v0, table, new_lens=list(lens))
    torch.cuda.synchronize()
    return layer, table, g


def _step_both(layer, table, g, Hq, from_partials):
    """One decode step through each entry point on identical cache copies; returns
    (out, cache bytes, lens) of the workspace call and of the allocation-free call."""
    from tinytron_amd import ops

    lay = layer.layout
    Hkv, D = lay.num_heads, lay.head_dim
    pos = layer._lens_dev[layer._cur].clone()
    B = pos.shape[0]
    max_len = int(pos.max().item()) + 1
    if from_partials:
        N = (Hq + 2 * Hkv) * D
        inputs = dict(partials=(torch.randn(3, B, N, generator=g) * 0.5).to(DEV), num_q_heads=Hq)
    else:
        inputs = dict(q=torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(DEV),
                      k=torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16).to(DEV),
                      v=torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16).to(DEV))
    k0, v0 = lay.k.clone(), lay.v.clone()
    results = []
    for no_alloc in (False, True):
        lay.k.copy_(k0)
        lay.v.copy_(v0)
        lens = torch.full_like(pos, -1)
        out = torch.full((B, Hq, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        ws = None if no_alloc else ops.Workspace(DEV)
        ops.decode_attention_append(table, pos, lay, max_len, lens_out=lens, out=out, workspace=ws,
                                    no_alloc=no_alloc, **inputs)
        torch.cuda.synchronize()
        results.append((out.clone(), lay.k.clone(), lay.v.clone(), lens.clone()))
    return results


def _assert_same(a, b, what):
    for x, y, name in zip(a, b, ("out", "k cache", "v cache", "lens")):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y), f"{what}: {name} differs"


@pytest.mark.parametrize("paged,D,Hq,Hkv,from_partials", [
    (True, 128, 32, 8, False),
    (False, 64, 32, 8, True),
    (True, 64, 16, 1, True),
])
def test_noalloc_step_equals_workspace_step_twice(paged, D, Hq, Hkv, from_partials):
    print(f"\nno-alloc step: paged={paged} D={D} Hq={Hq} Hkv={Hkv} partials={from_partials}", flush=True)
    big = [1, 17, 300, 1030, 64, 513, 5, 777] * 4          # 32 sequences
    small = [3, 129, 40, 16, 900]                             # then 5 shorter ones
    for i, lens in enumerate((big, small)):
        layer, table, g = _layer(paged, D, Hq, Hkv, lens, seed=10 + i)
        ref, got = _step_both(layer, table, g, Hq, from_partials)
        assert torch.isfinite(ref[0].float()).all()
        _assert_same(ref, got, f"call {i + 1} (B={len(lens)})")
        assert torch.equal(got[3].cpu(), torch.tensor(lens, dtype=torch.int32) + 1)


def test_noalloc_refuses_a_workspace_beyond_the_scratch():
    """B 1024, 128 / 8 heads, D 128: (8192 + waves) * 16 * 130 * 4 bytes of
    partials exceed the 32 MiB scratch; the call raises before any launch and
    leaves the cache and out untouched."""
    from tinytron_amd import _lib, ops

    B, Hq, Hkv, D, P = 1024, 128, 8, 128, 16
    table = torch.arange(B, dtype=torch.int32, device=DEV).view(B, 1)
    lay = ops.KVLayout(k=torch.zeros(B * Hkv * P * D, dtype=torch.bfloat16, device=DEV),
                       v=torch.zeros(B * Hkv * P * D, dtype=torch.bfloat16, device=DEV),
                       strides=(0, Hkv * P * D, P * D), num_heads=Hkv, head_dim=D, page_size=P, capacity=P,
                       kind="bf16", page_table=table, num_pages=B)
    rope = ops.build_rope_table(P, D, device=DEV)
    pos = torch.zeros(B, dtype=torch.int32, device=DEV)
    q = torch.ones(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    kv = torch.ones(B, Hkv, D, dtype=torch.bfloat16, device=DEV)
    out = torch.full((B, Hq, D), 7.0, dtype=torch.bfloat16, device=DEV)
    need = 16 * 8 * B * (D + 2) * 4
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="smaller than"):
        ops.decode_attention_append(rope, pos, lay, 1, q=q, k=kv, v=kv, out=out, no_alloc=True)
    torch.cuda.synchronize()
    assert not lay.k.any() and (out == 7.0).all()
