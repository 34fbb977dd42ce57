"""GPU parity: fused RoPE + KV append vs the CPU oracle, bit for bit.

Covers the reference's contiguous LayerPagedKVCache layout (cache.py:27-42)
and the paged pool, bf16 / fp32 / fp8-e4m3fn caches, ragged positions, T > 1
with ragged new_lens, strided (transposed-view) inputs as Attention.forward
produces them (attn.py:389-391), and untouched slots staying untouched.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import kvcache as okv
from oracle.numerics import (bf16_bits_to_f32, f32_to_bf16_bits, quantize_e4m3_rows)
from oracle.rope import rope_apply
from tests.kv_inputs import bf16_randn, contiguous_geometry, paged_geometry

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _to_dev_bf16(bits: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def _bits(t: "torch.Tensor") -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(kind, paged, D, T, seed, Hq=8, Hkv=2, P=16, ragged_new=False, from_partials=False):
    from tinytron_amd import ops

    rng = np.random.default_rng(seed)
    B = 3
    positions = np.array([5, 17, 0], dtype=np.int32)
    new_lens = np.array([T, max(1, T - 1), T], dtype=np.int32) if ragged_new else np.full(B, T, np.int32)
    cap_needed = positions + T
    max_seq = 64
    act = torch.float32 if kind == "f32" else torch.bfloat16
    if paged:
        layout, numel, ptab, num_pages = paged_geometry(cap_needed + 7, Hkv, D, P, rng)
    else:
        layout, numel = contiguous_geometry(B, Hkv, D, max_seq, P, fp8=kind == "fp8")
    # inputs laid out [B, T, H, D] and viewed [B, H, T, D] as q_proj(x).view().transpose() gives
    qb, qf = bf16_randn(rng, (B, T, Hq, D))
    kb, kf = bf16_randn(rng, (B, T, Hkv, D))
    vb, vf = bf16_randn(rng, (B, T, Hkv, D))
    if kind == "f32":
        qf = rng.standard_normal((B, T, Hq, D)).astype(np.float32)
        kf = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
        vf = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
        q = torch.from_numpy(qf).to(DEV)
        k = torch.from_numpy(kf).to(DEV)
        v = torch.from_numpy(vf).to(DEV)
    else:
        q, k, v = _to_dev_bf16(qb), _to_dev_bf16(kb), _to_dev_bf16(vb)
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if from_partials:
        # q|k|v as 3 fp32 split-K partials [S, B, (Hq + 2 Hkv) D]; the inputs the
        # oracle sees are bf16(partial 0 + partial 1 + partial 2), added in order
        assert T == 1 and kind != "f32"
        N = (Hq + 2 * Hkv) * D
        parts = (rng.standard_normal((3, B, N)) * 1.5).astype(np.float32)
        tot = (parts[0] + parts[1]) + parts[2]
        proj = bf16_bits_to_f32(f32_to_bf16_bits(tot)).reshape(B, 1, N)
        qf = proj[:, :, :Hq * D].reshape(B, 1, Hq, D)
        kf = proj[:, :, Hq * D:(Hq + Hkv) * D].reshape(B, 1, Hkv, D)
        vf = proj[:, :, (Hq + Hkv) * D:].reshape(B, 1, Hkv, D)
    table = ops.build_rope_table(128, D, dtype=act, device=DEV)
    table_np = table.float().cpu().numpy()

    sentinel16 = np.uint16(0x7FC1)
    if kind == "fp8":
        k_store = torch.full((numel,), 0x7E, dtype=torch.uint8, device=DEV)
        v_store = torch.full((numel,), 0x7E, dtype=torch.uint8, device=DEV)
        k_scale = torch.full((okv.fp8_scale_numel(numel // D),), -1.0, dtype=torch.float32, device=DEV)
        v_scale = k_scale.clone()
    elif kind == "bf16":
        k_store = torch.full((numel,), int(sentinel16.view(np.int16)), dtype=torch.int16, device=DEV).view(torch.bfloat16)
        v_store = k_store.clone()
        k_scale = v_scale = None
    else:
        k_store = torch.full((numel,), -7.0, dtype=torch.float32, device=DEV)
        v_store = k_store.clone()
        k_scale = v_scale = None
    dev_table = None if not paged else torch.from_numpy(ptab).to(DEV)
    kv = ops.KVLayout(
        k=k_store, v=v_store, strides=(layout.seq_stride, layout.page_stride, layout.head_stride),
        num_heads=Hkv, head_dim=D, page_size=P, capacity=layout.capacity if paged else max_seq,
        kind=kind, page_table=dev_table, num_pages=(num_pages if paged else 0),
        k_scale=k_scale, v_scale=v_scale,
    )
    pos_t = torch.from_numpy(positions).to(DEV)
    nl_t = torch.from_numpy(new_lens).to(DEV) if ragged_new else None
    if from_partials:
        q_out = ops.rope_append_partials(torch.from_numpy(parts).to(DEV), Hq, table, pos_t, kv)
    else:
        q_out = ops.rope_append(q, k, v, table, pos_t, kv, new_lens=nl_t)
    torch.cuda.synchronize()

    # ---- oracle ----
    dt = "f32" if kind == "f32" else "bf16"
    pos_bt = positions[:, None] + np.arange(T)[None, :]
    rows = table_np[pos_bt]  # [B, T, D]
    q_ref = rope_apply(qf, rows[:, :, None, :], dt)        # [B, T, Hq, D]
    k_ref = rope_apply(kf, rows[:, :, None, :], dt)
    v_ref = vf
    # q_out: every token (new_lens only limits the cache write)
    q_dev = q_out.float().cpu().numpy().transpose(0, 2, 1, 3)
    if kind == "f32":
        assert np.array_equal(q_dev.view(np.uint32), q_ref.view(np.uint32))
    else:
        assert np.array_equal(_bits(q_out).transpose(0, 2, 1, 3), f32_to_bf16_bits(q_ref))

    if kind == "fp8":
        exp_k = np.full(numel, 0x7E, np.uint8)
        exp_v = np.full(numel, 0x7E, np.uint8)
        exp_ks = np.full(okv.fp8_scale_numel(numel // D), -1.0, np.float32)
        exp_vs = exp_ks.copy()
        okv.append_fp8(exp_k, exp_ks, layout, k_ref.transpose(0, 2, 1, 3), positions, new_lens)
        okv.append_fp8(exp_v, exp_vs, layout, v_ref.transpose(0, 2, 1, 3), positions, new_lens)
        got_k = k_store.cpu().numpy()
        got_v = v_store.cpu().numpy()
        assert np.array_equal(got_k, exp_k), f"k codes differ at {np.flatnonzero(got_k != exp_k)[:8]}"
        assert np.array_equal(got_v, exp_v)
        assert np.array_equal(k_scale.cpu().numpy().view(np.uint32), exp_ks.view(np.uint32))
        assert np.array_equal(v_scale.cpu().numpy().view(np.uint32), exp_vs.view(np.uint32))
    elif kind == "bf16":
        exp_k = np.full(numel, sentinel16, np.uint16)
        exp_v = np.full(numel, sentinel16, np.uint16)
        okv.append(exp_k, layout, f32_to_bf16_bits(k_ref).transpose(0, 2, 1, 3), positions, new_lens)
        okv.append(exp_v, layout, f32_to_bf16_bits(v_ref).transpose(0, 2, 1, 3), positions, new_lens)
        assert np.array_equal(_bits(k_store), exp_k), f"k differs at {np.flatnonzero(_bits(k_store) != exp_k)[:8]}"
        assert np.array_equal(_bits(v_store), exp_v)
    else:
        exp_k = np.full(numel, -7.0, np.float32)
        exp_v = np.full(numel, -7.0, np.float32)
        okv.append(exp_k, layout, k_ref.transpose(0, 2, 1, 3), positions, new_lens)
        okv.append(exp_v, layout, v_ref.transpose(0, 2, 1, 3), positions, new_lens)
        assert np.array_equal(k_store.cpu().numpy().view(np.uint32), exp_k.view(np.uint32))
        assert np.array_equal(v_store.cpu().numpy().view(np.uint32), exp_v.view(np.uint32))


@pytest.mark.parametrize("kind", ["bf16", "fp8", "f32"])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_append_decode(kind, paged, D):
    _case(kind, paged, D, T=1, seed=11 + D)


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
@pytest.mark.parametrize("paged", [False, True])
def test_rope_append_prefill_ragged(kind, paged):
    _case(kind, paged, 128, T=9, seed=5, ragged_new=True)


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_append_from_split_k_partials(kind, paged, D):
    """q|k|v taken from the stacked projection's fp32 split-K partials: the
    kernel's in-order sum rounded to bf16 gives the same rotated q and cache
    bytes as the oracle on those rounded values."""
    _case(kind, paged, D, 1, seed=300 + D + paged, from_partials=True)


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_rope_append_packed_rows_equal_grid(kind, paged, D):
    """Packed prompt rows (no padding: token t of sequence b is row
    row_offsets[b] + t) give the same cache bytes, fp8 scales, lengths and
    rotated q rows t < new_lens[b] as the [B, H, T, D] grid path pinned to the
    oracle above; a sequence with no new tokens and sequences with tokens
    already cached included."""
    packed_vs_grid(kind, paged, D, Hq=8, Hkv=2, new=[21, 3, 0, 1, 17], pre=[0, 5, 9, 0, 30], seed=D + 2 * paged)


def packed_vs_grid(kind, paged, D, Hq, Hkv, new, pre, seed, page=16):
    """rope_append_rows on packed rows against rope_append on the [B, H, T, D]
    grid of the same tokens: cache bytes, scales, lengths, rotated q rows."""
    from tinytron_amd import ops
    from tinytron_amd.cache import PagedKVCache
    from tinytron_amd.model import ModelConfig

    B, T = len(new), max(max(new), 1)
    cap = ((max(p + n for p, n in zip(pre, new)) + 8 + page - 1) // page) * page
    cfg = ModelConfig(num_layer=1, hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      block_size=cap)
    kvd = torch.float8_e4m3fn if kind == "fp8" else None
    g = torch.Generator().manual_seed(seed)
    layers = []
    for _ in range(2):
        cache = PagedKVCache.from_model_config(cfg, B, page, DEV, torch.bfloat16, kv_cache_dtype=kvd, paged_pool=paged,
                                               seq_capacity=[cap] * B)
        layer = cache.get_layer_cache(0)
        layer.set_lengths(pre)
        layers.append(layer)
    lay_a, lay_b = layers[0].layout, layers[1].layout
    for x, y in ((lay_a.k, lay_b.k), (lay_a.v, lay_b.v)):  # same bytes in the never-written slots
        r = torch.randint(0, 256, (x.numel() * x.element_size(),), generator=g, dtype=torch.uint8).to(DEV)
        x.view(torch.uint8).copy_(r)
        y.view(torch.uint8).copy_(r)
    if kind == "fp8":
        for x, y in ((lay_a.k_scale, lay_b.k_scale), (lay_a.v_scale, lay_b.v_scale)):
            x.fill_(-1.0)
            y.fill_(-1.0)
    qg = torch.randn(B, T, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    kg = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    vg = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    table = ops.build_rope_table(cap + T, D, device=DEV)
    q_grid = layers[0].rope_append(qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2), table, new_lens=new)
    qp, kp, vp = (torch.cat([t[b, :n] for b, n in enumerate(new)]) for t in (qg, kg, vg))
    offs = torch.tensor(np.cumsum([0] + new[:-1]), dtype=torch.int32, device=DEV)
    q_rows = layers[1].rope_append_rows(qp, kp, vp, table, new, offs, T)
    torch.cuda.synchronize()
    assert layers[0].seq_lens_host == layers[1].seq_lens_host == [p + n for p, n in zip(pre, new)]
    assert torch.equal(layers[0].seq_lens, layers[1].seq_lens)
    for x, y in ((lay_a.k, lay_b.k), (lay_a.v, lay_b.v)):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), "cache bytes differ"
    if kind == "fp8":
        assert torch.equal(lay_a.k_scale, lay_b.k_scale) and torch.equal(lay_a.v_scale, lay_b.v_scale)
    for b, n in enumerate(new):
        assert torch.equal(q_grid[b, :, :n].view(torch.int16), q_rows[b, :, :n].view(torch.int16)), f"q of sequence {b}"


def test_rope_table_matches_closed_form():
    """The table is an input of the bit-exact RoPE; its values follow the
    reference's fp32 op sequence, so they sit within fp32 angle rounding
    (pos * f * 2^-23, from pow and the product) of the fp64 closed form, and
    within the same bound of the numpy oracle's table."""
    from tinytron_amd import ops
    from oracle.rope import rope_table

    D, n = 128, 4096
    t = ops.build_rope_table(n, D, dtype=torch.float32, device=DEV).cpu().numpy()
    ref = rope_table(n, D, dtype="f32")
    pos = np.arange(n, dtype=np.float64)[:, None]
    inv = 1.0 / (10000.0 ** (np.arange(0, D, 2) / D))
    exact = np.concatenate([np.cos(pos * inv), np.sin(pos * inv)], -1)
    bound = np.concatenate([pos * inv, pos * inv], -1) * 2.0 ** -21 + 2e-7
    assert np.all(np.abs(t - exact) <= bound)
    assert np.all(np.abs(ref - exact) <= bound)
    bf = ops.build_rope_table(n, D, dtype=torch.bfloat16, device=DEV).float().cpu().numpy()
    assert np.all(np.abs(bf - exact) <= bound + np.abs(exact) * 2.0 ** -8)
