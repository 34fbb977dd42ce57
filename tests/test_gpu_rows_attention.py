"""GPU parity: row attention (tt_rows_attn_*, the VALU kernel with a row ->
sequence map) vs the fp64 oracle.

Row r attends to the first row_lens[r] cached tokens of sequence
seq_of_row[r]; rows of a prefill chunk (row_lens = cached + t + 1) give the
reference's cache-causal prefill attention (attn.py:321-341) for fp32 caches
and for head dims whose rows are not whole 16-byte fragments, which the
prefill kernel does not take. Tolerance as for decode attention:
|out - ref| <= 2e-3 + 2e-2 |ref| (bf16 / fp8 caches; fp32 caches 1e-5 +
1e-4 |ref|). Caches are NaN outside the written tokens, so a read past a
row's length shows.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle.attention import decode_attention as ref_decode
from oracle.attention import prefill_attention as ref_prefill
from tests.kv_inputs import bf16_randn, contiguous_geometry, fill_cache_values, paged_geometry, sm_scale

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(arr, dtype):
    if dtype == torch.bfloat16:
        return torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(DEV)


def _cache(lengths, Hkv, D, kind, paged, rng, P=16):
    """A cache holding lengths[b] random tokens per sequence (NaN elsewhere):
    (KVLayout, fp32 keys / values per sequence as the kernels read them)."""
    from tinytron_amd import ops

    lengths = np.asarray(lengths, np.int32)
    B = len(lengths)
    cap = max(int(((lengths.max() + P - 1) // P) * P), P)
    if paged:
        layout, numel, ptab, num_pages = paged_geometry(np.maximum(lengths, 1), Hkv, D, P, rng)
    else:
        layout, numel = contiguous_geometry(B, Hkv, D, cap, P)
    if kind == "f32":
        keys = [rng.standard_normal((int(L), Hkv, D)).astype(np.float32) for L in lengths]
        values = [rng.standard_normal((int(L), Hkv, D)).astype(np.float32) for L in lengths]
        ks = np.full(numel, np.nan, np.float32)
        vs = np.full(numel, np.nan, np.float32)
        for b, L in enumerate(lengths):
            offs = layout.token_offsets(b, int(L))
            idx = (offs[..., None] + np.arange(D, dtype=np.int64)).reshape(-1)
            ks[idx] = keys[b].reshape(-1)
            vs[idx] = values[b].reshape(-1)
        k_store, v_store = _dev(ks, None), _dev(vs, None)
        data = {"keys": keys, "values": values}
    else:
        data = fill_cache_values(layout, numel, B, lengths, rng, fp8=kind == "fp8")
        tdt = None if kind == "fp8" else torch.bfloat16
        k_store, v_store = _dev(data["k_store"], tdt), _dev(data["v_store"], tdt)
    kv = ops.KVLayout(
        k=k_store, v=v_store, strides=(layout.seq_stride, layout.page_stride, layout.head_stride),
        num_heads=Hkv, head_dim=D, page_size=P, capacity=int(layout.capacity), kind=kind,
        page_table=(torch.from_numpy(ptab).to(DEV) if paged else None), num_pages=(num_pages if paged else 0),
        k_scale=(_dev(data["k_scale"], None) if kind == "fp8" else None),
        v_scale=(_dev(data["v_scale"], None) if kind == "fp8" else None))
    return kv, data["keys"], data["values"]


def _queries(rng, shape, kind):
    if kind == "f32":
        qf = rng.standard_normal(shape).astype(np.float32)
        return _dev(qf, None), qf
    qb, qf = bf16_randn(rng, shape)
    return _dev(qb, torch.bfloat16), qf


def _check(got, ref, kind):
    rtol, atol = (1e-4, 1e-5) if kind == "f32" else (2e-2, 2e-3)
    assert np.all(np.isfinite(got)), "non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} out of tolerance; max err {err.max():.3e}"


@pytest.mark.parametrize("kind,D", [("f32", 64), ("f32", 30), ("f32", 128), ("bf16", 30), ("bf16", 18),
                                    ("bf16", 64), ("fp8", 40), ("fp8", 64)])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (6, 2), (8, 2)])
def test_rows_vs_oracle(kind, D, paged, Hq, Hkv):
    """Rows over a ragged cache: each row reads a random prefix (0 .. L_b
    tokens, zero-length rows give zeros) of a random sequence."""
    from tinytron_amd import ops

    rng = np.random.default_rng(sum(map(ord, kind)) * 1000 + D * 10 + int(paged) + 7 * Hq)
    lengths = [1, 17, 300, 64, 129]
    kv, keys, values = _cache(lengths, Hkv, D, kind, paged, rng)
    R = 23
    seq = rng.integers(0, len(lengths), R).astype(np.int32)
    lens = np.array([rng.integers(0, lengths[s] + 1) for s in seq], np.int32)
    lens[0] = 0
    lens[1] = lengths[seq[1]]
    q, qf = _queries(rng, (R, Hq, D), kind)
    out = ops.rows_attention(q, kv, _dev(seq, None), _dev(lens, None), int(lens.max()), len(lengths))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = ref_decode(qf, [keys[s][:n] for s, n in zip(seq, lens)], [values[s][:n] for s, n in zip(seq, lens)], Hkv,
                     sm_scale(D))
    assert np.all(got[0] == 0.0)
    _check(got, ref, kind)


@pytest.mark.parametrize("kind,D", [("f32", 64), ("bf16", 30), ("fp8", 48)])
@pytest.mark.parametrize("paged", [False, True])
def test_prefill_rows_vs_oracle(kind, D, paged, monkeypatch):
    """prefill_attention_rows over a partly cached ragged chunk (cached[b]
    tokens before it, new[b] after) against the oracle's causal prefill; the
    launch cap is lowered so the chunk also runs as several launches."""
    from tinytron_amd import ops

    rng = np.random.default_rng(7 + D + paged)
    cached, new = [0, 40, 5, 100], [30, 1, 17, 0]
    T, Hq, Hkv = max(new), 6, 2
    kv, keys, values = _cache([c + n for c, n in zip(cached, new)], Hkv, D, kind, paged, rng)
    q, qf = _queries(rng, (len(cached), Hq, T, D), kind)
    ref = ref_prefill(qf, keys, values, cached, new, Hkv, sm_scale(D))
    for cap in (ops.ROWS_ATTN_MAX_ROWS, 7):
        monkeypatch.setattr(ops, "ROWS_ATTN_MAX_ROWS", cap)
        out = ops.prefill_attention_rows(q, kv, cached, new)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        for b, n in enumerate(new):
            assert np.all(got[b, n:] == 0.0)
        _check(got, ref, kind)


def test_rows_reject_bad_arguments():
    """Host-side validation: a missing row map and a zero sequence count are
    refused before any launch."""
    from tinytron_amd import _lib, ops

    rng = np.random.default_rng(3)
    kv, _, _ = _cache([5, 9], 2, 64, "bf16", False, rng)
    q, _ = _queries(rng, (3, 4, 64), "bf16")
    seq = torch.zeros(3, dtype=torch.int32, device=DEV)
    lens = torch.ones(3, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="num_seqs"):
        ops.rows_attention(q, kv, seq, lens, 1, 0)
    lib = _lib.load()
    st = lib.tt_rows_attn_bf16(q.data_ptr(), _lib.strides(*q.stride()[:2]), kv.k.data_ptr(), kv.v.data_ptr(),
                               _lib.strides(*kv.strides), None, lens.data_ptr(), 1, None, 0, 0, 2, q.data_ptr(),
                               _lib.strides(*q.stride()[:2]), 3, 4, 2, 64, 16, 0.125, None, 0, None)
    assert st == _lib.TT_ERR_INVALID_ARGUMENT
