"""GPU parity at the benchmark's full sizes (C2, C3, C4 and one C5 layer), where
the fp64 oracle over the whole batch would take minutes, through properties
that hold at any size. The workload is bench.py's own (same builder, seed and
step calls), so what the bench times is what is checked here.

* Cache indexing, bit-exact: the step's RoPE + append changes exactly the
  appended slot of every (sequence, KV head), located with the oracle's slot
  formula (oracle.kvcache.CacheLayout over the same page table), and writes
  there the oracle's rotated k (bf16 rounding in the reference's op order) and
  v, or their e4m3 codes and per-(token, head) scales. Every other byte of the
  pool is unchanged.
* The rotated query rows equal the oracle's, bit for bit.
* Attention: every output is finite, and sampled segments (the longest, the
  shortest and random ones), gathered back from the pool with the oracle's
  slot formula, match the fp64 oracle within |out - ref| <= 2e-3 + 2e-2 |ref|
  (fp8: the oracle on the dequantised values).
* Partition invariance: the balanced partition (an equal run of tiles per
  wave, merged per segment) and the fixed-split kernel (other split points,
  other merge order) agree over all B x H_q rows within the same tolerance.
* The fused step (RoPE + append inside the attention launch) equals the
  two-launch step bit for bit: output, pool bytes and lengths.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import bench
from oracle.attention import decode_attention as ref_attention
from oracle import kvcache as okv
from oracle.kvcache import CacheLayout
from oracle.numerics import dequantize_e4m3_rows, f32_to_bf16_bits, quantize_e4m3_rows
from oracle.rope import rope_apply
from tests.kv_inputs import sm_scale

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL, ATOL = 2e-2, 2e-3
SEED = 1337  # bench.py's default


def _assert_close(got, ref, what):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} out of tolerance; max err {err.max():.3e}"


def _oracle_layout(cfg, lay):
    table = lay.page_table.cpu().numpy() if lay.page_table is not None else None
    s = lay.strides
    return CacheLayout(num_heads=cfg["hkv"], head_dim=cfg["head_dim"], page_size=cfg["page"], seq_stride=s[0],
                       page_stride=s[1], head_stride=s[2], page_table=table, capacity=lay.capacity)


def _pool(lay):
    ts = [lay.k, lay.v] + ([lay.k_scale, lay.v_scale] if lay.kind == "fp8" else [])
    return [t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t for t in ts]


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32) if t.element_size() == 4 else t


def _gather(store, olay, b, length):
    """[length, H, D] of sequence b through the oracle's slot formula."""
    D = olay.head_dim
    offs = torch.from_numpy(olay.token_offsets(b, length)).to(DEV)
    return store[offs[..., None] + torch.arange(D, device=DEV)]


def _expected_append(cfg, wl):
    """Oracle's rotated k / v rows [B, H_kv, D] of the step's token and the rotated q."""
    rows = wl["rope"].float().cpu().numpy()[wl["ctx"].numpy()]  # [B, D] at positions
    q = wl["q_in"][:, :, 0].float().cpu().numpy()
    k = wl["k_in"][:, :, 0].float().cpu().numpy()
    v = wl["v_in"][:, :, 0].float().cpu().numpy()
    q_rot = rope_apply(q, rows[:, None, :])
    k_rot = rope_apply(k, rows[:, None, :])
    return q_rot, k_rot, v


def _check_append(cfg, wl, olay, before, after):
    B, hkv, D = cfg["batch"], cfg["hkv"], cfg["head_dim"]
    _, k_rot, v = _expected_append(cfg, wl)
    pos = wl["ctx"].numpy()
    offs = np.array([[olay.token_offset(b, h, int(pos[b])) for h in range(hkv)] for b in range(B)], np.int64)
    elems = torch.from_numpy((offs[..., None] + np.arange(D)).reshape(-1)).to(DEV)
    if cfg["fp8"]:
        kc, ks = quantize_e4m3_rows(k_rot)
        vc, vs = quantize_e4m3_rows(v)
        want = [kc.reshape(-1), vc.reshape(-1)]
        want_s = [ks.reshape(-1), vs.reshape(-1)]
        rows = torch.from_numpy(okv.fp8_scale_index(offs // D).reshape(-1)).to(DEV)
    else:
        want = [f32_to_bf16_bits(k_rot).reshape(-1).view(np.int16), f32_to_bf16_bits(v).reshape(-1).view(np.int16)]
    for i in range(2):
        a, z = _bits(after[i]), _bits(before[i])
        changed = torch.nonzero(a != z).flatten()
        assert torch.isin(changed, elems).all(), f"pool {i}: {int((~torch.isin(changed, elems)).sum())} bytes " \
                                                 "changed outside the appended slots"
        got = a[elems].cpu().numpy()
        assert np.array_equal(got, want[i]), f"pool {i}: appended slot differs from the oracle " \
                                             f"({int((got != want[i]).sum())} elements)"
    if cfg["fp8"]:
        for i in range(2):
            a, z = after[2 + i], before[2 + i]
            changed = torch.nonzero(_bits(a) != _bits(z)).flatten()
            # the K and V views share one array (V 16 slots in): the other view's writes show 16 slots away
            slots = torch.cat([rows, rows + 16, rows - 16])
            assert torch.isin(changed, slots).all(), "scale written outside the appended slots"
            assert np.array_equal(a[rows].cpu().numpy(), want_s[i]), "appended scales differ from the oracle"


def _sampled(total, rng, n_random=2):
    t = total.numpy()
    picks = [int(np.argmax(t)), int(np.argmin(t))] + [int(x) for x in rng.choice(len(t), n_random, replace=False)]
    return sorted(set(picks))


@pytest.mark.parametrize("config", ["c3", "c4", "c2", "c5a"])
def test_full_size_step(config):
    from tinytron_amd import ops

    cfg = bench.CONFIGS[config]
    B, hq, hkv, D = cfg["batch"], cfg["hq"], cfg["hkv"], cfg["head_dim"]
    print(f"full-size step {config}: B {B}, {hq}/{hkv} heads, D {D}, fp8 {cfg['fp8']}", flush=True)
    wl = bench.build_workload(cfg, SEED, torch, ops)
    lay = wl["layout"]
    olay = _oracle_layout(cfg, lay)
    before = [t.clone() for t in _pool(lay)]

    # two-launch step: RoPE + append, then attention over positions + 1
    lens_a = torch.full_like(wl["positions"], -1)
    q_rot = ops.rope_append(wl["q_in"], wl["k_in"], wl["v_in"], wl["rope"], wl["positions"], lay, lens_out=lens_a)
    ws = ops.Workspace(DEV)
    out = ops.decode_attention(q_rot.view(B, hq, D), lay, wl["seq_lens"], wl["max_len"], workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(lens_a, wl["seq_lens"])
    after = [t.clone() for t in _pool(lay)]

    # cache indexing and the rotated q, bit-exact against the oracle
    _check_append(cfg, wl, olay, before, after)
    q_ref, _, _ = _expected_append(cfg, wl)
    assert np.array_equal(_bits(q_rot).cpu().numpy().reshape(B, hq, D), f32_to_bf16_bits(q_ref).view(np.int16))

    # sampled segments against the fp64 oracle over the pool's own bytes
    got = out.float().cpu().numpy()
    assert np.all(np.isfinite(got)), "non-finite attention output"
    qf = q_rot.float().cpu().numpy().reshape(B, hq, D)
    total = wl["total"]
    for b in _sampled(total, np.random.default_rng(7)):
        L = int(total[b])
        if cfg["fp8"]:
            kc, vc = _gather(lay.k.view(torch.uint8), olay, b, L), _gather(lay.v.view(torch.uint8), olay, b, L)
            rows = torch.from_numpy(okv.fp8_scale_index(olay.token_offsets(b, L) // D)).to(DEV)
            keys = dequantize_e4m3_rows(kc.cpu().numpy(), lay.k_scale[rows].cpu().numpy())
            values = dequantize_e4m3_rows(vc.cpu().numpy(), lay.v_scale[rows].cpu().numpy())
        else:
            keys = _gather(lay.k, olay, b, L).float().cpu().numpy()
            values = _gather(lay.v, olay, b, L).float().cpu().numpy()
        ref = ref_attention(qf[b:b + 1], [keys], [values], hkv, sm_scale(D))
        _assert_close(got[b:b + 1], ref, f"sequence {b} (L {L})")

    # partition invariance over every row
    fixed = ops.decode_attention(q_rot.view(B, hq, D), lay, wl["seq_lens"], wl["max_len"], split_tokens=1024,
                                 workspace=ws)
    _assert_close(got, fixed.float().cpu().numpy(), "balanced vs fixed split")

    # the fused step from the same starting pool
    for t, s in zip(_pool(lay), before):
        t.copy_(s)
    lens_b = torch.full_like(wl["positions"], -1)
    out_f = ops.decode_attention_append(wl["rope"], wl["positions"], lay, wl["max_len"], q=wl["q_in"][:, :, 0],
                                        k=wl["k_in"][:, :, 0], v=wl["v_in"][:, :, 0], lens_out=lens_b,
                                        workspace=ops.Workspace(DEV))
    torch.cuda.synchronize()
    assert torch.equal(lens_b, lens_a)
    assert torch.equal(_bits(out_f), _bits(out)), "fused step output differs from the two-launch step"
    for x, y in zip(_pool(lay), after):
        assert torch.equal(_bits(x), _bits(y)), "fused step pool bytes differ from the two-launch step"
