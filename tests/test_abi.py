"""The C ABI library: loads, exports every symbol include/tinytron_amd.h
declares, reports its version, sizes workspaces, and rejects invalid
arguments with the documented status codes before launching anything.

These tests make no compute call. The argument-rejection cases pass fake
(non-dereferenced) device pointers, so they run only where no GPU is
visible: every case must fail validation, and none may ever launch.
"""
import ctypes
import re
from pathlib import Path

import pytest

from tinytron_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "tinytron_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tt_[a-z0-9_]+)\s*\(", text)))


def _no_gpu():
    try:
        import torch

        return not torch.cuda.is_available()
    except Exception:
        return True


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"


def test_decode_layer_struct_matches_header(tmp_path):
    """The ctypes tt_decode_layer_t has the C struct's size and field offsets
    (compiled from the header with the host C compiler)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    fields = [f[0] for f in _lib.DecodeLayer._fields_]
    src = tmp_path / "layout.c"
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"tinytron_amd.h\"\nint main(void) {\n"
                   "  printf(\"%zu\\n\", sizeof(tt_decode_layer_t));\n"
                   + "".join(f"  printf(\"%zu\\n\", offsetof(tt_decode_layer_t, {f}));\n" for f in fields)
                   + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    want = [ctypes.sizeof(_lib.DecodeLayer)] + [getattr(_lib.DecodeLayer, f).offset for f in fields]
    assert got == want


def test_decode_layers_validates_before_launching():
    """tt_decode_layers_bf16: no layers is a no-op; a NULL array, a bad
    k_chunk and a NULL buffer are refused, the message naming the layer and
    the step (every case fails validation before any launch)."""
    lib = _lib.load()
    assert lib.tt_decode_layers_bf16(None, 0, 1, None) == _lib.TT_OK
    assert lib.tt_decode_layers_bf16(None, 1, 1, None) == _lib.TT_ERR_INVALID_ARGUMENT
    arr = (_lib.DecodeLayer * 1)()
    assert lib.tt_decode_layers_bf16(ctypes.addressof(arr), 1, 1, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert b"layer 0: bad k_chunk" in lib.tt_last_error_string()
    arr[0].kc_qkv = arr[0].kc_o = arr[0].kc_down = 256
    assert lib.tt_decode_layers_bf16(ctypes.addressof(arr), 1, 1, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert lib.tt_last_error_string().startswith(b"layer 0, q|k|v: ")


def test_noalloc_scratch_size_matches_header():
    m = re.search(r"#define TT_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", HEADER.read_text())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES


def test_abi_version():
    assert _lib.load().tt_abi_version() == _lib.ABI_VERSION == 7


def test_workspace_and_split_sizing():
    lib = _lib.load()
    # C3: B 64, 32/8 heads, D 128, longest sequence 16385 tokens
    split = lib.tt_decode_split_tokens(64, 8, 16385)
    assert split in (128, 256, 512, 1024)
    nbytes = lib.tt_decode_workspace_bytes(64, 32, 8, 128, 16385, split)
    splits = -(-16385 // split)
    assert nbytes == 64 * 8 * splits * 4 * (128 + 2) * 4
    assert lib.tt_decode_workspace_bytes(0, 32, 8, 128, 100, 0) == 0
    # per segment: what the VALU kernel's automatic split needs (the MFMA kernels need none)
    assert lib.tt_decode_workspace_bytes(64, 32, 8, 128, 16385, -1) == nbytes


def _pick(lib, lens, hkv, head_dim, fp8=0):
    arr = (ctypes.c_int32 * max(len(lens), 1))(*lens)
    return lib.tt_decode_pick_split(ctypes.addressof(arr), len(lens), hkv, head_dim, fp8)


@pytest.mark.skipif(not _no_gpu(), reason="the resident round is 256 workgroups per tile round only on the stand-in")
def test_pick_split():
    """Equal lengths: per segment (-1) for MFMA head dims and B * H_kv a
    multiple of the resident round (256 CUs here: one workgroup per CU at tile
    width 128, two at 64 and 32). Ragged lengths: paired (-2) for B <= 256,
    (B + 1) / 2 * H_kv a multiple of the CUs, and no rank pair's line (tiles +
    2 per segment) above 1.06 times the pairs' mean; else balanced (0)."""
    lib = _lib.load()
    assert _pick(lib, [4096] * 32, 8, 128) == -1   # C2: 256 segments, D 128
    assert _pick(lib, [100] * 64, 8, 64) == -1     # 512 segments, D 64
    assert _pick(lib, [100] * 32, 8, 64) == 0      # 256 segments at D 64: half a round
    assert _pick(lib, [100] * 33, 8, 128) == 0
    assert _pick(lib, [100] * 64, 8, 96, 1) == -1  # fp8, padded tile 128
    assert _pick(lib, [100] * 64, 8, 24, 1) == 0   # fp8 rows not whole 16-byte fragments
    assert _pick(lib, [100] * 64, 8, 30) == 0      # VALU head_dim
    assert _pick(lib, [], 8, 128) == 0
    assert lib.tt_decode_pick_split(None, 64, 8, 128, 0) == 0
    # ragged: 32 long and 32 short sequences whose rank pairs (p, 63 - p) hold
    # 154 line positions each: long_i = 32 (100 + i) tokens (102 + i
    # positions), short_j = 32 (50 - j) tokens (52 - j)
    longs = [32 * (100 + i) for i in range(32)]
    shorts = [32 * (50 - j) for j in range(32)]
    even = longs + shorts
    assert _pick(lib, even, 8, 64) == -2            # 32 pairs x 8 heads = 256 workgroups
    assert _pick(lib, even[::-1], 8, 128) == -2     # order does not matter; D 128
    assert _pick(lib, even, 8, 64, 1) == -2         # fp8
    assert _pick(lib, even, 4, 64) == 0             # 128 workgroups: half the CUs
    assert _pick(lib, even, 16, 64) == -2           # 512: two rounds
    # the longest pair 8 positions heavier: 162 / (154 + 8 / 32) = 1.050 of the mean
    assert _pick(lib, longs[:-1] + [longs[-1] + 8 * 32] + shorts, 8, 64) == -2
    # 12 heavier: 166 / 154.375 = 1.075
    assert _pick(lib, longs[:-1] + [longs[-1] + 12 * 32] + shorts, 8, 64) == 0
    # odd batch: the middle rank alone (B 63: 32 workgroups x 8 heads)
    odd = [32 * (i + 1) for i in range(63)]        # pairs 68 positions, the middle rank 34 alone
    assert _pick(lib, odd, 8, 64) == -2             # 68 / ((31 x 68 + 34) / 32) = 1.016
    # two long sequences among short ones: pairs of 205 and of 6 positions
    assert _pick(lib, [32 * 200] * 2 + [32] * 62, 8, 64) == 0
    assert _pick(lib, [1] * 257, 8, 64) == 0 and _pick(lib, list(range(1, 258)), 8, 64) == 0  # B > 256


FAKE = 0x10000  # 16-byte aligned, never dereferenced: validation fails first


def _attn(lib, **kw):
    args = dict(q=FAKE, q_strides=(4096, 128), k=FAKE, v=FAKE, cache_strides=(0, 2048 * 8, 2048),
                seq_lens=FAKE, max_len=100, page_table=FAKE, max_pages=10, num_pages=100, out=FAKE,
                out_strides=(4096, 128), batch=2, hq=32, hkv=8, head_dim=128, page_size=16, sm_scale=0.088,
                split=0, ws=FAKE, ws_bytes=1 << 30)
    args.update(kw)
    a = args
    return lib.tt_gqa_decode_attn_bf16(
        a["q"], _lib.strides(*a["q_strides"]), a["k"], a["v"], _lib.strides(*a["cache_strides"]),
        a["seq_lens"], a["max_len"], a["page_table"], a["max_pages"], a["num_pages"], a["out"],
        _lib.strides(*a["out_strides"]), a["batch"], a["hq"], a["hkv"], a["head_dim"], a["page_size"],
        a["sm_scale"], a["split"], None, a["ws"], a["ws_bytes"], None)


@pytest.mark.skipif(not _no_gpu(), reason="fake-pointer validation cases run only without a GPU")
@pytest.mark.parametrize("kw,code,msg", [
    (dict(q=None), _lib.TT_ERR_INVALID_ARGUMENT, "NULL"),
    (dict(head_dim=136, q_strides=(4352, 136)), _lib.TT_ERR_UNSUPPORTED, "head_dim"),
    (dict(head_dim=7, q_strides=(224, 7)), _lib.TT_ERR_UNSUPPORTED, "head_dim"),
    (dict(hq=48, hkv=2), _lib.TT_ERR_UNSUPPORTED, "group size"),
    (dict(hq=30, hkv=8), _lib.TT_ERR_INVALID_ARGUMENT, "divisible"),
    (dict(split=300), _lib.TT_ERR_INVALID_ARGUMENT, "split_tokens"),
    (dict(split=-3), _lib.TT_ERR_INVALID_ARGUMENT, "split_tokens"),
    (dict(split=-2, batch=257), _lib.TT_ERR_UNSUPPORTED, "at most 256 sequences"),
    (dict(ws_bytes=16), _lib.TT_ERR_WORKSPACE_TOO_SMALL, "workspace"),
    (dict(page_size=24), _lib.TT_ERR_UNSUPPORTED, "power-of-two"),
    (dict(max_len=161), _lib.TT_ERR_INVALID_ARGUMENT, "exceeds the page table"),
    (dict(page_table=None, cache_strides=(1 << 20, 4096, 1 << 16)), _lib.TT_ERR_UNSUPPORTED, "dense pages"),
    (dict(q=FAKE + 2), _lib.TT_ERR_INVALID_ARGUMENT, "aligned"),
])
def test_attention_rejects_invalid_arguments(kw, code, msg):
    lib = _lib.load()
    assert _attn(lib, **kw) == code
    assert msg in lib.tt_last_error_string().decode()


@pytest.mark.skipif(not _no_gpu(), reason="fake-pointer validation cases run only without a GPU")
def test_fused_step_rejects_fixed_splits():
    """The fused decode step runs the balanced (0), per-segment (-1) or paired (-2) partition only."""
    lib = _lib.load()
    s2 = _lib.strides(512, 64)
    args = [FAKE, s2, FAKE, s2, FAKE, s2, 0, 0, FAKE, 100, FAKE, None, 50, None, 0, 0, FAKE, FAKE,
            _lib.strides(2 * 64 * 64, 16 * 64, 64 * 64), 64, FAKE, s2, 2, 8, 2, 64, 16, 0.125]
    assert lib.tt_decode_attn_append_bf16(*args, 512, None, FAKE, 1 << 30, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert "split_tokens" in lib.tt_last_error_string().decode()


@pytest.mark.skipif(not _no_gpu(), reason="fake-pointer validation cases run only without a GPU")
def test_rope_append_rejects_invalid_arguments():
    lib = _lib.load()
    s3 = _lib.strides(1, 1, 1)
    common = [FAKE, s3, FAKE, s3, FAKE, s3, FAKE, s3, FAKE, 100, FAKE, None, None, None, 0, 0, FAKE, FAKE]
    tail = [_lib.strides(0, 2048, 256), 64, 2, 1, 8, 2]
    # odd head_dim
    assert lib.tt_rope_append_bf16(*common, *tail, 127, 16, None) == _lib.TT_ERR_UNSUPPORTED
    # fp8 without scales
    assert lib.tt_rope_append_fp8(*common, None, None, *tail, 128, 16, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert "k_scale" in lib.tt_last_error_string().decode()
    # page_size 0 (the reference raises for page_size <= 0, cache.py:22-23)
    assert lib.tt_rope_append_bf16(*common, *tail, 128, 0, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert "page_size must be positive" in lib.tt_last_error_string().decode()
    # lens_out aliasing positions
    aliased = list(common)
    aliased[12] = FAKE
    assert lib.tt_rope_append_bf16(*aliased, *tail, 128, 16, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert "alias" in lib.tt_last_error_string().decode()
    # paged without pool size
    common_paged = list(common)
    common_paged[13] = FAKE
    assert lib.tt_rope_append_bf16(*common_paged, *tail, 128, 16, None) == _lib.TT_ERR_INVALID_ARGUMENT


@pytest.mark.skipif(not _no_gpu(), reason="fake-pointer validation cases run only without a GPU")
def test_prefill_row_entries_reject_invalid_arguments():
    lib = _lib.load()

    def err():
        return lib.tt_last_error_string().decode()

    # residual add + RMSNorm over prompt rows
    assert lib.tt_add_rmsnorm_rows_bf16(FAKE, FAKE, 2048, FAKE, 1e-6, FAKE, 10, 1002, None) == _lib.TT_ERR_UNSUPPORTED
    assert lib.tt_add_rmsnorm_rows_bf16(FAKE, FAKE, 9000, FAKE, 1e-6, FAKE, 10, 8196, None) == _lib.TT_ERR_UNSUPPORTED
    assert lib.tt_add_rmsnorm_rows_bf16(FAKE, FAKE, 1024, FAKE, 1e-6, FAKE, 10, 2048, None) == \
        _lib.TT_ERR_INVALID_ARGUMENT and "row stride" in err()
    assert lib.tt_add_rmsnorm_rows_bf16(FAKE, FAKE, 2048, FAKE, 1e-6, FAKE + 2, 10, 2048, None) == \
        _lib.TT_ERR_INVALID_ARGUMENT and "aligned" in err()
    assert lib.tt_add_rmsnorm_rows_bf16(None, FAKE, 2048, FAKE, 1e-6, FAKE, 10, 2048, None) == \
        _lib.TT_ERR_INVALID_ARGUMENT
    # SwiGLU over prompt rows
    assert lib.tt_silu_mul_rows_bf16(FAKE, 6144, FAKE, 6144, 10, 6142, FAKE, None) == _lib.TT_ERR_UNSUPPORTED
    assert lib.tt_silu_mul_rows_bf16(FAKE, 100, FAKE, 6144, 10, 6144, FAKE, None) == _lib.TT_ERR_INVALID_ARGUMENT
    assert lib.tt_silu_mul_rows_bf16(FAKE, 6144, None, 6144, 10, 6144, FAKE, None) == _lib.TT_ERR_INVALID_ARGUMENT
    # RoPE + append from packed rows: offsets and new_lens are required, rows >= 1
    s2, s3 = _lib.strides(3072, 64), _lib.strides(4096, 64, 1)
    head = [FAKE, s2, FAKE, s2, FAKE, s2]
    mid = [FAKE, s3, FAKE, 100, FAKE, FAKE, None, None, 0, 0, FAKE, FAKE, None, None,
           _lib.strides(0, 2048, 256), 64, 2, 8, 32, 8, 64, 16, 0, None]
    assert lib.tt_rope_append_rows_bf16(*head, None, 10, *mid) == _lib.TT_ERR_INVALID_ARGUMENT and "row_offsets" in err()
    assert lib.tt_rope_append_rows_bf16(*head, FAKE, 0, *mid) == _lib.TT_ERR_INVALID_ARGUMENT and "num_rows" in err()


def test_status_maps_to_python_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.TT_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(RuntimeError):
        _lib.check(700, "x")
    _lib.check(0, "x")
