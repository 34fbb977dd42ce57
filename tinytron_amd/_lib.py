"""ctypes binding of libtinytron_amd.so (the C ABI in include/tinytron_amd.h).

The library is built in-tree (``python -m tinytron_amd.build``). Loading
fails loudly when it is missing: there is no CPU or PyTorch fallback for the
decode path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libtinytron_amd.so")
ABI_VERSION = 7

TT_OK = 0
TT_ERR_INVALID_ARGUMENT = -1
TT_ERR_UNSUPPORTED = -2
TT_ERR_WORKSPACE_TOO_SMALL = -3

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.c_void_p  # device int32 pointers are passed as raw addresses
_f32 = ctypes.c_float
_size = ctypes.c_size_t

_ROPE_COMMON = [
    _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,  # q_in, k_in, v_in, q_out (+ strides)
    _vp, _i64,                                       # rope_table, rope_table_len
    _i32p, _i32p, _i32p,                             # positions, new_lens, lens_out
    _i32p, _i64, _i64,                               # page_table, max_pages, num_pages
    _vp, _vp,                                        # k_cache, v_cache
]
_ROPE_TAIL = [
    _i64p,                                           # cache_strides
    _i64, _i64, _i64, _i64, _i64, _i64, _i64,        # capacity, batch, num_new, hq, hkv, head_dim, page_size
    _vp,                                             # stream
]

_ROPE_PART_HEAD = [
    _vp, _i64p, _vp, _i64p, _vp, _i64p,              # q_in, k_in, v_in partials (+ strides)
    _i64, _i64,                                      # splits, split_stride
    _vp, _i64p,                                      # q_out (+ strides)
    _vp, _i64,                                       # rope_table, rope_table_len
    _i32p, _i32p, _i32p,                             # positions, new_lens, lens_out
    _i32p, _i64, _i64,                               # page_table, max_pages, num_pages
    _vp, _vp,                                        # k_cache, v_cache
]

_PREFILL_TAIL = [
    _i32p, _i32p, _i64,                              # positions, new_lens, max_seq_len
    _i32p, _i64, _i64,                               # page_table, max_pages, num_pages
    _vp, _i64p,                                      # out, out_strides {b, t, h}
    _i64, _i64, _i64, _i64, _i64, _i64,              # batch, num_new, hq, hkv, head_dim, page_size
    _f32, _vp,                                       # sm_scale, stream
]

_ATTN_HEAD = [_vp, _i64p, _vp, _vp]                  # q, q_strides, k_cache, v_cache
_ATTN_TAIL = [
    _i64p,                                           # cache_strides
    _i32p, _i64,                                     # seq_lens, max_seq_len
    _i32p, _i64, _i64,                               # page_table, max_pages, num_pages
    _vp, _i64p,                                      # out, out_strides
    _i64, _i64, _i64, _i64, _i64,                    # batch, hq, hkv, head_dim, page_size
    _f32, _i64,                                      # sm_scale, split_tokens
    _vp, _size,                                      # workspace, workspace_bytes
    _vp,                                             # stream
]
# bf16 / fp8 decode attention: the length order (paired partition) after split_tokens
_ATTN_TAIL_ORDER = _ATTN_TAIL[:-3] + [_i32p] + _ATTN_TAIL[-3:]

_ROWS_TAIL = [
    _i64p,                                           # cache_strides
    _i32p, _i32p, _i64,                              # seq_of_row, row_lens, max_row_len
    _i32p, _i64, _i64, _i64,                         # page_table, max_pages, num_pages, num_seqs
    _vp, _i64p,                                      # out, out_strides
    _i64, _i64, _i64, _i64, _i64,                    # rows, hq, hkv, head_dim, page_size
    _f32, _vp, _size, _vp,                           # sm_scale, workspace, workspace_bytes, stream
]

_DECODE_APPEND_HEAD = [
    _vp, _i64p, _vp, _i64p, _vp, _i64p,             # q_in, k_in, v_in (+ {batch, head} strides)
    _i64, _i64,                                      # splits, split_stride
    _vp, _i64,                                       # rope_table, rope_table_len
    _i32p, _i32p, _i64,                              # positions, lens_out, max_seq_len
    _i32p, _i64, _i64,                               # page_table, max_pages, num_pages
    _vp, _vp,                                        # k_cache, v_cache
]
_DECODE_APPEND_TAIL = [
    _i64p, _i64,                                     # cache_strides, capacity
    _vp, _i64p,                                      # out, out_strides
    _i64, _i64, _i64, _i64, _i64,                    # batch, H_q, H_kv, head_dim, page_size
    _f32, _i64, _i32p,                               # sm_scale, split_tokens, length_order
    _vp, _size, _vp,                                 # workspace, workspace_bytes, stream
]
_DECODE_APPEND_TAIL_NOALLOC = _DECODE_APPEND_TAIL[:-6] + [_f32, _vp]  # sm_scale, stream (scratch inside)
NOALLOC_SCRATCH_BYTES = 32 << 20  # TT_NOALLOC_SCRATCH_BYTES

_SAMPLE = [
    _vp, _i64, _i64, _i64,                           # logits, row stride, rows, vocab
    _f32, _i64, _f32,                                # temperature, top_k, top_p
    ctypes.c_uint64, ctypes.c_uint64,                # seed, offset
    _vp, _vp, _vp, _i64,                             # tokens, token_logprob, logprobs, logprobs row stride
    _vp, _size,                                      # workspace, workspace_bytes
    _vp,                                             # stream
]

SIGNATURES = {
    "tt_abi_version": ([], ctypes.c_int),
    "tt_last_error_string": ([], ctypes.c_char_p),
    "tt_rope_append_bf16": (_ROPE_COMMON + _ROPE_TAIL, ctypes.c_int),
    "tt_rope_append_f32": (_ROPE_COMMON + _ROPE_TAIL, ctypes.c_int),
    "tt_rope_append_fp8": (_ROPE_COMMON + [_vp, _vp] + _ROPE_TAIL, ctypes.c_int),
    "tt_rope_append_rows_bf16": ([
        _vp, _i64p, _vp, _i64p, _vp, _i64p,         # q_in, k_in, v_in (+ {row, head} strides)
        _i32p, _i64,                                 # row_offsets, num_rows
        _vp, _i64p,                                  # q_out, q_out_strides
        _vp, _i64, _i32p, _i32p, _i32p,              # rope_table, table_len, positions, new_lens, lens_out
        _i32p, _i64, _i64,                           # page_table, max_pages, num_pages
        _vp, _vp, _vp, _vp,                          # k_cache, v_cache, k_scale, v_scale
        _i64p, _i64,                                 # cache_strides, capacity
        _i64, _i64, _i64, _i64, _i64, _i64,          # batch, num_new, H_q, H_kv, head_dim, page_size
        ctypes.c_int, _vp], ctypes.c_int),           # fp8_cache, stream
    "tt_rope_append_partials_bf16": (_ROPE_PART_HEAD + _ROPE_TAIL, ctypes.c_int),
    "tt_rope_append_partials_fp8": (_ROPE_PART_HEAD + [_vp, _vp] + _ROPE_TAIL, ctypes.c_int),
    "tt_gqa_decode_attn_bf16": (_ATTN_HEAD + _ATTN_TAIL_ORDER, ctypes.c_int),
    "tt_gqa_decode_attn_fp8": (_ATTN_HEAD + [_vp, _vp] + _ATTN_TAIL_ORDER, ctypes.c_int),
    "tt_gqa_decode_attn_f32": (_ATTN_HEAD + _ATTN_TAIL, ctypes.c_int),
    "tt_rows_attn_bf16": (_ATTN_HEAD + _ROWS_TAIL, ctypes.c_int),
    "tt_rows_attn_fp8": (_ATTN_HEAD + [_vp, _vp] + _ROWS_TAIL, ctypes.c_int),
    "tt_rows_attn_f32": (_ATTN_HEAD + _ROWS_TAIL, ctypes.c_int),
    "tt_decode_split_tokens": ([_i64, _i64, _i64], ctypes.c_int64),
    "tt_decode_pick_split": ([_vp, _i64, _i64, _i64, ctypes.c_int32], ctypes.c_int64),
    "tt_decode_workspace_bytes": ([_i64, _i64, _i64, _i64, _i64, _i64], ctypes.c_size_t),
    "tt_prefill_attn_bf16": ([_vp, _i64p, _vp, _vp, _i64p] + _PREFILL_TAIL, ctypes.c_int),
    "tt_prefill_attn_fp8": ([_vp, _i64p, _vp, _vp, _vp, _vp, _i64p] + _PREFILL_TAIL, ctypes.c_int),
    "tt_linear_splitk_bf16": ([_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp], ctypes.c_int),
    "tt_linear_splitk_packed_bf16": ([_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp], ctypes.c_int),
    "tt_splitk_reduce_bf16": ([_vp, _i64, _i64, _i64, _vp, _vp], ctypes.c_int),
    "tt_add_rmsnorm_bf16": ([_vp, _vp, _i64, _vp, ctypes.c_float, _vp, _i64, _i64, _vp], ctypes.c_int),
    "tt_silu_mul_bf16": ([_vp, _i64, _i64, _i64, _vp, _vp], ctypes.c_int),
    "tt_linear_swiglu_packed_bf16": ([_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp], ctypes.c_int),
    "tt_swiglu_gemm_supported": ([_i64, _i64], ctypes.c_int),
    "tt_add_rmsnorm_rows_bf16": ([_vp, _vp, _i64, _vp, ctypes.c_float, _vp, _i64, _i64, _vp], ctypes.c_int),
    "tt_silu_mul_rows_bf16": ([_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp], ctypes.c_int),
    "tt_decode_attn_append_bf16": (_DECODE_APPEND_HEAD + _DECODE_APPEND_TAIL, ctypes.c_int),
    "tt_decode_attn_append_fp8": (_DECODE_APPEND_HEAD + [_vp, _vp] + _DECODE_APPEND_TAIL, ctypes.c_int),
    "tt_decode_attn_append_bf16_noalloc": (_DECODE_APPEND_HEAD + _DECODE_APPEND_TAIL_NOALLOC, ctypes.c_int),
    "tt_sample_bf16": (_SAMPLE, ctypes.c_int),
    "tt_sample_f32": (_SAMPLE, ctypes.c_int),
    "tt_sample_workspace_bytes": ([_i64, _i64, _i64], _size),
    "tt_decode_layers_bf16": ([_vp, _i64, _i64, _vp], ctypes.c_int),
}



class DecodeLayer(ctypes.Structure):
    """tt_decode_layer_t: one layer's fused bf16 decode step (buffers, packed
    weights, cache and attention arguments) for tt_decode_layers_bf16."""
    _fields_ = [
        ("x", _vp), ("h", _vp), ("partials", _vp), ("attn_out", _vp), ("act", _vp),
        ("w_qkv", _vp), ("w_o", _vp), ("w_gu", _vp), ("w_down", _vp),
        ("ln2_weight", _vp), ("next_norm_weight", _vp), ("eps", _f32),
        ("batch", _i64), ("hidden", _i64), ("intermediate", _i64), ("num_q_heads", _i64),
        ("num_kv_heads", _i64), ("head_dim", _i64),
        ("kc_qkv", _i64), ("kc_o", _i64), ("kc_gu", _i64), ("kc_down", _i64),
        ("fp8_cache", ctypes.c_int32), ("rope_table", _vp), ("rope_table_len", _i64),
        ("positions", _vp), ("lens_out", _vp),
        ("page_table", _vp), ("max_pages", _i64), ("num_pages", _i64),
        ("k_cache", _vp), ("v_cache", _vp), ("k_scale", _vp), ("v_scale", _vp),
        ("cache_strides", _i64 * 3), ("capacity", _i64), ("page_size", _i64),
        ("sm_scale", _f32), ("split_tokens", _i64), ("length_order", _vp),
        ("workspace", _vp), ("workspace_bytes", _size),
    ]


_LIB = None


def load() -> ctypes.CDLL:
    """Load (once) and type the library; raise if it is missing or stale."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH.name} is not built; run `python -m tinytron_amd.build` (hipcc, gfx950). "
            "The decode path has no fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    version = lib.tt_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH.name} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def strides(*values: int):
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr


def check(status: int, what: str) -> None:
    """Map a library status to the exception the reference would raise."""
    if status == TT_OK:
        return
    msg = load().tt_last_error_string().decode(errors="replace")
    if status < 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {status}: {msg}")
