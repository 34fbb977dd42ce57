"""PyTorch-facing wrappers of the gfx950 decode-step kernels.

Tensors are validated here (device, dtype, shape, strides), then their raw
device pointers go through the C ABI (include/tinytron_amd.h) on the current
torch stream. There is no fallback: every entry point needs the HIP library
and CUDA(HIP) tensors.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib

FP8_DTYPE = torch.float8_e4m3fn


def build_rope_table(num_positions: int, head_dim: int, theta: float = 10000.0,
                     dtype: torch.dtype = torch.bfloat16, device="cuda") -> torch.Tensor:
    """[num_positions, D] table = [cos(p f_i) | sin(p f_i)], i < D/2, in ``dtype``.

    Built on ``device`` with the reference's own op sequence
    (tinytron/model/modules/attn.py:30-54: inv_freq, the fp32 outer product,
    cos/sin, cast to the activation dtype), so on the GPU it holds the bytes
    the reference's rope_impl computes there. Only the first half of
    ``emb = cat(freqs, freqs)`` is kept; the second half is identical.
    """
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    dev = torch.device(device)
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=dev) / head_dim))
    pos = torch.arange(num_positions, device=dev).unsqueeze(0).float()
    freqs = torch.einsum("bt,d->btd", pos, inv_freq)[0]
    return torch.cat([freqs.cos().to(dtype), freqs.sin().to(dtype)], dim=-1).contiguous()


@dataclass
class KVLayout:
    """Device view of one layer's cache as the kernels address it.

    ``k``/``v`` are the storage tensors (bf16, fp32, or uint8 e4m3fn codes);
    ``strides`` = (seq, page, head) element strides; ``page_table`` is None
    for the contiguous [B, H, pages, P, D] store or an int32 [B, max_pages]
    device tensor for the pool [num_pages, H, P, D]. fp8 scales are fp32 in
    16-row groups (``fp8_scale_index``; ``fp8_scales`` allocates them).
    """

    k: torch.Tensor
    v: torch.Tensor
    strides: tuple
    num_heads: int
    head_dim: int
    page_size: int
    capacity: int
    kind: str  # "bf16" | "f32" | "fp8"
    page_table: torch.Tensor | None = None
    num_pages: int = 0
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None

    @property
    def max_pages(self) -> int:
        return 0 if self.page_table is None else int(self.page_table.shape[1])


def fp8_scale_index(row):
    """Index of row ``row``'s K scale in k_scale (and of its V scale in v_scale)
    of an fp8 cache, row = element offset of d = 0 / head_dim: rows grouped by
    16, each group's 16 K scales then its 16 V scales (ints, numpy or torch
    integer arrays)."""
    return row + (row // 16) * 16


def fp8_scales(rows: int, device) -> tuple:
    """(k_scale, v_scale) of an fp8 cache with ``rows`` (token, head) rows: one
    fp32 array of 2 x rows entries (rows rounded up to 16) and its view 16
    entries in, so that each 16-row group's K and V scales share a 128-byte
    line (fp8_scale_index)."""
    t = torch.empty(2 * (-(-int(rows) // 16) * 16), dtype=torch.float32, device=device)
    return t, t[16:]


def _stream(device: torch.device) -> int:
    """The current stream's handle on the tensor's device (torch's raw-stream
    accessor: the Python stream object costs microseconds per launch)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("tinytron_amd kernels need GPU tensors (no CPU fallback)")


def _ptr(t):
    return None if t is None else t.data_ptr()


def _act_kind(dtype: torch.dtype) -> str:
    if dtype == torch.bfloat16:
        return "bf16"
    if dtype == torch.float32:
        return "f32"
    raise ValueError(f"unsupported activation dtype {dtype}")


def _check_lastdim(name: str, t: torch.Tensor, dims: int) -> None:
    if t.dim() != dims:
        raise ValueError(f"{name} must have {dims} dims, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in head_dim")


def rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, table: torch.Tensor,
                positions: torch.Tensor, layout: KVLayout, q_out: torch.Tensor | None = None,
                new_lens: torch.Tensor | None = None, lens_out: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE q and k at per-sequence positions, append k/v to the cache.

    q [B, H_q, T, D], k/v [B, H_kv, T, D] (any strides, head_dim contiguous);
    positions int32 [B] = slot of token 0 per sequence; lens_out (int32 [B],
    optional) receives the lengths after the append; returns rotated q.
    Restates rope_impl (attn.py:13-63) + LayerPagedKVCache.append
    (cache.py:34-45) in one launch.
    """
    _require_cuda(q, k, v, table, positions, layout.k, layout.v)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_lastdim(name, t, 4)
    B, Hq, T, D = q.shape
    if k.shape != (B, layout.num_heads, T, D) or v.shape != k.shape:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)} / cache heads")
    if D != layout.head_dim:
        raise ValueError(f"head_dim {D} does not match the cache's {layout.head_dim}")
    kind = _act_kind(q.dtype)
    if k.dtype != q.dtype or v.dtype != q.dtype or table.dtype != q.dtype:
        raise ValueError("q, k, v and the rope table must share one dtype")
    if layout.kind == "fp8" and kind != "bf16":
        raise ValueError("an fp8 cache takes bf16 activations")
    if layout.kind != "fp8" and layout.kind != kind:
        raise ValueError(f"cache dtype {layout.kind} does not match activations {kind}")
    if table.dim() != 2 or table.shape[1] != D or not table.is_contiguous():
        raise ValueError("rope table must be a contiguous [positions, head_dim] tensor")
    if positions.dtype != torch.int32 or positions.shape != (B,):
        raise ValueError("positions must be int32 [B]")
    if new_lens is not None and (new_lens.dtype != torch.int32 or new_lens.shape != (B,)):
        raise ValueError("new_lens must be int32 [B]")
    if lens_out is not None and (lens_out.dtype != torch.int32 or lens_out.shape != (B,)):
        raise ValueError("lens_out must be int32 [B]")
    if q_out is None:
        q_out = torch.empty(B, Hq, T, D, dtype=q.dtype, device=q.device)
    _check_lastdim("q_out", q_out, 4)
    lib = _lib.load()
    common = [
        _ptr(q), _lib.strides(*q.stride()[:3]), _ptr(k), _lib.strides(*k.stride()[:3]),
        _ptr(v), _lib.strides(*v.stride()[:3]), _ptr(q_out), _lib.strides(*q_out.stride()[:3]),
        _ptr(table), table.shape[0], _ptr(positions), _ptr(new_lens), _ptr(lens_out),
        _ptr(layout.page_table), layout.max_pages, layout.num_pages,
        _ptr(layout.k), _ptr(layout.v),
    ]
    tail = [_lib.strides(*layout.strides), layout.capacity, B, T, Hq, layout.num_heads, D,
            layout.page_size, _stream(q.device)]
    if layout.kind == "fp8":
        st = lib.tt_rope_append_fp8(*common, _ptr(layout.k_scale), _ptr(layout.v_scale), *tail)
    elif layout.kind == "bf16":
        st = lib.tt_rope_append_bf16(*common, *tail)
    else:
        st = lib.tt_rope_append_f32(*common, *tail)
    _lib.check(st, "rope_append")
    return q_out


def rope_append_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, table: torch.Tensor,
                     positions: torch.Tensor, layout: KVLayout, row_offsets: torch.Tensor, new_lens: torch.Tensor,
                     num_new: int, q_out: torch.Tensor | None = None,
                     lens_out: torch.Tensor | None = None) -> torch.Tensor:
    """rope_append for a prompt batch packed without padding: q [N, H_q, D],
    k / v [N, H_kv, D] (strides {row, head}, head_dim contiguous); token t of
    sequence b is row row_offsets[b] + t for t < new_lens[b] (int32 [B]).
    Returns the rotated q on the [B, H_q, num_new, D] grid (rows past
    new_lens[b] not written); k / v go to each sequence's next slots."""
    _require_cuda(q, k, v, table, positions, layout.k, layout.v, row_offsets, new_lens)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_lastdim(name, t, 3)
    N, Hq, D = q.shape
    B = positions.shape[0]
    if k.shape != (N, layout.num_heads, D) or v.shape != k.shape:
        raise ValueError(f"k/v shape {tuple(k.shape)} does not match q {tuple(q.shape)} / cache heads")
    if D != layout.head_dim:
        raise ValueError(f"head_dim {D} does not match the cache's {layout.head_dim}")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype or table.dtype != q.dtype:
        raise ValueError("packed rows take bf16 q, k, v and rope table")
    if layout.kind not in ("bf16", "fp8"):
        raise ValueError("packed rows append to a bf16 or fp8 cache")
    if table.dim() != 2 or table.shape[1] != D or not table.is_contiguous():
        raise ValueError("rope table must be a contiguous [positions, head_dim] tensor")
    for name, t in (("positions", positions), ("row_offsets", row_offsets), ("new_lens", new_lens)):
        if t.dtype != torch.int32 or t.shape != (B,):
            raise ValueError(f"{name} must be int32 [B]")
    if lens_out is not None and (lens_out.dtype != torch.int32 or lens_out.shape != (B,)):
        raise ValueError("lens_out must be int32 [B]")
    if q_out is None:
        q_out = torch.empty(B, Hq, num_new, D, dtype=q.dtype, device=q.device)
    _check_lastdim("q_out", q_out, 4)
    fp8 = layout.kind == "fp8"
    st = _lib.load().tt_rope_append_rows_bf16(
        _ptr(q), _lib.strides(*q.stride()[:2]), _ptr(k), _lib.strides(*k.stride()[:2]), _ptr(v),
        _lib.strides(*v.stride()[:2]), _ptr(row_offsets), N, _ptr(q_out), _lib.strides(*q_out.stride()[:3]),
        _ptr(table), table.shape[0], _ptr(positions), _ptr(new_lens), _ptr(lens_out),
        _ptr(layout.page_table), layout.max_pages, layout.num_pages, _ptr(layout.k), _ptr(layout.v),
        _ptr(layout.k_scale) if fp8 else None, _ptr(layout.v_scale) if fp8 else None,
        _lib.strides(*layout.strides), layout.capacity, B, num_new, Hq, layout.num_heads, D, layout.page_size,
        1 if fp8 else 0, _stream(q.device))
    _lib.check(st, "rope_append_rows")
    return q_out


def rope_append_partials(partials: torch.Tensor, num_q_heads: int, table: torch.Tensor, positions: torch.Tensor,
                         layout: KVLayout, q_out: torch.Tensor | None = None,
                         lens_out: torch.Tensor | None = None) -> torch.Tensor:
    """rope_append for one new token per sequence whose q|k|v come as the fp32
    split-K partials [S, B, (H_q + 2 H_kv) D] of the stacked projection: the
    kernel sums the splits in order and rounds to bf16 (the projection's
    output) before RoPE + append. Returns rotated q [B, H_q, 1, D] (bf16)."""
    _require_cuda(partials, table, positions, layout.k, layout.v)
    if partials.dtype != torch.float32 or partials.dim() != 3 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 [S, B, N] tensor")
    S, B, N = partials.shape
    Hkv, D = layout.num_heads, layout.head_dim
    if N != (num_q_heads + 2 * Hkv) * D:
        raise ValueError(f"partials have {N} columns, expected (H_q + 2 H_kv) * D = {(num_q_heads + 2 * Hkv) * D}")
    if table.dtype != torch.bfloat16 or table.dim() != 2 or table.shape[1] != D or not table.is_contiguous():
        raise ValueError("rope table must be a contiguous bf16 [positions, head_dim] tensor")
    if layout.kind not in ("bf16", "fp8"):
        raise ValueError("split-K partial inputs are for bf16 activations (bf16 or fp8 cache)")
    if positions.dtype != torch.int32 or positions.shape != (B,):
        raise ValueError("positions must be int32 [B]")
    if lens_out is not None and (lens_out.dtype != torch.int32 or lens_out.shape != (B,)):
        raise ValueError("lens_out must be int32 [B]")
    if q_out is None:
        q_out = torch.empty(B, num_q_heads, 1, D, dtype=torch.bfloat16, device=partials.device)
    _check_lastdim("q_out", q_out, 4)
    base = partials.data_ptr()
    in_strides = _lib.strides(N, D, N)  # [B, H, T = 1, D] views of one split
    lib = _lib.load()
    head = [base, in_strides, base + num_q_heads * D * 4, in_strides, base + (num_q_heads + Hkv) * D * 4, in_strides,
            S, B * N, _ptr(q_out), _lib.strides(*q_out.stride()[:3]),
            _ptr(table), table.shape[0], _ptr(positions), None, _ptr(lens_out),
            _ptr(layout.page_table), layout.max_pages, layout.num_pages, _ptr(layout.k), _ptr(layout.v)]
    tail = [_lib.strides(*layout.strides), layout.capacity, B, 1, num_q_heads, Hkv, D, layout.page_size,
            _stream(partials.device)]
    if layout.kind == "fp8":
        st = lib.tt_rope_append_partials_fp8(*head, _ptr(layout.k_scale), _ptr(layout.v_scale), *tail)
    else:
        st = lib.tt_rope_append_partials_bf16(*head, *tail)
    _lib.check(st, "rope_append_partials")
    return q_out


class Workspace:
    """Grow-only device scratch for the split-K partials of one stream."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.buf = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self.buf


def attention_tile_dim(head_dim: int, kind: str) -> int:
    """Tile width of the MFMA attention kernels for a ``kind`` ("bf16" / "fp8")
    cache of this head_dim (the library's tile rule): 32 (bf16 only), 64 or 128
    when a row is a whole number of 16-byte fragments (head_dim a multiple of 8
    bf16 / 16 fp8 values) and head_dim <= 128; 0 otherwise, where decode
    attention runs the VALU kernel and the fused decode step and the prefill
    kernel do not apply."""
    if kind not in ("bf16", "fp8") or head_dim <= 0 or head_dim > 128:
        return 0
    if head_dim % (16 if kind == "fp8" else 8):
        return 0
    if kind == "bf16" and head_dim <= 32:
        return 32
    return 64 if head_dim <= 64 else 128


def split_tokens_for(batch: int, num_kv_heads: int, max_seq_len: int) -> int:
    return int(_lib.load().tt_decode_split_tokens(batch, num_kv_heads, max_seq_len))


# split_tokens of the per-segment partition: one workgroup per (sequence, KV
# head), merged inside the launch (no merge launch, no workspace)
SPLIT_PER_SEGMENT = -1
# split_tokens of the paired partition: one workgroup per pair of length ranks
# (p, B - 1 - p) and KV head, merged inside the launch (B <= 256)
SPLIT_PAIRED = -2


def pick_split(seq_lens_host, num_kv_heads: int, head_dim: int, kind: str) -> int:
    """split_tokens for decode attention over these host-side lengths
    (tt_decode_pick_split): SPLIT_PER_SEGMENT when they are all equal and
    B * H_kv fills whole rounds of the GPU's resident workgroups;
    SPLIT_PAIRED when they differ, B <= 256, the rank pairs' workgroups fill
    whole rounds of the GPU's CUs and their work is within 6 % of the mean;
    else 0 (the balanced partition)."""
    if kind not in ("bf16", "fp8") or len(seq_lens_host) == 0:
        return 0
    lens = (ctypes.c_int32 * len(seq_lens_host))(*[int(x) for x in seq_lens_host])
    return int(_lib.load().tt_decode_pick_split(ctypes.addressof(lens), len(seq_lens_host), num_kv_heads, head_dim,
                                                int(kind == "fp8")))


def workspace_bytes(batch: int, hq: int, hkv: int, head_dim: int, max_seq_len: int, split_tokens: int = 0) -> int:
    return int(_lib.load().tt_decode_workspace_bytes(batch, hq, hkv, head_dim, max_seq_len, split_tokens))


def _check_order(length_order, B: int):
    if length_order is not None and (length_order.dtype != torch.int32 or length_order.shape != (B,)
                                     or not length_order.is_cuda or not length_order.is_contiguous()):
        raise ValueError("length_order must be a contiguous int32 [B] device tensor")


def length_order(lengths) -> list:
    """The batch's sequence indices by length, longest first, ties by index:
    the order the paired partition pairs (ranks p and B - 1 - p)."""
    return sorted(range(len(lengths)), key=lambda b: (-int(lengths[b]), b))


def decode_attention(q: torch.Tensor, layout: KVLayout, seq_lens: torch.Tensor, max_seq_len: int,
                     out: torch.Tensor | None = None, sm_scale: float | None = None, split_tokens: int = 0,
                     workspace: Workspace | None = None, length_order: torch.Tensor | None = None) -> torch.Tensor:
    """GQA decode attention of q [B, H_q, D] over each sequence's seq_lens[b] cached tokens.

    Restates get_kv + gqa_impl + the all-True decode mask + SDPA
    (cache.py:47-51, attn.py:66-95, 420-423). ``max_seq_len`` is a host-side
    bound of seq_lens used to size the grid. ``length_order`` (SPLIT_PAIRED,
    bf16 / fp8 caches; optional): int32 [B] on the device, a permutation of
    the batch ordered as ``length_order()`` orders seq_lens, which spares the
    kernel its own ranking; None ranks on the device.
    """
    _require_cuda(q, layout.k, layout.v, seq_lens)
    _check_lastdim("q", q, 3)
    B, Hq, D = q.shape
    kind = _act_kind(q.dtype)
    if layout.kind == "fp8":
        if kind != "bf16":
            raise ValueError("an fp8 cache takes bf16 queries")
    elif layout.kind != kind:
        raise ValueError(f"cache dtype {layout.kind} does not match q {kind}")
    if D != layout.head_dim:
        raise ValueError(f"head_dim {D} does not match the cache's {layout.head_dim}")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (B,):
        raise ValueError("seq_lens must be int32 [B]")
    _check_order(length_order, B)
    if max_seq_len > layout.capacity:
        raise ValueError(f"max_seq_len {max_seq_len} exceeds the cache capacity {layout.capacity}")
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    _check_lastdim("out", out, 3)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    hkv = layout.num_heads
    need = workspace_bytes(B, Hq, hkv, D, max_seq_len, split_tokens)
    ws = (workspace or Workspace(q.device)).get(need)
    lib = _lib.load()
    head = [_ptr(q), _lib.strides(*q.stride()[:2]), _ptr(layout.k), _ptr(layout.v)]
    tail = [
        _lib.strides(*layout.strides), _ptr(seq_lens), int(max_seq_len),
        _ptr(layout.page_table), layout.max_pages, layout.num_pages,
        _ptr(out), _lib.strides(*out.stride()[:2]),
        B, Hq, hkv, D, layout.page_size, float(sm_scale), int(split_tokens),
        _ptr(ws), ws.numel(), _stream(q.device),
    ]
    order = [_ptr(length_order)]
    if layout.kind == "fp8":
        st = lib.tt_gqa_decode_attn_fp8(*head, _ptr(layout.k_scale), _ptr(layout.v_scale), *tail[:-3], *order,
                                        *tail[-3:])
    elif layout.kind == "bf16":
        st = lib.tt_gqa_decode_attn_bf16(*head, *tail[:-3], *order, *tail[-3:])
    else:
        st = lib.tt_gqa_decode_attn_f32(*head, *tail)
    _lib.check(st, "decode_attention")
    return out


ROWS_ATTN_MAX_ROWS = 65535  # query rows per tt_rows_attn_* launch


def rows_attention(q: torch.Tensor, layout: KVLayout, seq_of_row: torch.Tensor, row_lens: torch.Tensor,
                   max_row_len: int, num_seqs: int, out: torch.Tensor | None = None, sm_scale: float | None = None,
                   workspace: Workspace | None = None) -> torch.Tensor:
    """GQA attention of query rows q [R, H_q, D], row r over the first
    row_lens[r] cached tokens of sequence seq_of_row[r] (int32 [R] each; the
    cache holds num_seqs sequences); returns out [R, H_q, D] (zeros where
    row_lens[r] <= 0). Rows t of a prefill chunk with row_lens = cached + t + 1
    give the reference's cache-causal prefill attention (attn.py:321-341) for
    the caches and head dims the prefill kernel does not take (fp32, rows that
    are not whole 16-byte fragments); launches of at most ROWS_ATTN_MAX_ROWS
    rows."""
    _require_cuda(q, layout.k, layout.v, seq_of_row, row_lens)
    _check_lastdim("q", q, 3)
    R, Hq, D = q.shape
    kind = _act_kind(q.dtype)
    if layout.kind == "fp8":
        if kind != "bf16":
            raise ValueError("an fp8 cache takes bf16 queries")
    elif layout.kind != kind:
        raise ValueError(f"cache dtype {layout.kind} does not match q {kind}")
    if D != layout.head_dim:
        raise ValueError(f"head_dim {D} does not match the cache's {layout.head_dim}")
    for name, t in (("seq_of_row", seq_of_row), ("row_lens", row_lens)):
        if t.dtype != torch.int32 or t.shape != (R,):
            raise ValueError(f"{name} must be int32 [R]")
    if max_row_len > layout.capacity:
        raise ValueError(f"max_row_len {max_row_len} exceeds the cache capacity {layout.capacity}")
    if out is None:
        out = torch.empty(R, Hq, D, dtype=q.dtype, device=q.device)
    _check_lastdim("out", out, 3)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    hkv = layout.num_heads
    lib = _lib.load()
    fn = {"fp8": lib.tt_rows_attn_fp8, "bf16": lib.tt_rows_attn_bf16, "f32": lib.tt_rows_attn_f32}[layout.kind]
    scales = [_ptr(layout.k_scale), _ptr(layout.v_scale)] if layout.kind == "fp8" else []
    workspace = workspace or Workspace(q.device)
    for r0 in range(0, R, ROWS_ATTN_MAX_ROWS):
        n = min(ROWS_ATTN_MAX_ROWS, R - r0)
        ws = workspace.get(workspace_bytes(n, Hq, hkv, D, max_row_len, 0))
        qc, oc = q[r0:r0 + n], out[r0:r0 + n]
        st = fn(_ptr(qc), _lib.strides(*qc.stride()[:2]), _ptr(layout.k), _ptr(layout.v), *scales,
                _lib.strides(*layout.strides), _ptr(seq_of_row[r0:r0 + n]), _ptr(row_lens[r0:r0 + n]),
                int(max_row_len), _ptr(layout.page_table), layout.max_pages, layout.num_pages, int(num_seqs),
                _ptr(oc), _lib.strides(*oc.stride()[:2]), n, Hq, hkv, D, layout.page_size, float(sm_scale),
                _ptr(ws), ws.numel(), _stream(q.device))
        _lib.check(st, "rows_attention")
    return out


def prefill_attention_rows(q: torch.Tensor, layout: KVLayout, cached, new_lens, out: torch.Tensor | None = None,
                           sm_scale: float | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """prefill_attention through rows_attention: q [B, H_q, T, D] (rotated),
    host lists cached[b] (tokens before the chunk) and new_lens[b]; returns out
    [B, T, H_q, D] with row t < new_lens[b] of sequence b attending to its
    cached[b] + t + 1 first tokens (rows past new_lens[b] are zero)."""
    B, Hq, T, D = q.shape
    cached = [int(x) for x in cached]
    new_lens = [min(int(x), T) for x in new_lens]
    lens = torch.zeros(B, T, dtype=torch.int32)
    steps = torch.arange(1, T + 1, dtype=torch.int32)
    for b in range(B):
        n = new_lens[b]
        lens[b, :n] = cached[b] + steps[:n]
    seq = torch.arange(B, dtype=torch.int32).repeat_interleave(T)
    q_rows = q.transpose(1, 2).contiguous().view(B * T, Hq, D)
    if out is None:
        out = torch.empty(B, T, Hq, D, dtype=q.dtype, device=q.device)
    o_rows = out.view(B * T, Hq, D) if out.is_contiguous() else torch.empty(B * T, Hq, D, dtype=q.dtype,
                                                                            device=q.device)
    max_len = max((c + n for c, n in zip(cached, new_lens)), default=0)
    rows_attention(q_rows, layout, seq.to(q.device, non_blocking=True), lens.view(-1).to(q.device, non_blocking=True),
                   max(max_len, 1), B, out=o_rows, sm_scale=sm_scale, workspace=workspace)
    if o_rows.data_ptr() != out.data_ptr():
        out.copy_(o_rows.view(B, T, Hq, D))
    return out


FUSED_STEP_MAX_SPLITS = 4  # split-K partials decode_attention_append sums per input


def decode_attention_append(table: torch.Tensor, positions: torch.Tensor, layout: KVLayout, max_seq_len: int,
                            q: torch.Tensor | None = None, k: torch.Tensor | None = None, v: torch.Tensor | None = None,
                            partials: torch.Tensor | None = None, num_q_heads: int | None = None,
                            lens_out: torch.Tensor | None = None, out: torch.Tensor | None = None,
                            sm_scale: float | None = None, workspace: Workspace | None = None,
                            no_alloc: bool = False, split_tokens: int = 0,
                            length_order: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step in one launch pair: RoPE of this step's q and k at
    positions[b], append of k / v at that slot, and GQA attention over the
    positions[b] + 1 cached tokens (rope_append followed by decode_attention,
    without writing the rotated q). Inputs: bf16 q [B, H_q, D] and k / v
    [B, H_kv, D] (strided views, head_dim contiguous), or ``partials`` fp32
    [S, B, (H_q + 2 H_kv) D] of the stacked q|k|v projection with
    ``num_q_heads``. ``max_seq_len`` bounds positions + 1. Returns out
    [B, H_q, D] bf16. ``no_alloc`` (bf16 caches) runs the allocation-free
    entry point, whose workspace is the library's per-GPU scratch
    (``workspace`` is then unused; pass ``out`` to allocate nothing at all;
    calls that overlap on one GPU race on that scratch). ``split_tokens``: 0
    (balanced partition), SPLIT_PER_SEGMENT or SPLIT_PAIRED (no workspace;
    not with ``no_alloc``); ``length_order`` as for decode_attention, ordered
    by positions."""
    _require_cuda(table, positions, layout.k, layout.v)
    if split_tokens not in (0, SPLIT_PER_SEGMENT, SPLIT_PAIRED):
        raise ValueError(f"the fused decode step takes split_tokens 0, {SPLIT_PER_SEGMENT} or {SPLIT_PAIRED}, "
                         f"got {split_tokens}")
    if layout.kind not in ("bf16", "fp8"):
        raise ValueError("the fused decode step takes a bf16 or fp8 cache")
    Hkv, D = layout.num_heads, layout.head_dim
    if partials is not None:
        _require_cuda(partials)
        if partials.dtype != torch.float32 or partials.dim() != 3 or not partials.is_contiguous():
            raise ValueError("partials must be a contiguous fp32 [S, B, N] tensor")
        S, B, N = partials.shape
        if S > FUSED_STEP_MAX_SPLITS:
            raise ValueError(f"the fused step sums at most {FUSED_STEP_MAX_SPLITS} split-K partials, got {S}")
        Hq = int(num_q_heads)
        if N != (Hq + 2 * Hkv) * D:
            raise ValueError(f"partials have {N} columns, expected (H_q + 2 H_kv) * D = {(Hq + 2 * Hkv) * D}")
        base = partials.data_ptr()
        st_in = _lib.strides(N, D)
        ins = [base, st_in, base + Hq * D * 4, st_in, base + (Hq + Hkv) * D * 4, st_in, S, B * N]
        dev = partials.device
    else:
        _require_cuda(q, k, v)
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check_lastdim(name, t, 3)
            if t.dtype != torch.bfloat16:
                raise ValueError("the fused decode step takes bf16 q / k / v")
        B, Hq, Dq = q.shape
        if Dq != D or k.shape != (B, Hkv, D) or v.shape != k.shape:
            raise ValueError(f"q {tuple(q.shape)} / k {tuple(k.shape)} / v {tuple(v.shape)} do not match the cache")
        ins = [_ptr(q), _lib.strides(*q.stride()[:2]), _ptr(k), _lib.strides(*k.stride()[:2]),
               _ptr(v), _lib.strides(*v.stride()[:2]), 0, 0]
        dev = q.device
    if table.dtype != torch.bfloat16 or table.dim() != 2 or table.shape[1] != D or not table.is_contiguous():
        raise ValueError("rope table must be a contiguous bf16 [positions, head_dim] tensor")
    if positions.dtype != torch.int32 or positions.shape != (B,):
        raise ValueError("positions must be int32 [B]")
    if lens_out is not None and (lens_out.dtype != torch.int32 or lens_out.shape != (B,)):
        raise ValueError("lens_out must be int32 [B]")
    _check_order(length_order, B)
    if not 1 <= max_seq_len <= layout.capacity:
        raise ValueError(f"max_seq_len {max_seq_len} must be in [1, capacity {layout.capacity}]")
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    _check_lastdim("out", out, 3)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    lib = _lib.load()
    head = ins + [_ptr(table), table.shape[0], _ptr(positions), _ptr(lens_out), int(max_seq_len),
                  _ptr(layout.page_table), layout.max_pages, layout.num_pages, _ptr(layout.k), _ptr(layout.v)]
    tail = [_lib.strides(*layout.strides), layout.capacity, _ptr(out), _lib.strides(*out.stride()[:2]),
            B, Hq, Hkv, D, layout.page_size, float(sm_scale)]
    if no_alloc:  # the library's own per-GPU scratch: nothing is allocated (HIP graph capture, serving loops)
        if layout.kind != "bf16":
            raise ValueError("the allocation-free decode step takes a bf16 cache")
        if split_tokens != 0:
            raise ValueError("the allocation-free decode step runs the balanced partition (split_tokens 0)")
        st = lib.tt_decode_attn_append_bf16_noalloc(*head, *tail, _stream(dev))
        _lib.check(st, "decode_attention_append (no allocation)")
        return out
    tail += [int(split_tokens), _ptr(length_order)]
    if split_tokens < 0:  # merged inside the launch: no workspace
        tail += [None, 0, _stream(dev)]
    else:
        need = workspace_bytes(B, Hq, Hkv, D, max_seq_len, 0)
        ws = (workspace or Workspace(dev)).get(need)
        tail += [_ptr(ws), ws.numel(), _stream(dev)]
    if layout.kind == "fp8":
        st = lib.tt_decode_attn_append_fp8(*head, _ptr(layout.k_scale), _ptr(layout.v_scale), *tail)
    else:
        st = lib.tt_decode_attn_append_bf16(*head, *tail)
    _lib.check(st, "decode_attention_append")
    return out


# -- decode-step layer operations ----------------------------------------------------------

def _rows(t: torch.Tensor, name: str) -> tuple:
    """(rows, row stride) of a 2-D row-major view (last dim contiguous)."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D view with a contiguous last dimension")
    return t.shape[0], t.stride(0)


class PackedWeight:
    """A [N, K] bf16 weight in the GEMM's fragment order ([N/16][K/32][64][8])."""

    def __init__(self, weight: torch.Tensor):
        N, K = weight.shape
        if N % 16 or K % 32:
            raise ValueError("packing needs N % 16 == 0 and K % 32 == 0")
        self.shape = (N, K)
        self.data = weight.detach().reshape(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()

    def unpack(self) -> torch.Tensor:
        N, K = self.shape
        return self.data.permute(0, 3, 1, 2, 4).reshape(N, K)


def linear_partials(x: torch.Tensor, weight, partials: torch.Tensor | None = None,
                    k_chunk: int = 512) -> torch.Tensor:
    """Split-K partials [K / k_chunk, M, N] (fp32) of x [M, K] @ weight[N, K]^T (bf16).

    nn.Linear(bias=False) under bf16 autocast (attn.py:141-145, mlp.py:24-26)
    for M <= a few hundred rows; sum the partials with splitk_reduce_bf16 or
    a consuming op (add_rmsnorm, silu_mul). ``weight`` is a bf16 tensor or a
    PackedWeight."""
    packed = isinstance(weight, PackedWeight)
    wt = weight.data if packed else weight
    _require_cuda(x, wt)
    if x.dtype != torch.bfloat16 or wt.dtype != torch.bfloat16:
        raise ValueError("linear_partials takes bf16 x and weight")
    M, ldx = _rows(x, "x")
    if packed:
        N, Kw = weight.shape
        ldw = Kw
    else:
        N, ldw = _rows(weight, "weight")
        Kw = weight.shape[1]
    K = x.shape[1]
    if Kw != K:
        raise ValueError(f"x has K = {K}, weight has {Kw}")
    S = K // k_chunk
    if partials is None:
        partials = torch.empty(S, M, N, dtype=torch.float32, device=x.device)
    elif partials.dtype != torch.float32 or partials.numel() < S * M * N or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 buffer of at least K / k_chunk * M * N elements")
    lib = _lib.load()
    if packed:
        st = lib.tt_linear_splitk_packed_bf16(_ptr(x), ldx, _ptr(wt), _ptr(partials), M, N, K, k_chunk,
                                              _stream(x.device))
    else:
        st = lib.tt_linear_splitk_bf16(_ptr(x), ldx, _ptr(wt), ldw, _ptr(partials), M, N, K, k_chunk,
                                       _stream(x.device))
    _lib.check(st, "linear_partials")
    return partials.view(-1)[:S * M * N].view(S, M, N)


def splitk_reduce_bf16(partials: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(sum over the first axis) of fp32 partials [S, M, N]."""
    _require_cuda(partials)
    S, M, N = partials.shape
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=partials.device)
    if not out.is_contiguous() or out.shape != (M, N) or out.dtype != torch.bfloat16:
        raise ValueError("out must be a contiguous bf16 [M, N] tensor")
    _lib.check(_lib.load().tt_splitk_reduce_bf16(_ptr(partials), S, M, N, _ptr(out), _stream(partials.device)),
               "splitk_reduce_bf16")
    return out


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, partials: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """x += bf16(sum of partials) (in place, if given); returns bf16 RMSNorm(x) [M, C].

    The residual add of Block.forward (gpt.py:40-41) fused with the next
    RMSNorm (norm.py:6-19)."""
    _require_cuda(x, weight)
    if x.dtype != torch.float32 or weight.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("add_rmsnorm takes a contiguous fp32 residual x [M, C] and fp32 weight [C]")
    M, C = x.shape
    S = 0
    if partials is not None:
        S = partials.shape[0]
        if partials.shape[1:] != (M, C) or not partials.is_contiguous():
            raise ValueError("partials must be contiguous [S, M, C]")
    if out is None:
        out = torch.empty(M, C, dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().tt_add_rmsnorm_bf16(_ptr(x), _ptr(partials), S, _ptr(weight), float(eps), _ptr(out), M, C,
                                                 _stream(x.device)), "add_rmsnorm")
    return out


def add_rmsnorm_rows(x: torch.Tensor, weight: torch.Tensor, eps: float, addend: torch.Tensor | None = None,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """x += float(addend) (in place, if given: a projection's bf16 output [M, C],
    row stride a multiple of 4); returns bf16 RMSNorm(x) [M, C]. The residual
    add (gpt.py:40-41) and the next RMSNorm (norm.py:6-19) over prompt rows."""
    _require_cuda(x, weight)
    if x.dtype != torch.float32 or weight.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("add_rmsnorm_rows takes a contiguous fp32 residual x [M, C] and fp32 weight [C]")
    M, C = x.shape
    lda = 0
    if addend is not None:
        if addend.dtype != torch.bfloat16 or addend.shape != (M, C) or addend.stride(1) != 1:
            raise ValueError("addend must be bf16 [M, C] with unit column stride")
        lda = addend.stride(0)
    if out is None:
        out = torch.empty(M, C, dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().tt_add_rmsnorm_rows_bf16(_ptr(x), _ptr(addend), lda, _ptr(weight), float(eps), _ptr(out),
                                                      M, C, _stream(x.device)), "add_rmsnorm_rows")
    return out


def silu_mul_rows(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(bf16(silu(g)) * u) from the bf16 gate and up projection outputs
    [M, I] (unit column stride; mlp.py:44-45 under autocast)."""
    _require_cuda(gate, up)
    for name, t in (("gate", gate), ("up", up)):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"{name} must be bf16 [M, I] with unit column stride")
    if up.shape != gate.shape:
        raise ValueError("gate and up must have one shape")
    M, inter = gate.shape
    if out is None:
        out = torch.empty(M, inter, dtype=torch.bfloat16, device=gate.device)
    _lib.check(_lib.load().tt_silu_mul_rows_bf16(_ptr(gate), gate.stride(0), _ptr(up), up.stride(0), M, inter,
                                                   _ptr(out), _stream(gate.device)), "silu_mul_rows")
    return out


def silu_mul(partials: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(bf16(silu(g)) * u) from partials [S, M, 2I] of a stacked gate|up projection (mlp.py:44-45)."""
    _require_cuda(partials)
    S, M, I2 = partials.shape
    inter = I2 // 2
    if out is None:
        out = torch.empty(M, inter, dtype=torch.bfloat16, device=partials.device)
    _lib.check(_lib.load().tt_silu_mul_bf16(_ptr(partials), S, M, inter, _ptr(out), _stream(partials.device)),
               "silu_mul")
    return out


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """[2I, K]: the gate and up weights [I, K] with rows interleaved by 8 (rows
    16j .. 16j+7 = gate rows 8j .. 8j+7, rows 16j+8 .. 16j+15 = up rows 8j ..
    8j+7), the row order linear_swiglu's packed weight takes."""
    inter, K = gate.shape
    if up.shape != gate.shape or inter % 8:
        raise ValueError("gate and up must both be [I, K] with I % 8 == 0")
    return torch.stack([gate.reshape(inter // 8, 8, K), up.reshape(inter // 8, 8, K)], dim=1).reshape(2 * inter, K)


def swiglu_supported(K: int, inter: int) -> bool:
    """Whether linear_swiglu takes this K and intermediate size."""
    return bool(_lib.load().tt_swiglu_gemm_supported(int(K), int(inter)))


def linear_swiglu(x: torch.Tensor, weight: "PackedWeight", out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(bf16(silu(bf16 g)) * bf16 u) [M, I] with g = x @ Wg^T, u = x @ Wu^T in
    fp32 over the whole K, in one launch (mlp.py:24-26, 44-45 under autocast).
    ``weight`` is PackedWeight(interleave_gate_up(Wg, Wu))."""
    if not isinstance(weight, PackedWeight):
        raise ValueError("linear_swiglu takes a PackedWeight of interleave_gate_up(gate, up)")
    _require_cuda(x, weight.data)
    if x.dtype != torch.bfloat16 or weight.data.dtype != torch.bfloat16:
        raise ValueError("linear_swiglu takes bf16 x and weight")
    M, ldx = _rows(x, "x")
    N, K = weight.shape
    if x.shape[1] != K or N % 2:
        raise ValueError(f"x {tuple(x.shape)} does not match the weight {weight.shape}")
    inter = N // 2
    if out is None:
        out = torch.empty(M, inter, dtype=torch.bfloat16, device=x.device)
    if out.dtype != torch.bfloat16 or out.shape != (M, inter) or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{M}, {inter}] with a contiguous last dimension")
    st = _lib.load().tt_linear_swiglu_packed_bf16(_ptr(x), ldx, _ptr(weight.data), _ptr(out), out.stride(0), M,
                                                  inter, K, _stream(x.device))
    _lib.check(st, "linear_swiglu")
    return out


def prefill_attention(q: torch.Tensor, layout: KVLayout, positions: torch.Tensor, max_seq_len: int,
                      new_lens: torch.Tensor | None = None, out: torch.Tensor | None = None,
                      sm_scale: float | None = None) -> torch.Tensor:
    """Causal GQA attention of T new tokens per sequence over its cache (after rope_append).

    q [B, H_q, T, D] bf16 (rotated; any strides with D contiguous),
    positions int32 [B] = tokens cached before the new ones, new_lens int32
    [B] (optional) = new tokens per sequence; returns out [B, T, H_q, D]
    (rows t >= new_lens[b] untouched). Restates the prefill branch of the
    reference attention (attn.py:321-341) for a ragged batch."""
    _require_cuda(q, layout.k, layout.v, positions)
    _check_lastdim("q", q, 4)
    if q.dtype != torch.bfloat16 or layout.kind not in ("bf16", "fp8"):
        raise ValueError("prefill_attention takes bf16 q with a bf16 or fp8 cache")
    B, Hq, T, D = q.shape
    if D != layout.head_dim:
        raise ValueError(f"head_dim {D} does not match the cache's {layout.head_dim}")
    if positions.dtype != torch.int32 or positions.shape != (B,):
        raise ValueError("positions must be int32 [B]")
    if new_lens is not None and (new_lens.dtype != torch.int32 or new_lens.shape != (B,)):
        raise ValueError("new_lens must be int32 [B]")
    if max_seq_len > layout.capacity:
        raise ValueError(f"max_seq_len {max_seq_len} exceeds the cache capacity {layout.capacity}")
    if out is None:
        out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=q.device)
    _check_lastdim("out", out, 4)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    lib = _lib.load()
    head = [_ptr(q), _lib.strides(*q.stride()[:3]), _ptr(layout.k), _ptr(layout.v)]
    tail = [_lib.strides(*layout.strides), _ptr(positions), _ptr(new_lens), int(max_seq_len),
            _ptr(layout.page_table), layout.max_pages, layout.num_pages,
            _ptr(out), _lib.strides(*out.stride()[:3]), B, T, Hq, layout.num_heads, D, layout.page_size,
            float(sm_scale), _stream(q.device)]
    if layout.kind == "fp8":
        st = lib.tt_prefill_attn_fp8(*head, _ptr(layout.k_scale), _ptr(layout.v_scale), *tail)
    else:
        st = lib.tt_prefill_attn_bf16(*head, *tail)
    _lib.check(st, "prefill_attention")
    return out


SAMPLE_MAX_VOCAB = {torch.bfloat16: 65536, torch.float32: 32768}


_SAMPLE_WS = {}  # (device index, stream) -> Workspace of the sampler's candidate path


def sample_tokens(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                  top_p: float | None = None, seed: int = 0, offset: int = 0, return_logprob: bool = False,
                  return_logprobs: bool = False, out: torch.Tensor | None = None,
                  workspace: Workspace | None = None):
    """One token per row of ``logits`` [M, V] (bf16 or fp32, last dim contiguous).

    filter_logits + sample_next_token / sample_next_token_with_log_prob
    (tinytron/inference/sampler.py:6-62) in one kernel launch: temperature,
    top-k, top-p, then top_k == 1 takes the first maximum and otherwise a
    draw from softmax(filtered) keyed by (seed, offset, row). Returns tokens
    int64 [M]; with ``return_logprob`` also the chosen tokens' log-probabilities
    [M]; with ``return_logprobs`` also log_softmax of the filtered logits
    [M, V] (-inf where filtered). With 2 <= top_k <= 64 over more than 8192
    logits, each 8192-logit chunk of a row is reduced to its top-k candidates
    by a workgroup of its own first (``workspace``, by default one per device
    and stream)."""
    _require_cuda(logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a 2-D view [M, V] with a contiguous last dimension")
    if logits.dtype not in SAMPLE_MAX_VOCAB:
        raise ValueError(f"logits must be bf16 or fp32, got {logits.dtype}")
    M, V = logits.shape
    dev = logits.device
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.shape != (M,) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 [M] tensor")
    lp = torch.empty(M, dtype=torch.float32, device=dev) if return_logprob else None
    full = torch.empty(M, V, dtype=torch.float32, device=dev) if return_logprobs else None
    lib = _lib.load()
    stream = _stream(dev)
    need = 0 if return_logprobs else int(lib.tt_sample_workspace_bytes(M, V, int(top_k or 0)))
    ws = None
    if need:
        if workspace is None:
            workspace = _SAMPLE_WS.setdefault((dev.index, stream), Workspace(dev))
        ws = workspace.get(need)
    fn = lib.tt_sample_bf16 if logits.dtype == torch.bfloat16 else lib.tt_sample_f32
    st = fn(_ptr(logits), logits.stride(0), M, V, float(temperature), int(top_k or 0),
            1.0 if top_p is None else float(top_p), int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1),
            _ptr(out), _ptr(lp), _ptr(full), V, _ptr(ws), 0 if ws is None else ws.numel(), stream)
    _lib.check(st, "sample_tokens")
    res = (out,)
    if return_logprob:
        res += (lp,)
    if return_logprobs:
        res += (full,)
    return res[0] if len(res) == 1 else res
