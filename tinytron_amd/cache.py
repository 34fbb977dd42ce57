"""KV caches for the gfx950 decode path.

Drop-in counterparts of tinytron/inference/cache.py:

* ``LayerPagedKVCache`` keeps the reference's constructor
  ``(batch_size, num_heads, head_dim, max_seq_len, page_size, device, dtype)``,
  storage ``[B, H, ceil(S/P), P, D]`` with the flat view
  ``[B, H, ceil(S/P)*P, D]`` (cache.py:27-32), ``append(k, v) -> previous
  length`` with the reference's overflow ``ValueError`` (cache.py:34-45),
  ``get_kv()`` (cache.py:47-51) and ``current_length``. It is built with
  ``num_heads = num_key_value_heads``: K/V are appended before the GQA
  expansion, so the cache holds each KV head once and the attention kernel
  maps query head h to KV head h // (H_q / H_kv).
* ``PagedLayerKVCache`` is a physical page pool ``[num_pages, H, P, D]``
  addressed through an int32 page table ``[B, max_pages]`` (no counterpart in
  the reference, whose "paged" store is dense).
* ``PagedKVCache`` is the model-level list with ``from_model_config`` and
  ``get_layer_cache`` (cache.py:54-97).

Beyond the reference protocol both layer caches keep one length per sequence
(the reference has one batch-wide ``current_length``, cache.py:26) in two
device int32 buffers that alternate between steps (the fused append writes
the new lengths into the other buffer, so no separate increment runs), with a
host mirror for overflow checks and launch sizing. The fused path is
``rope_append`` + ``attend``; ``append``/``get_kv`` are the reference
protocol for callers that bring their own attention.
"""
from __future__ import annotations

import math

import torch

from . import ops

FP8 = torch.float8_e4m3fn


def cache_kind(dtype: torch.dtype) -> str:
    if dtype == torch.bfloat16:
        return "bf16"
    if dtype == torch.float32:
        return "f32"
    if dtype == FP8:
        return "fp8"
    raise ValueError(f"unsupported KV cache dtype {dtype}")


def _quantize_rows(x: torch.Tensor):
    """Per-(token, head) fp8 quantization: scale = absmax/448, code = e4m3(x/scale)."""
    xf = x.float()
    scale = xf.abs().amax(dim=-1) / 448.0
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    codes = (xf / safe[..., None]).to(FP8).view(torch.uint8)
    codes = torch.where((scale > 0)[..., None], codes, torch.zeros_like(codes))
    return codes, scale


class _LayerCacheBase:
    """Length bookkeeping and the fused append/attend path shared by both layouts."""

    def _init_lengths(self, batch_size: int, device) -> None:
        self.batch_size = batch_size
        self._lens_dev = [torch.zeros(batch_size, dtype=torch.int32, device=device),
                          torch.zeros(batch_size, dtype=torch.int32, device=device)]
        self._cur = 0
        self._caps = None  # per-sequence capacities, filled on first use
        self._host_lens = [0] * batch_size
        self._pending_new_lens = None
        self.workspace = None
        self.static_max_len = None  # graph capture: launch-size bound fixed at the capacity
        self._split = None  # ops.pick_split over the base lengths, computed on first use after they change
        self._order = None  # the paired partition's length order (_order_buf once filled), with _split
        self._order_buf = None  # device int32 [B]: one buffer for the cache's life, so captured graphs keep it

    # -- lengths ---------------------------------------------------------------
    @property
    def seq_lens(self) -> torch.Tensor:
        """Device int32 [B]: tokens cached per sequence."""
        return self._lens_dev[self._cur]

    # Host lengths are base + shift: a one-token step adds 1 to every sequence
    # by bumping the shift, so the per-layer bookkeeping of a decode step does
    # not walk the batch.
    @property
    def _host_lens(self) -> list:
        return [x + self._shift for x in self._base] if self._shift else list(self._base)

    @_host_lens.setter
    def _host_lens(self, lens) -> None:
        self._base = [int(x) for x in lens]
        self._shift = 0
        self._base_max = max(self._base) if self._base else 0
        self._room = None  # min over b of capacity - base, recomputed on demand
        self._split = None

    def _advance_all(self, n: int) -> None:
        self._shift += n

    @property
    def seq_lens_host(self) -> list:
        return self._host_lens

    @property
    def current_length(self) -> int:
        """Longest sequence; equals the reference's batch-wide length when lengths are uniform."""
        return self._base_max + self._shift if self._base else 0

    def capacity_of(self, b: int) -> int:
        raise NotImplementedError

    def _check_room(self, adds) -> None:
        if self._caps is None:
            self._caps = [self.capacity_of(b) for b in range(self.batch_size)]
        if self._room is None:
            self._room = min((c - x for c, x in zip(self._caps, self._base)), default=0)
        if adds and min(adds) == max(adds) and int(adds[0]) <= self._room - self._shift:
            return  # the same add everywhere, and every sequence has room for it
        lens = self._host_lens
        for b, add in enumerate(adds):
            end = lens[b] + int(add)
            cap = self._caps[b]
            if end > cap:
                raise ValueError(f"KV cache overflow: requested sequence length {end}, max supported is {cap}")

    def set_lengths(self, lens) -> None:
        """Declare that sequence b holds lens[b] tokens (e.g. after external writes)."""
        lens = [int(x) for x in lens]
        for b, n in enumerate(lens):
            if n < 0 or n > self.capacity_of(b):
                raise ValueError(f"KV cache overflow: requested sequence length {n}, max supported is {self.capacity_of(b)}")
        self._host_lens = lens
        self.seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))

    def set_pending_new_lens(self, new_lens) -> None:
        """Ragged prefill: the next multi-token append writes only new_lens[b] tokens of sequence b."""
        self._pending_new_lens = None if new_lens is None else [int(x) for x in new_lens]

    # -- fused path ------------------------------------------------------------
    def rope_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rope_table: torch.Tensor,
                    new_lens=None) -> torch.Tensor:
        """RoPE + append in one kernel at each sequence's own position; returns rotated q.

        rope_impl (attn.py:13-63) + append (cache.py:34-45) with per-sequence
        positions; raises the reference's overflow ValueError before launching.
        """
        T = q.shape[2]
        if new_lens is None and T > 1:
            new_lens = self._pending_new_lens
        adds = [T] * self.batch_size if new_lens is None else [min(int(n), T) for n in new_lens]
        self._check_room(adds)
        nl = None
        if new_lens is not None:
            nl = torch.tensor(adds, dtype=torch.int32).to(self.seq_lens.device, non_blocking=True)
        nxt = 1 - self._cur
        q_rot = ops.rope_append(q, k, v, rope_table, self._lens_dev[self._cur], self.layout, new_lens=nl,
                                lens_out=self._lens_dev[nxt])
        self._cur = nxt
        self._host_lens = [a + b for a, b in zip(self._host_lens, adds)]
        return q_rot

    def rope_append_rows(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rope_table: torch.Tensor,
                         new_lens, row_offsets: torch.Tensor, num_new: int) -> torch.Tensor:
        """rope_append of a packed prompt batch (q [N, H_q, D], k / v [N, H_kv, D];
        sequence b's new_lens[b] tokens are rows row_offsets[b] ...); returns the
        rotated q on the [B, H_q, num_new, D] grid."""
        adds = [int(n) for n in new_lens]
        self._check_room(adds)
        nl = torch.tensor(adds, dtype=torch.int32).to(self.seq_lens.device, non_blocking=True)
        nxt = 1 - self._cur
        q_rot = ops.rope_append_rows(q, k, v, rope_table, self._lens_dev[self._cur], self.layout, row_offsets, nl,
                                     num_new, lens_out=self._lens_dev[nxt])
        self._cur = nxt
        self._host_lens = [a + b for a, b in zip(self._host_lens, adds)]
        return q_rot

    def rope_append_partials(self, partials: torch.Tensor, num_q_heads: int, rope_table: torch.Tensor) -> torch.Tensor:
        """One-token rope_append whose q|k|v are the split-K partials [S, B, N]
        of the stacked q|k|v projection (summed and rounded inside the kernel)."""
        self._check_room([1] * self.batch_size)
        nxt = 1 - self._cur
        q_rot = ops.rope_append_partials(partials, num_q_heads, rope_table, self._lens_dev[self._cur], self.layout,
                                         lens_out=self._lens_dev[nxt])
        self._cur = nxt
        self._advance_all(1)
        return q_rot

    def decode_step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rope_table: torch.Tensor,
                    out: torch.Tensor | None = None) -> torch.Tensor:
        """One-token RoPE + append + attention in one launch pair from bf16
        q [B, H_q, D] and k / v [B, H_kv, D]; returns out [B, H_q, D] (the
        two-launch rope_append + attend, bit for bit)."""
        return self._decode_step(rope_table, out, q=q, k=k, v=v)

    def decode_step_partials(self, partials: torch.Tensor, num_q_heads: int, rope_table: torch.Tensor,
                             out: torch.Tensor | None = None) -> torch.Tensor:
        """As decode_step with q|k|v given as the split-K partials [S, B, N] of
        the stacked projection (summed and rounded inside the kernel)."""
        return self._decode_step(rope_table, out, partials=partials, num_q_heads=num_q_heads)

    def _attention_split(self) -> int:
        """split_tokens of this cache's decode attention (ops.pick_split over
        the host lengths): the per-segment partition while every sequence has
        the same length, the paired one for a ragged batch whose rank pairs
        fill the GPU evenly (both one launch, merged in LDS), else the
        balanced partition (0). Decode steps add the same count to every
        length, which changes neither equality nor the ranks, so the pick is
        made once per change of the base lengths."""
        if self._split is None:
            lay = self.layout
            split = ops.pick_split(self._base, lay.num_heads, lay.head_dim, lay.kind)
            if split == ops.SPLIT_PAIRED and not torch.cuda.is_current_stream_capturing():
                # the rank order, once per change of the lengths (a step adds the same count to
                # every length): the kernel reads its pair instead of ranking the batch itself.
                # Written in place into one buffer, so a graph captured with it reads the current
                # order; any permutation gives correct results (a stale one only pairs worse).
                # Under graph capture no host copy can be recorded: the buffer keeps its last
                # order, or the kernel ranks on the device while there is none.
                if self._order_buf is None:
                    self._order_buf = torch.empty(self.batch_size, dtype=torch.int32, device=lay.k.device)
                self._order_buf.copy_(torch.tensor(ops.length_order(self._base), dtype=torch.int32))
                self._order = self._order_buf
            self._split = split
        return self._split

    def _decode_step(self, rope_table, out, **inputs) -> torch.Tensor:
        self._check_room([1] * self.batch_size)
        if self.workspace is None:
            self.workspace = ops.Workspace(rope_table.device)
        bound = self.static_max_len if self.static_max_len is not None else self.current_length + 1
        nxt = 1 - self._cur
        split = self._attention_split()
        out = ops.decode_attention_append(rope_table, self._lens_dev[self._cur], self.layout, bound,
                                          lens_out=self._lens_dev[nxt], out=out, workspace=self.workspace,
                                          split_tokens=split, length_order=self._order, **inputs)
        self._cur = nxt
        self._advance_all(1)
        return out

    def begin_decode_step(self):
        """For a caller that issues this layer's one-token decode step itself
        (the model's one-call layer sequence): checks that every sequence has
        room for one more token and returns (positions, lens_out, bound,
        split_tokens, length_order), the arguments decode_step would pass: the
        lengths before the step, the buffer the kernel writes the lengths
        after it into, the launch bound, the attention partition and its rank
        order (or None). Follow the launch with advance_host(1)."""
        self._check_room([1] * self.batch_size)
        bound = self.static_max_len if self.static_max_len is not None else self.current_length + 1
        split = self._attention_split()
        return self._lens_dev[self._cur], self._lens_dev[1 - self._cur], bound, split, self._order

    def prefill_attend(self, q_rot: torch.Tensor, new_lens, out: torch.Tensor | None = None,
                       kernel: bool = True) -> torch.Tensor:
        """Causal attention of the chunk just appended by rope_append (q_rot
        [B, H_q, T, D], new_lens[b] tokens of sequence b) over each sequence's
        cache; returns [B, T, H_q, D]. bf16 activations over a bf16 / fp8 cache
        whose rows are whole 16-byte fragments take the prefill kernel (rows
        past new_lens[b] untouched); fp32 and the other head dims take row
        attention, one query row per new token (rows past new_lens[b] zero;
        ``kernel=False`` takes it for every case)."""
        lay = self.layout
        T = q_rot.shape[2]
        if kernel and q_rot.dtype == torch.bfloat16 and lay.kind in ("bf16", "fp8") \
                and ops.attention_tile_dim(lay.head_dim, lay.kind) \
                and q_rot.shape[1] // lay.num_heads <= 16:
            prev = self._lens_dev[1 - self._cur]  # the lengths before the append (the other buffer)
            nl = torch.tensor([int(n) for n in new_lens], dtype=torch.int32).to(prev.device, non_blocking=True)
            return ops.prefill_attention(q_rot, lay, prev, self.current_length, new_lens=nl, out=out)
        adds = [min(int(n), T) for n in new_lens]
        cached = [x - a for x, a in zip(self._host_lens, adds)]
        if self.workspace is None:
            self.workspace = ops.Workspace(q_rot.device)
        return ops.prefill_attention_rows(q_rot, lay, cached, adds, out=out, workspace=self.workspace)

    def attend(self, q: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """GQA decode attention of q [B, H_q, D] over every cached token of each sequence."""
        if self.workspace is None:
            self.workspace = ops.Workspace(q.device)
        bound = self.static_max_len if self.static_max_len is not None else self.current_length
        split = self._attention_split()
        return ops.decode_attention(q, self.layout, self.seq_lens, bound, out=out, workspace=self.workspace,
                                    split_tokens=split, length_order=self._order)

    # -- host-state snapshots for graph capture ------------------------------------
    def host_state(self):
        return (list(self._host_lens), self._cur, self._split)

    def set_host_state(self, state) -> None:
        self._host_lens, self._cur = list(state[0]), state[1]
        # the lengths are those the partition was picked for (and the length order uploaded):
        # keep the pick rather than pick and upload again
        self._split = state[2]

    def advance_host(self, n: int = 1) -> None:
        """Mirror a replayed one-token step: lengths + n, length buffers swapped n times."""
        self._advance_all(n)
        self._cur = (self._cur + n) & 1

    # -- gathers for the protocol / prefill ----------------------------------------
    def _token_index(self, b: int, length: int) -> torch.Tensor:
        """Element offsets [length] of tokens 0..length-1 of sequence b, head 0, d 0."""
        raise NotImplementedError

    def gather(self, b: int, length: int, dtype: torch.dtype | None = None):
        """Dense (K, V) [1, H, length, D] of sequence b (dequantized for fp8).
        ``length`` may not exceed the sequence's capacity (ValueError)."""
        lay = self.layout
        D, H = lay.head_dim, lay.num_heads
        if length < 0 or length > self.capacity_of(b):
            raise ValueError(f"cannot gather {length} tokens of sequence {b}: it holds at most {self.capacity_of(b)}")
        base = self._token_index(b, length)                                   # [L]
        idx = base[None, :, None] + (torch.arange(H, device=base.device) * lay.strides[2])[:, None, None] \
            + torch.arange(D, device=base.device)[None, None, :]              # [H, L, D]
        if lay.kind == "fp8":
            sidx = ops.fp8_scale_index((base[None, :] + (torch.arange(H, device=base.device) * lay.strides[2])[:, None])
                                       // D)
            k = lay.k[idx].view(FP8).float() * lay.k_scale[sidx][..., None]
            v = lay.v[idx].view(FP8).float() * lay.v_scale[sidx][..., None]
            dt = dtype or torch.bfloat16
            return k.to(dt)[None], v.to(dt)[None]
        return lay.k[idx][None], lay.v[idx][None]

    def _write_tokens(self, b: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """k/v [H, T, D] into slots start..start+T-1 of sequence b (no RoPE)."""
        lay = self.layout
        D, H = lay.head_dim, lay.num_heads
        T = k.shape[1]
        base = self._token_index(b, start + T)[start:]
        idx = base[None, :, None] + (torch.arange(H, device=base.device) * lay.strides[2])[:, None, None] \
            + torch.arange(D, device=base.device)[None, None, :]
        if lay.kind == "fp8":
            sidx = ops.fp8_scale_index((base[None, :] + (torch.arange(H, device=base.device) * lay.strides[2])[:, None])
                                       // D)
            kc, ks = _quantize_rows(k)
            vc, vs = _quantize_rows(v)
            lay.k[idx] = kc
            lay.v[idx] = vc
            lay.k_scale[sidx] = ks
            lay.v_scale[sidx] = vs
        else:
            lay.k[idx] = k.to(lay.k.dtype)
            lay.v[idx] = v.to(lay.v.dtype)

    # -- reference protocol -------------------------------------------------------
    def append(self, k: torch.Tensor, v: torch.Tensor) -> int:
        """cache.py:34-45: write k/v [B, H, T, D] after each sequence's tokens, return the previous length."""
        T = k.size(2)
        self._check_room([T] * self.batch_size)
        previous = self.current_length
        for b in range(self.batch_size):
            self._write_tokens(b, self._host_lens[b], k[b], v[b])
        self.set_lengths([n + T for n in self._host_lens])
        return previous

    def get_kv(self):
        """cache.py:47-51: (K, V) [B, H, current_length, D] (dense copies for the
        pool and fp8). With ragged lengths (which the reference's one batch-wide
        length cannot express) sequence b contributes its own lens[b] tokens and
        zeros after them; no slot past a sequence's length is read."""
        L = self.current_length
        ks, vs = [], []
        for b, n in enumerate(self._host_lens):
            k, v = self.gather(b, n)
            if n < L:
                pad = (0, 0, 0, L - n)
                k, v = torch.nn.functional.pad(k, pad), torch.nn.functional.pad(v, pad)
            ks.append(k)
            vs.append(v)
        return torch.cat(ks, 0), torch.cat(vs, 0)


class LayerPagedKVCache(_LayerCacheBase):
    """The reference's per-layer store (cache.py:11-51), H = num_key_value_heads."""

    def __init__(self, batch_size: int, num_heads: int, head_dim: int, max_seq_len: int, page_size: int,
                 device, dtype: torch.dtype) -> None:
        if page_size <= 0:
            raise ValueError(f"page_size must be positive, got {page_size}")
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        kind = cache_kind(dtype)
        num_pages = math.ceil(max_seq_len / page_size)
        if kind == "fp8":  # its scales group 16 rows: a (sequence, head) holds a multiple of 16 token slots
            while (num_pages * page_size) % 16:
                num_pages += 1
        shape = (batch_size, num_heads, num_pages, page_size, head_dim)
        store = torch.uint8 if kind == "fp8" else dtype
        self._k_pages = torch.empty(shape, device=device, dtype=store)
        self._v_pages = torch.empty(shape, device=device, dtype=store)
        self._k_flat = self._k_pages.view(batch_size, num_heads, num_pages * page_size, head_dim)
        self._v_flat = self._v_pages.view(batch_size, num_heads, num_pages * page_size, head_dim)
        k_scale = v_scale = None
        if kind == "fp8":
            k_scale, v_scale = ops.fp8_scales(math.prod(shape[:-1]), device)
        pd = page_size * head_dim
        self.layout = ops.KVLayout(
            k=self._k_pages.view(-1), v=self._v_pages.view(-1),
            strides=(num_heads * num_pages * pd, pd, num_pages * pd), num_heads=num_heads, head_dim=head_dim,
            page_size=page_size, capacity=max_seq_len, kind=kind, k_scale=k_scale, v_scale=v_scale)
        self._init_lengths(batch_size, device)

    def capacity_of(self, b: int) -> int:
        return self.max_seq_len

    def _token_index(self, b: int, length: int) -> torch.Tensor:
        lay = self.layout
        t = torch.arange(length, device=lay.k.device)
        return b * lay.strides[0] + t * lay.head_dim

    def get_kv(self):
        if self.layout.kind != "fp8" and len(set(self._host_lens)) == 1:
            L = self.current_length
            return self._k_flat[:, :, :L, :], self._v_flat[:, :, :L, :]
        return super().get_kv()


class PagedLayerKVCache(_LayerCacheBase):
    """Physical page pool [num_pages, H, P, D] + page table [B, max_pages] (int32).

    Sequence b's token t lives in physical page page_table[b, t // P] at slot
    t % P. Page size must be a power of two >= 16 (one 16-token MFMA block
    never straddles a page).
    """

    def __init__(self, page_table: torch.Tensor, num_pages: int, num_heads: int, head_dim: int, page_size: int,
                 device, dtype: torch.dtype) -> None:
        if page_size <= 0:
            raise ValueError(f"page_size must be positive, got {page_size}")
        if page_size < 16 or page_size & (page_size - 1):
            raise ValueError(f"paged pools need a power-of-two page_size >= 16, got {page_size}")
        kind = cache_kind(dtype)
        self.page_size = page_size
        self.num_pages = num_pages
        table_cpu = page_table.to(torch.int32).cpu()
        if table_cpu.dim() != 2:
            raise ValueError("page_table must be [B, max_pages]")
        # a sequence owns the leading run of valid entries of its row (its capacity)
        self._pages_of = [int(torch.cumprod((row >= 0).to(torch.int64), 0).sum()) for row in table_cpu]
        if table_cpu.numel() and int(table_cpu.max()) >= num_pages:
            raise ValueError("page_table refers to pages beyond the pool")
        self.page_table = table_cpu.to(device)
        store = torch.uint8 if kind == "fp8" else dtype
        shape = (num_pages, num_heads, page_size, head_dim)
        self._k = torch.empty(shape, device=device, dtype=store)
        self._v = torch.empty(shape, device=device, dtype=store)
        k_scale = v_scale = None
        if kind == "fp8":
            k_scale, v_scale = ops.fp8_scales(math.prod(shape[:-1]), device)
        self.layout = ops.KVLayout(
            k=self._k.view(-1), v=self._v.view(-1), strides=(0, num_heads * page_size * head_dim, page_size * head_dim),
            num_heads=num_heads, head_dim=head_dim, page_size=page_size,
            capacity=int(table_cpu.shape[1]) * page_size, kind=kind, page_table=self.page_table,
            num_pages=num_pages, k_scale=k_scale, v_scale=v_scale)
        self.max_seq_len = self.layout.capacity
        self._init_lengths(int(table_cpu.shape[0]), device)

    def capacity_of(self, b: int) -> int:
        return self._pages_of[b] * self.page_size

    def _token_index(self, b: int, length: int) -> torch.Tensor:
        if length > self.capacity_of(b):  # beyond the sequence's pages the table holds -1
            raise ValueError(f"sequence {b} owns {self._pages_of[b]} pages; {length} tokens do not fit")
        lay = self.layout
        t = torch.arange(length, device=lay.k.device)
        phys = self.page_table[b].long()[t // self.page_size]
        return phys * lay.strides[1] + (t % self.page_size) * lay.head_dim


def random_page_table(capacities, page_size: int, seed: int = 1337, extra_pages: int = 0):
    """Pages for each sequence's capacity, assigned in (sequence, logical page)
    order from a seeded random permutation of the pool. Unused entries are -1.
    Returns (page_table int32 [B, max_pages] on the CPU, num_pages)."""
    need = [max(1, math.ceil(int(c) / page_size)) for c in capacities]
    total = sum(need) + extra_pages
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    table = torch.full((len(need), max(need) if need else 1), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[off:off + n]
        off += n
    return table, total


class PagedKVCache:
    """Model-level cache: one layer cache per transformer layer (cache.py:54-97)."""

    def __init__(self, layer_caches) -> None:
        self._layer_caches = list(layer_caches)
        ws = None
        for c in self._layer_caches:  # layers run one after another on one stream
            if ws is None:
                ws = ops.Workspace(c.layout.k.device)
            c.workspace = ws

    @classmethod
    def from_model_config(cls, model_config, batch_size: int, page_size: int, device, dtype: torch.dtype,
                          *, kv_cache_dtype: torch.dtype | None = None, seq_capacity=None,
                          paged_pool: bool = False, page_seed: int = 1337) -> "PagedKVCache":
        """As cache.py:58-94 with num_heads = num_key_value_heads.

        ``kv_cache_dtype`` (default: ``dtype``) may be torch.float8_e4m3fn.
        ``paged_pool`` builds a page pool per layer sharing one seeded random
        page table sized for ``seq_capacity`` (tokens per sequence, default
        block_size).
        """
        heads = model_config.num_key_value_heads
        head_dim = model_config.hidden_size // model_config.num_attention_heads
        cdt = kv_cache_dtype or dtype
        if not paged_pool:
            layers = [LayerPagedKVCache(batch_size, heads, head_dim, model_config.block_size, page_size, device, cdt)
                      for _ in range(model_config.num_layer)]
            return cls(layers)
        caps = seq_capacity if seq_capacity is not None else [model_config.block_size] * batch_size
        table, n_pages = random_page_table(caps, page_size, seed=page_seed)
        layers = [PagedLayerKVCache(table, n_pages, heads, head_dim, page_size, device, cdt)
                  for _ in range(model_config.num_layer)]
        return cls(layers)

    def get_layer_cache(self, layer_idx: int):
        return self._layer_caches[layer_idx]

    def __len__(self) -> int:
        return len(self._layer_caches)

    def set_pending_new_lens(self, new_lens) -> None:
        for c in self._layer_caches:
            c.set_pending_new_lens(new_lens)

    def host_state(self):
        return [c.host_state() for c in self._layer_caches]

    def set_host_state(self, states) -> None:
        for c, st in zip(self._layer_caches, states):
            c.set_host_state(st)

    def advance_host(self, n: int = 1) -> None:
        for c in self._layer_caches:
            c.advance_host(n)

    def set_static_max_len(self, n) -> None:
        """Fix every layer's attention launch bound (split size, grid, workspace) at n
        tokens, so one captured step stays valid while lengths grow; None restores
        bounds taken from the current lengths."""
        for c in self._layer_caches:
            c.static_max_len = n

    def parity(self) -> int:
        """Which of the two device length buffers holds the current lengths (same in every layer)."""
        return self._layer_caches[0]._cur

    def check_room(self, add: int) -> None:
        """Raise the reference's overflow error unless every sequence can take ``add`` more tokens."""
        for c in self._layer_caches:
            c._check_room([add] * c.batch_size)


class ConcatKVStore:
    """Device store behind the reference's non-paged cache: the per-layer tuple
    (k, v) of GQA-expanded heads [B, H_q, T, D] that attn.py:174-186 grows by
    torch.cat at every call (engine.py:168-178 with use_paged_kv_cache=False).

    The tuples handed out are views ``[:, :, :length]`` of a contiguous
    [B, H_q, capacity, D] store that the kernels address as a contiguous
    [B, H, pages, 16, D] cache with H = H_q (one KV head per query head, as
    the expanded tensors are). A call that continues the newest tuple appends
    in place; one that continues an older or a foreign tuple gets a new store
    with that tuple copied in, so earlier tuples keep the values they had (the
    reference's torch.cat never changes its inputs). Capacity grows by
    doubling (16-token pages)."""

    PAGE = 16

    def __init__(self) -> None:
        self.k = self.v = None
        self.length = 0
        self.capacity = 0
        self.layout = None

    def _owns(self, past) -> bool:
        k, v = past
        return (self.k is not None and k.data_ptr() == self.k.data_ptr() and v.data_ptr() == self.v.data_ptr()
                and k.shape[2] == self.length and k.stride() == self.k.stride() and v.stride() == self.v.stride())

    def _allocate(self, B: int, H: int, D: int, capacity: int, dtype, device) -> None:
        cap = -(-capacity // self.PAGE) * self.PAGE
        self.k = torch.empty(B, H, cap, D, dtype=dtype, device=device)
        self.v = torch.empty(B, H, cap, D, dtype=dtype, device=device)
        self.capacity = cap
        self.layout = ops.KVLayout(k=self.k.view(-1), v=self.v.view(-1), strides=(H * cap * D, self.PAGE * D, cap * D),
                                   num_heads=H, head_dim=D, page_size=self.PAGE, capacity=cap,
                                   kind=cache_kind(dtype))

    def prepare(self, past, B: int, H: int, D: int, add: int, dtype, device) -> int:
        """Make room for `add` tokens after `past` (None or a (k, v) tuple
        [B, H, T_past, D]); returns T_past."""
        if past is None:
            t_past = 0
        else:
            k, v = past
            if k.dim() != 4 or k.shape[:2] != (B, H) or k.shape[3] != D or v.shape != k.shape:
                raise ValueError(f"past key/value shapes {tuple(k.shape)} / {tuple(v.shape)} do not match "
                                 f"[{B}, {H}, T, {D}]")
            t_past = int(k.shape[2])
        need = t_past + add
        fits = self.k is not None and self.k.shape[:2] == (B, H) and self.k.dtype == dtype and \
            self.k.device == torch.device(device) and need <= self.capacity
        if past is not None and self._owns(past) and fits:
            return t_past  # continue the newest tuple in place
        old_k = old_v = None
        if past is not None:
            old_k, old_v = past
        self._allocate(B, H, D, max(need, 2 * self.capacity if self.k is not None else need), dtype, device)
        if t_past:
            self.k[:, :, :t_past].copy_(old_k)
            self.v[:, :, :t_past].copy_(old_v)
        return t_past

    def views(self, length: int):
        """The (k, v) tuple of the first `length` tokens; they become the newest."""
        self.length = length
        return self.k[:, :, :length], self.v[:, :, :length]
