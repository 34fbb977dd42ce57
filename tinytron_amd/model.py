"""Dense GQA GPT around the gfx950 decode path.

Mirrors the reference's model stack (tinytron/model/gpt.py:20-115,
modules/attn.py:102-440, modules/norm.py:6-19, modules/mlp.py:16-45,
config.py:7-29) with the same module names, parameter names, shapes, seeded
init and forward signatures, so state dicts load unchanged and the engine's
model call (engine.py:188, 220-225) is the same.

Numerics follow the reference under bf16 autocast (engine.py:180-185)
without autocast's per-call weight casts: projection weights are stored in
the compute dtype, the residual stream, norms and the embedding stay fp32,
and every projection takes bf16 inputs and returns bf16 -- the values
autocast produces from fp32 weights.

``Attention.forward`` is the drop-in of attn.py:378-440: with one of this
package's caches, a decode step (T = 1) is one split-K GQA attention launch
pair that also applies RoPE to the step's token and appends it to the cache
(fp32 caches: a RoPE + append kernel, then the attention kernels); prefill
(T > 1) writes the cache with the RoPE + append kernel and attends with the
prefill kernel (bf16 activations; SDPA per sequence for fp32). No CPU
fallback.

``GPT.forward`` runs a bf16 decode step (T = 1) as a fused layer sequence
when the shapes allow it (``GPT.fused_decode``): per layer, one skinny
split-K GEMM for the stacked q|k|v projection, the attention launch pair
(which sums those partials, applies RoPE and appends k / v itself), the
c_proj GEMM, residual add + RMSNorm in one kernel, one GEMM for the stacked
gate|up projection, SwiGLU, the down GEMM, and the next residual add +
RMSNorm -- 9 launches instead of about 30 (bf16 and fp8 caches), with the
same math and bf16 rounding points as the module path. A bf16 prefill with
``logits_index`` (the engine's) runs on the packed prompt tokens
(``GPT.fused_prefill``): the projections, residual add + RMSNorm and SwiGLU
see only the sum(new_lens) real tokens, not the B x T padded grid.
"""
from __future__ import annotations

import ctypes
import math
import weakref
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, ops
from .cache import ConcatKVStore, LayerPagedKVCache, PagedLayerKVCache


@dataclass(frozen=True)
class ModelConfig:
    """config.py:7-29 (the dense fields the decode path uses)."""

    seed: int = 1337
    block_size: int = 4096
    vocab_size: int = 50304
    num_layer: int = 32
    num_attention_heads: int = 128
    num_key_value_heads: int = 8
    hidden_size: int = 1024
    intermediate_size: int = 4096
    dropout: float = 0.0
    init_std: float = 0.013
    tied_lm_head: bool = True
    rope_theta: float = 10000.0


_ROPE_TABLES: dict = {}


def rope_table_for(n_positions: int, head_dim: int, theta: float, dtype: torch.dtype, device) -> torch.Tensor:
    """Shared cos/sin table (attn.py:30-54) covering at least n_positions."""
    key = (str(torch.device(device)), head_dim, float(theta), dtype)
    t = _ROPE_TABLES.get(key)
    if t is None or t.shape[0] < n_positions:
        n = max(n_positions, 4096 if t is None else 2 * t.shape[0])
        t = ops.build_rope_table(n, head_dim, theta, dtype=dtype, device=device)
        _ROPE_TABLES[key] = t
    return t


def _same_objects(refs, objs) -> bool:
    """Whether weak references (None for None) still name exactly these objects."""
    return len(refs) == len(objs) and all((o is None) if r is None else (r() is o) for r, o in zip(refs, objs))


def _is_fused_cache(past_kv) -> bool:
    return isinstance(past_kv, (LayerPagedKVCache, PagedLayerKVCache))


class Attention(nn.Module):
    """attn.py:102-440 (single-GPU path) with the fused gfx950 decode step."""

    def __init__(self, config: ModelConfig, layer_idx: int, device=None, dtype=torch.float32):
        super().__init__()
        assert config.hidden_size % config.num_attention_heads == 0
        self.config = config
        self.layer_idx = layer_idx
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        if self.num_attention_heads % self.num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        self.head_dim = config.hidden_size // config.num_attention_heads
        self.n_embd = config.hidden_size
        kw = dict(bias=False, device=device, dtype=dtype)
        self.q_proj = nn.Linear(config.hidden_size, self.num_attention_heads * self.head_dim, **kw)
        self.k_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, **kw)
        self.v_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, **kw)
        self.c_proj = nn.Linear(config.hidden_size, config.hidden_size, **kw)
        self.prefill_kernel = True  # bf16 prefill through the prefill attention kernel (else row attention)
        self._concat = None  # ConcatKVStore behind the non-paged (tuple) cache, made on first use
        self._init_weights(config.seed, layer_idx)

    def _init_weights(self, base_seed: int, layer_idx: int) -> None:
        """attn.py:148-160: every projection of layer i drawn after seeding seed + i."""
        for lin in (self.q_proj, self.k_proj, self.v_proj, self.c_proj):
            g = torch.Generator(device=lin.weight.device).manual_seed(base_seed + layer_idx)
            with torch.no_grad():
                w = torch.empty(lin.weight.shape, dtype=torch.float32, device=lin.weight.device)
                w.normal_(0.0, self.config.init_std, generator=g)
                lin.weight.copy_(w)

    def forward(self, x: torch.Tensor, past_kv=None, use_cache: bool = False, position_offset: int = 0):
        B, T, C = x.size()
        act = self.q_proj.weight.dtype
        xa = x.to(act)
        q = self.q_proj(xa).view(B, T, self.num_attention_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(xa).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(xa).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        if not _is_fused_cache(past_kv):
            return self._forward_concat(q, k, v, past_kv, use_cache, position_offset)
        lens = past_kv.seq_lens_host
        if len(set(lens)) == 1 and lens[0] != position_offset:
            raise ValueError(f"position_offset {position_offset} does not match the cache length {lens[0]}")
        table = rope_table_for(past_kv.max_seq_len + T, self.head_dim, self.config.rope_theta, act, x.device)
        if T == 1 and act == torch.bfloat16 and past_kv.layout.kind in ("bf16", "fp8") \
                and ops.attention_tile_dim(self.head_dim, past_kv.layout.kind):
            y = past_kv.decode_step(q[:, :, 0], k[:, :, 0], v[:, :, 0], table)  # RoPE + append + attention
            y = y.view(B, 1, C)
        elif T == 1:
            q_rot = past_kv.rope_append(q, k, v, table)                     # [B, H_q, 1, D]
            y = past_kv.attend(q_rot.view(B, self.num_attention_heads, self.head_dim))
            y = y.view(B, 1, C)
        else:
            y = self._prefill(q, k, v, past_kv, table, lens)
        y = self.c_proj(y)
        return y, (past_kv if use_cache else None)

    def _forward_concat(self, q, k, v, past_kv, use_cache: bool, position_offset: int):
        """The reference's non-paged paths (attn.py:174-186, 314-341): past_kv
        None or the (k, v) tuple of GQA-expanded heads [B, H_q, T_past, D];
        returns the new tuple [B, H_q, T_past + T, D] with use_cache (else
        None). RoPE + append of the new tokens (k / v expanded first, as the
        reference appends after gqa_impl) into the layer's ConcatKVStore, then
        decode attention (T = 1) or causal prefill attention over it with one
        KV head per query head."""
        B, Hq, T, D = q.shape
        act = q.dtype
        if self._concat is None:
            self._concat = ConcatKVStore()
        store = self._concat
        t_past = store.prepare(past_kv, B, Hq, D, T, act, q.device)
        if position_offset != t_past:
            raise ValueError(f"position_offset {position_offset} does not match the cached length {t_past}")
        G = Hq // self.num_key_value_heads
        ke = k.repeat_interleave(G, dim=1) if G > 1 else k
        ve = v.repeat_interleave(G, dim=1) if G > 1 else v
        table = rope_table_for(t_past + T, D, self.config.rope_theta, act, q.device)
        pos = torch.full((B,), t_past, dtype=torch.int32, device=q.device)
        q_rot = ops.rope_append(q, ke, ve, table, pos, store.layout)
        if T == 1:
            y = ops.decode_attention(q_rot.view(B, Hq, D), store.layout, pos + 1, t_past + 1).view(B, 1, self.n_embd)
        elif self.prefill_kernel and act == torch.bfloat16 and ops.attention_tile_dim(D, store.layout.kind):
            y = ops.prefill_attention(q_rot, store.layout, pos, t_past + T).view(B, T, self.n_embd)
        else:
            y = ops.prefill_attention_rows(q_rot, store.layout, [t_past] * B, [T] * B).view(B, T, self.n_embd)
        new_kv = store.views(t_past + T) if use_cache else None
        return self.c_proj(y), new_kv

    def _prefill(self, q, k, v, cache, table, lens_before):
        """T > 1: append all (ragged) prompt tokens with the fused kernel, then
        causal attention over each sequence's cached prefix (attn.py:321-341):
        the prefill kernel for bf16 activations, row attention (one query row
        per new token) for fp32 and the head dims that kernel does not take."""
        B, _, T, D = q.shape
        new = cache._pending_new_lens or [T] * B
        q_rot = cache.rope_append(q, k, v, table, new_lens=new)
        y = torch.zeros(B, T, self.n_embd, dtype=q.dtype, device=q.device)
        cache.prefill_attend(q_rot, new, out=y.view(B, T, self.num_attention_heads, D), kernel=self.prefill_kernel)
        return y


class RMSNorm(nn.Module):
    """norm.py:6-19 (named LayerNorm in the reference): fp32 math, eps 1e-6."""

    def __init__(self, config: ModelConfig, device=None):
        super().__init__()
        self.variance_epsilon = 1e-6
        self.weight = nn.Parameter(torch.ones(config.hidden_size, device=device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        input_dtype = x.dtype
        x = x.to(torch.float32)
        variance = x.pow(2).mean(-1, keepdim=True)
        x = x * torch.rsqrt(variance + self.variance_epsilon)
        return self.weight * x.to(input_dtype)


class MLP(nn.Module):
    """mlp.py:16-45: SwiGLU, seeded like the attention projections."""

    def __init__(self, config: ModelConfig, layer_idx: int, device=None, dtype=torch.float32):
        super().__init__()
        kw = dict(bias=False, device=device, dtype=dtype)
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, **kw)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, **kw)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, **kw)
        self.act_fn = nn.SiLU()
        for lin in (self.gate_proj, self.up_proj, self.down_proj):
            g = torch.Generator(device=lin.weight.device).manual_seed(config.seed + layer_idx)
            with torch.no_grad():
                w = torch.empty(lin.weight.shape, dtype=torch.float32, device=lin.weight.device)
                w.normal_(0.0, config.init_std, generator=g)
                lin.weight.copy_(w)

    def forward(self, x: torch.Tensor, use_cache: bool = False) -> torch.Tensor:
        xa = x.to(self.gate_proj.weight.dtype)
        return self.down_proj(self.act_fn(self.gate_proj(xa)) * self.up_proj(xa))


class Block(nn.Module):
    """gpt.py:20-45 (dense)."""

    def __init__(self, config: ModelConfig, layer_idx: int, device=None, dtype=torch.float32):
        super().__init__()
        self.ln_1 = RMSNorm(config, device)
        self.attn = Attention(config, layer_idx, device, dtype)
        self.ln_2 = RMSNorm(config, device)
        self.mlp = MLP(config, layer_idx, device, dtype)

    def forward(self, x, past_kv=None, use_cache=False, position_offset=0):
        attn_out, new_kv = self.attn(self.ln_1(x), past_kv=past_kv, use_cache=use_cache,
                                     position_offset=position_offset)
        x = x + attn_out
        x = x + self.mlp(self.ln_2(x), use_cache=use_cache)
        return x, None, new_kv


class GPT(nn.Module):
    """gpt.py:49-115 (dense, inference). ``dtype`` is the compute dtype of the
    projections; the embedding table and the residual stream stay fp32 and the
    tied lm_head uses a ``dtype`` copy of it, as autocast would."""

    def __init__(self, config: ModelConfig, device=None, dtype=torch.float32):
        super().__init__()
        self.config = config
        self.compute_dtype = dtype
        self.wte = nn.Embedding(config.vocab_size, config.hidden_size, device=device)
        self.blocks = nn.ModuleList([Block(config, i, device, dtype) for i in range(config.num_layer)])
        self.lnf = RMSNorm(config, device)
        g = torch.Generator(device=self.wte.weight.device).manual_seed(config.seed)
        with torch.no_grad():
            self.wte.weight.normal_(0.0, config.init_std, generator=g)
        if not config.tied_lm_head:
            raise ValueError("only the tied lm_head of the reference's default config is supported")
        self._lm_head_weight = None
        self.fused_decode = True   # bf16 decode steps through the fused layer kernels when shapes allow
        self.fused_prefill = True  # bf16 ragged prefill over the packed prompt tokens when shapes allow
        self._stacked = {}         # layer -> (source key, packed q|k|v, c_proj, gate|up, down weights)
        self._stacked_rows = {}    # layer -> (source key, plain q|k|v weight, plain gate|up weight)
        self._decode_bufs = {}     # (device, rows) -> split-K partial buffer
        self.native_decode_step = True  # the fused step's layer sequence issued in one library call
        self._native_plans = {}    # length-buffer parity -> (scalars, cache objects, model objects, array, buffers)
        self._native_bufs = {}     # (device, rows) -> residual x, norm output h, attention output, SwiGLU output
        self._native_ws = {}       # device -> workspace of the balanced attention partition

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        # reference checkpoints carry the tied lm_head as its own key (gpt.py:60-62)
        state_dict.pop(prefix + "lm_head.weight", None)
        self._lm_head_weight = None
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    def lm_head_weight(self) -> torch.Tensor:
        w = self._lm_head_weight
        if w is None or w.device != self.wte.weight.device or w.dtype != self.compute_dtype:
            w = self.wte.weight.detach().to(self.compute_dtype)
            self._lm_head_weight = w
        return w

    # -- fused bf16 decode step ------------------------------------------------------
    @staticmethod
    def _k_chunk(k: int) -> int:
        return 512 if k % 512 == 0 else (256 if k % 256 == 0 else 0)

    @staticmethod
    def _k_chunk_wide(k: int) -> int:
        """Split for the gate|up GEMM: its N fills every CU at 1024-wide chunks,
        which halve the partials that SwiGLU reads."""
        return 1024 if k % 1024 == 0 else GPT._k_chunk(k)

    @staticmethod
    def _k_chunk_small(k: int) -> int:
        """Split for the square c_proj GEMM: more, shorter splits keep every CU streaming."""
        return 256 if k % 256 == 0 else 0

    def _fused_decode_ok(self, cache, B: int) -> bool:
        c = self.config
        if not self.fused_decode or self.compute_dtype != torch.bfloat16 or not self.wte.weight.is_cuda:
            return False
        D = c.hidden_size // c.num_attention_heads
        n_qkv = (c.num_attention_heads + 2 * c.num_key_value_heads) * D
        return (c.hidden_size <= 8192 and n_qkv % 64 == 0
                and (2 * c.intermediate_size) % 64 == 0 and self._k_chunk(c.hidden_size) > 0
                and self._k_chunk_small(c.hidden_size) > 0 and self._k_chunk(c.intermediate_size) > 0
                and all(_is_fused_cache(cache.get_layer_cache(i)) for i in range(len(self.blocks))))

    def _stacked_weights(self, i: int):
        """Layer i's decode GEMM weights in the kernels' fragment order: q|k|v
        and gate|up stacked row-wise, c_proj, down (rebuilt when a source
        parameter changes: its storage or its in-place version counter)."""
        blk = self.blocks[i]
        srcs = (blk.attn.q_proj.weight, blk.attn.k_proj.weight, blk.attn.v_proj.weight, blk.attn.c_proj.weight,
                blk.mlp.gate_proj.weight, blk.mlp.up_proj.weight, blk.mlp.down_proj.weight)
        key = tuple((t.data_ptr(), t._version) for t in srcs)
        ent = self._stacked.get(i)
        if ent is None or ent[0] != key:
            with torch.no_grad():
                gu = (ops.interleave_gate_up(srcs[4], srcs[5]) if self._swiglu_fused()
                      else torch.cat(srcs[4:6]))
                ent = (key, ops.PackedWeight(torch.cat(srcs[:3])), ops.PackedWeight(srcs[3]),
                       ops.PackedWeight(gu), ops.PackedWeight(srcs[6]))
            self._stacked[i] = ent
        return ent[1:]

    def _swiglu_fused(self) -> bool:
        """gate|up + SwiGLU as one whole-K launch (ops.linear_swiglu) where the
        kernel takes the shape; else split-K partials + ops.silu_mul."""
        c = self.config
        return ops.swiglu_supported(c.hidden_size, c.intermediate_size)

    def _stacked_plain(self, i: int):
        """Layer i's q|k|v and gate|up weights stacked row-wise (plain bf16) for
        the prefill GEMMs: one wide product instead of three / two (rebuilt when
        a source parameter changes)."""
        blk = self.blocks[i]
        srcs = (blk.attn.q_proj.weight, blk.attn.k_proj.weight, blk.attn.v_proj.weight,
                blk.mlp.gate_proj.weight, blk.mlp.up_proj.weight)
        key = tuple((t.data_ptr(), t._version) for t in srcs)
        ent = self._stacked_rows.get(i)
        if ent is None or ent[0] != key:
            with torch.no_grad():
                ent = (key, torch.cat(srcs[:3]).contiguous(), torch.cat(srcs[3:]).contiguous())
            self._stacked_rows[i] = ent
        return ent[1:]

    def _partials(self, device, B: int) -> torch.Tensor:
        c = self.config
        D = c.hidden_size // c.num_attention_heads
        n_qkv = (c.num_attention_heads + 2 * c.num_key_value_heads) * D
        sizes = [(c.hidden_size // self._k_chunk(c.hidden_size)) * n_qkv,
                 (c.hidden_size // self._k_chunk_wide(c.hidden_size)) * 2 * c.intermediate_size,
                 (c.hidden_size // self._k_chunk_small(c.hidden_size)) * c.hidden_size,
                 (c.intermediate_size // self._k_chunk(c.intermediate_size)) * c.hidden_size]
        need = B * max(sizes)
        key = (str(device), B)
        buf = self._decode_bufs.get(key)
        if buf is None or buf.numel() < need:
            buf = torch.empty(need, dtype=torch.float32, device=device)
            self._decode_bufs[key] = buf
        return buf

    def _decode_step_fused(self, idx: torch.Tensor, cache, position_offset: int) -> torch.Tensor:
        """One decode step (gpt.py:84-115 with attn.py:378-440, mlp.py:44-45,
        norm.py:6-19 per layer) through the fused layer kernels; [B, 1, V] logits."""
        c = self.config
        B = idx.shape[0]
        C, Hq, Hkv = c.hidden_size, c.num_attention_heads, c.num_key_value_heads
        D = C // Hq
        eps = self.lnf.variance_epsilon
        kc_c, kc_i, kc_o = self._k_chunk(C), self._k_chunk(c.intermediate_size), self._k_chunk_small(C)
        kc_gu = self._k_chunk_wide(C)
        swiglu_fused = self._swiglu_fused()
        first = cache.get_layer_cache(0)
        lens = first.seq_lens_host
        if len(set(lens)) == 1 and lens[0] != position_offset:
            raise ValueError(f"position_offset {position_offset} does not match the cache length {lens[0]}")
        table = rope_table_for(first.max_seq_len + 1, D, c.rope_theta, torch.bfloat16, idx.device)
        pbuf = self._partials(idx.device, B)
        if self.native_decode_step and C // kc_c <= ops.FUSED_STEP_MAX_SPLITS and all(
                cache.get_layer_cache(i).layout.kind in ("bf16", "fp8")
                and ops.attention_tile_dim(D, cache.get_layer_cache(i).layout.kind) for i in range(len(self.blocks))):
            logits = self._decode_step_native(idx, cache, table, pbuf)
            if logits is not None:
                return logits.view(B, 1, -1)
        x = self.wte(idx).view(B, C).float().contiguous()          # fp32 residual stream
        h = ops.add_rmsnorm(x, self.blocks[0].ln_1.weight, eps)      # bf16 [B, C]
        for i, blk in enumerate(self.blocks):
            layer = cache.get_layer_cache(i)
            wqkv, wo, wgu, wd = self._stacked_weights(i)
            P = ops.linear_partials(h, wqkv, partials=pbuf, k_chunk=kc_c)
            if P.shape[0] <= ops.FUSED_STEP_MAX_SPLITS and layer.layout.kind in ("bf16", "fp8") \
                    and ops.attention_tile_dim(D, layer.layout.kind):
                y = layer.decode_step_partials(P, Hq, table)        # RoPE + append + attention, [B, Hq, D]
            else:
                q_rot = layer.rope_append_partials(P, Hq, table)     # sums the q|k|v partials itself
                y = layer.attend(q_rot.view(B, Hq, D))
            P = ops.linear_partials(y.view(B, C), wo, partials=pbuf, k_chunk=kc_o)
            h = ops.add_rmsnorm(x, blk.ln_2.weight, eps, partials=P)
            if swiglu_fused:
                a = ops.linear_swiglu(h, wgu)                        # [B, I], one launch, no partials
            else:
                a = ops.silu_mul(ops.linear_partials(h, wgu, partials=pbuf, k_chunk=kc_gu))
            P = ops.linear_partials(a, wd, partials=pbuf, k_chunk=kc_i)
            nxt = self.blocks[i + 1].ln_1.weight if i + 1 < len(self.blocks) else self.lnf.weight
            h = ops.add_rmsnorm(x, nxt, eps, partials=P)             # residual add + next norm (or lnf)
        logits = F.linear(h, self.lm_head_weight())
        return logits.view(B, 1, -1)

    def _decode_step_native(self, idx: torch.Tensor, cache, table: torch.Tensor, pbuf: torch.Tensor):
        """_decode_step_fused's layer sequence (every layer's cache taking the
        one-launch-pair attention step) issued by the library in one call,
        tt_decode_layers_bf16: the same kernels with the same arguments, so
        the same logits bit for bit, for about a third of the host time. The
        argument array is built once per cache, length-buffer parity,
        partition, weights and buffers, and checked against them every step.
        Returns the [B, V] logits, or None (then the per-op path runs) when the
        layers do not share one launch bound. A library error is raised with
        the layer it names; the layers before it have appended the step's
        token but their host lengths are not advanced (reset the cache)."""
        c = self.config
        B = idx.shape[0]
        C, Hq, Hkv, I = c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.intermediate_size
        D = C // Hq
        dev = idx.device
        n = len(self.blocks)
        layers = [cache.get_layer_cache(i) for i in range(n)]
        steps = [layer.begin_decode_step() for layer in layers]   # (positions, lens_out, bound, split, order)
        bound = steps[0][2]
        if any(st[2] != bound for st in steps):
            return None
        for layer in layers:
            if not 1 <= bound <= layer.layout.capacity:
                raise ValueError(f"max_seq_len {bound} must be in [1, capacity {layer.layout.capacity}]")
        ws_ptr = ws_n = 0
        if any(st[3] == 0 for st in steps):  # the balanced partition's split-K workspace, shared by the layers
            need = ops.workspace_bytes(B, Hq, Hkv, D, bound, 0)
            ws = self._native_ws.get(str(dev))
            if ws is None:
                ws = self._native_ws[str(dev)] = ops.Workspace(dev)
            buf = ws.get(need)
            ws_ptr, ws_n = buf.data_ptr(), buf.numel()
        weights = [self._stacked_weights(i) for i in range(n)]
        norms = [blk.ln_2.weight for blk in self.blocks] + [blk.ln_1.weight for blk in self.blocks[1:]] \
            + [self.lnf.weight]
        scalars = (B, table.data_ptr(), table.shape[0], pbuf.data_ptr(), ws_ptr, ws_n, tuple(st[3] for st in steps))
        cached = [o for layer, st in zip(layers, steps) for o in (layer.layout, st[0], st[4])]  # the cache's objects
        owned = [pw for w in weights for pw in w] + norms                                    # the model's objects
        plan = self._native_plans.get(layers[0]._cur)
        if plan is None or plan[0] != scalars or not _same_objects(plan[1], cached) \
                or len(plan[2]) != len(owned) or any(a is not b for a, b in zip(plan[2], owned)):
            arr, bufs = self._native_plan(layers, steps, weights, table, pbuf, ws_ptr, ws_n, dev, B)
            # the cache's objects are held weakly (a plan must not keep a finished cache alive), the
            # model's strongly (their identities cannot be reused while the plan compares them)
            plan = (scalars, [None if o is None else weakref.ref(o) for o in cached], owned, arr, bufs)
            self._native_plans[layers[0]._cur] = plan
        arr, (x, h) = plan[3], plan[4][:2]
        x.copy_(self.wte(idx).view(B, C))                                   # fp32 residual stream
        ops.add_rmsnorm(x, self.blocks[0].ln_1.weight, self.lnf.variance_epsilon, out=h)
        _lib.check(_lib.load().tt_decode_layers_bf16(ctypes.addressof(arr), n, bound, ops._stream(dev)),
                   "decode step")
        for layer in layers:
            layer.advance_host(1)
        return F.linear(h, self.lm_head_weight())

    def _native_plan(self, layers, steps, weights, table, pbuf, ws_ptr, ws_n, dev, B):
        """The tt_decode_layer_t array of one decode step and the model-owned
        buffers it points at (residual x, norm output h, attention output,
        SwiGLU output)."""
        c = self.config
        C, Hq, Hkv, I = c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.intermediate_size
        D = C // Hq
        bkey = (str(dev), B)
        bufs = self._native_bufs.get(bkey)
        if bufs is None:
            bufs = (torch.empty(B, C, dtype=torch.float32, device=dev),
                    torch.empty(B, C, dtype=torch.bfloat16, device=dev),
                    torch.empty(B, Hq * D, dtype=torch.bfloat16, device=dev),
                    torch.empty(B, I, dtype=torch.bfloat16, device=dev))
            self._native_bufs[bkey] = bufs
        x, h, y, a = bufs
        n = len(layers)
        arr = (_lib.DecodeLayer * n)()
        kc_gu = 0 if self._swiglu_fused() else self._k_chunk_wide(C)
        for i, (layer, st, w) in enumerate(zip(layers, steps, weights)):
            lay = layer.layout
            nxt = self.blocks[i + 1].ln_1.weight if i + 1 < n else self.lnf.weight
            for t in (self.blocks[i].ln_2.weight, nxt):
                if t.dtype != torch.float32 or not t.is_contiguous():
                    raise ValueError("the fused decode step takes contiguous fp32 norm weights")
            L = arr[i]
            L.x, L.h, L.partials, L.attn_out, L.act = x.data_ptr(), h.data_ptr(), pbuf.data_ptr(), y.data_ptr(), \
                a.data_ptr()
            L.w_qkv, L.w_o, L.w_gu, L.w_down = (pw.data.data_ptr() for pw in w)
            L.ln2_weight, L.next_norm_weight = self.blocks[i].ln_2.weight.data_ptr(), nxt.data_ptr()
            L.eps = self.lnf.variance_epsilon
            L.batch, L.hidden, L.intermediate, L.num_q_heads, L.num_kv_heads, L.head_dim = B, C, I, Hq, Hkv, D
            L.kc_qkv, L.kc_o, L.kc_gu, L.kc_down = self._k_chunk(C), self._k_chunk_small(C), kc_gu, self._k_chunk(I)
            L.fp8_cache = 1 if lay.kind == "fp8" else 0
            L.rope_table, L.rope_table_len = table.data_ptr(), table.shape[0]
            L.positions, L.lens_out = st[0].data_ptr(), st[1].data_ptr()
            L.page_table = ops._ptr(lay.page_table)
            L.max_pages, L.num_pages = lay.max_pages, lay.num_pages
            L.k_cache, L.v_cache = lay.k.data_ptr(), lay.v.data_ptr()
            L.k_scale, L.v_scale = ops._ptr(lay.k_scale), ops._ptr(lay.v_scale)
            L.cache_strides[:] = [int(s) for s in lay.strides]
            L.capacity, L.page_size = lay.capacity, lay.page_size
            L.sm_scale = 1.0 / math.sqrt(D)
            L.split_tokens = st[3]
            L.length_order = ops._ptr(st[4])
            L.workspace, L.workspace_bytes = (ws_ptr, ws_n) if st[3] == 0 else (None, 0)
        return arr, bufs

    # -- packed bf16 prefill ---------------------------------------------------------
    def _fused_prefill_ok(self, cache, idx: torch.Tensor, logits_index: torch.Tensor) -> bool:
        c = self.config
        if not self.fused_prefill or self.compute_dtype != torch.bfloat16 or not self.wte.weight.is_cuda:
            return False
        D = c.hidden_size // c.num_attention_heads
        if not (c.hidden_size % 4 == 0 and c.hidden_size <= 8192
                and c.num_attention_heads // c.num_key_value_heads <= 16 and c.intermediate_size % 4 == 0
                and all(blk.attn.prefill_kernel for blk in self.blocks)
                and all(_is_fused_cache(cache.get_layer_cache(i))
                        and ops.attention_tile_dim(D, cache.get_layer_cache(i).layout.kind)
                        for i in range(len(self.blocks)))):
            return False
        # every requested logit row must be one of the sequence's new tokens
        B, T = idx.shape
        new = cache.get_layer_cache(0)._pending_new_lens or [T] * B
        li = logits_index.reshape(-1).tolist()
        return len(li) == B and all(0 <= int(i) < min(int(n), T) for i, n in zip(li, new))

    def _prefill_fused(self, idx: torch.Tensor, cache, position_offset: int, logits_index: torch.Tensor) -> torch.Tensor:
        """Prefill of a ragged batch (gpt.py:84-115 over T prompt tokens, of
        which sequence b brings new_lens[b]) on the packed tokens only: the
        projections and the norm / SwiGLU kernels see sum(new_lens) rows instead
        of B * T; the RoPE + append kernel reads the packed q / k / v rows and
        writes the rotated q on the [B, T] grid the prefill attention kernel
        reads (padding rows are never written or read). Same math and bf16
        rounding points as the module path; returns the logits at
        logits_index[b] of each sequence, [B, 1, V]."""
        c = self.config
        B, T = idx.shape
        C, Hq, Hkv = c.hidden_size, c.num_attention_heads, c.num_key_value_heads
        D = C // Hq
        dev = idx.device
        first = cache.get_layer_cache(0)
        lens = first.seq_lens_host
        if len(set(lens)) == 1 and lens[0] != position_offset:
            raise ValueError(f"position_offset {position_offset} does not match the cache length {lens[0]}")
        new = [min(int(n), T) for n in (first._pending_new_lens or [T] * B)]
        cu = [0]
        for n in new:
            cu.append(cu[-1] + n)
        sel = torch.cat([torch.arange(n, dtype=torch.int64) + b * T for b, n in enumerate(new)]).to(dev)
        rows = torch.tensor(cu[:-1], dtype=torch.int64, device=dev) + logits_index.to(dev, torch.int64)
        table = rope_table_for(first.max_seq_len + T, D, c.rope_theta, torch.bfloat16, dev)
        eps = self.lnf.variance_epsilon
        x = self.wte(idx.reshape(-1).index_select(0, sel)).float().contiguous()  # fp32 residual stream [N, C]
        h = ops.add_rmsnorm_rows(x, self.blocks[0].ln_1.weight, eps)             # bf16 [N, C]
        offs = torch.tensor(cu[:-1], dtype=torch.int32, device=dev)
        N = cu[-1]
        y_grid = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
        I = c.intermediate_size
        for i, blk in enumerate(self.blocks):
            layer = cache.get_layer_cache(i)
            att = blk.attn
            wqkv, wgu = self._stacked_plain(i)
            qkv = F.linear(h, wqkv)                                              # [N, (H_q + 2 H_kv) D]
            q_rot = layer.rope_append_rows(qkv[:, :Hq * D].view(N, Hq, D),
                                           qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D),
                                           qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D), table, new, offs, T)
            layer.prefill_attend(q_rot, new, out=y_grid)
            y = y_grid.view(B * T, C).index_select(0, sel)
            h = ops.add_rmsnorm_rows(x, blk.ln_2.weight, eps, addend=F.linear(y, att.c_proj.weight))
            gu = F.linear(h, wgu)                                                # [N, 2I]
            m = ops.silu_mul_rows(gu[:, :I], gu[:, I:])
            nxt = self.blocks[i + 1].ln_1.weight if i + 1 < len(self.blocks) else self.lnf.weight
            h = ops.add_rmsnorm_rows(x, nxt, eps, addend=F.linear(m, blk.mlp.down_proj.weight))
        return F.linear(h.index_select(0, rows), self.lm_head_weight()).unsqueeze(1)

    def _forward_concat(self, idx, past_key_values, use_cache: bool, position_offset: int, logits_index):
        """gpt.py:95-115 without a paged cache: past_key_values None (the
        uncached forward, or the first call of the non-paged cache) or the list
        of per-layer (k, v) tuples; returns logits, plus the new list with
        use_cache."""
        B, _ = idx.size()
        if past_key_values is not None and len(past_key_values) != len(self.blocks):
            raise ValueError(f"past_key_values holds {len(past_key_values)} layers, the model {len(self.blocks)}")
        x = self.wte(idx)
        new_past = [] if use_cache else None
        for layer_idx, block in enumerate(self.blocks):
            layer_past = past_key_values[layer_idx] if past_key_values is not None else None
            x, _, new_kv = block(x, past_kv=layer_past, use_cache=use_cache, position_offset=position_offset)
            if use_cache:
                new_past.append(new_kv)
        if logits_index is not None:
            x = x[torch.arange(B, device=x.device), logits_index].unsqueeze(1)
        x = self.lnf(x)
        logits = F.linear(x.to(self.compute_dtype), self.lm_head_weight())
        return (logits, new_past) if use_cache else logits

    def forward(self, idx: torch.Tensor, targets=None, past_key_values=None, use_cache: bool = False,
                position_offset: int = 0, logits_index: torch.Tensor | None = None):
        """gpt.py:84-115. ``logits_index`` ([B], optional, prefill only)
        computes logits at one position per sequence ([B, 1, V]) instead of
        all T."""
        B, T = idx.size()
        assert T <= self.config.block_size, f"Cannot forward sequence of length {T}, block size is only {self.config.block_size}"
        if targets is not None:
            raise NotImplementedError("tinytron_amd.GPT is the inference path: the training loss (targets) is not "
                                      "part of it")
        paged_cache = past_key_values if hasattr(past_key_values, "get_layer_cache") else None
        if paged_cache is None:
            return self._forward_concat(idx, past_key_values, use_cache, position_offset, logits_index)
        if T == 1 and logits_index is None and targets is None and self._fused_decode_ok(paged_cache, B):
            logits = self._decode_step_fused(idx, paged_cache, position_offset)
            return (logits, paged_cache) if use_cache else logits
        if T > 1 and logits_index is not None and targets is None and self._fused_prefill_ok(paged_cache, idx,
                                                                                             logits_index):
            logits = self._prefill_fused(idx, paged_cache, position_offset, logits_index)
            return (logits, paged_cache) if use_cache else logits
        x = self.wte(idx)
        for layer_idx, block in enumerate(self.blocks):
            x, _, _ = block(x, past_kv=paged_cache.get_layer_cache(layer_idx), use_cache=use_cache,
                            position_offset=position_offset)
        if logits_index is not None:
            x = x[torch.arange(B, device=x.device), logits_index].unsqueeze(1)
        x = self.lnf(x)
        logits = F.linear(x.to(self.compute_dtype), self.lm_head_weight())
        if use_cache:
            return logits, paged_cache
        return logits
