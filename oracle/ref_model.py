"""torch-CPU restatement of the reference's dense GPT and generate loop
(test infrastructure; end-to-end token parity and the E2E CPU baseline).

Follows tinytron/model/gpt.py:33-115, modules/norm.py:14-19,
modules/mlp.py:44-45, modules/attn.py:378-440 (local decode path with the
H_q-expanded LayerPagedKVCache) and inference/engine.py:144-228 (greedy via
top_k = 1), op for op. Weights come from a state dict.

Two numeric modes:

* fp32 (default): the reference's CPU path, which runs without autocast
  (engine.py:180-184).
* ``autocast_bf16=True``: the reference on the GPU under
  torch.autocast(bfloat16) (engine.py:180-185), with autocast's rounding
  points made explicit: every projection (F.linear) takes bf16-rounded
  inputs and weights, accumulates in fp32 and returns bf16; RoPE, the cache
  and SiLU * up run in bf16; SDPA (an autocast bf16 op) attends over the
  bf16 q / K / V in fp32 and returns bf16; the embedding, the residual
  stream and RMSNorm stay fp32 (x + bf16 promotes to fp32; norm.py:14-19
  computes in fp32 and multiplies by the fp32 weight). Pinned in
  tests/test_oracle_ref_model.py against the fp32 code run under torch's own
  CPU autocast, so the rounding points come from torch's autocast policy.
"""
from __future__ import annotations

import time

import torch
import torch.nn.functional as F

from . import ref_path

BF16 = torch.bfloat16


class RefGPT:
    def __init__(self, state_dict: dict, num_layer: int, num_attention_heads: int, num_key_value_heads: int,
                 dtype=torch.float32, autocast_bf16: bool = False):
        self.w = {k: v.detach().to("cpu", dtype) for k, v in state_dict.items() if torch.is_tensor(v)}
        self.L = num_layer
        self.hq = num_attention_heads
        self.hkv = num_key_value_heads
        self.C = self.w["wte.weight"].shape[1]
        self.D = self.C // self.hq
        self.bf16 = autocast_bf16
        if autocast_bf16:  # bf16 copies of the projection weights (autocast's per-call weight cast)
            self.wb = {k: v.to(BF16).float() for k, v in self.w.items() if k.endswith("_proj.weight")}
            self.wb["wte.weight"] = self.w["wte.weight"].to(BF16).float()

    def _lin(self, x, name):
        """nn.Linear(bias=False): fp32, or autocast's bf16 in / fp32 accumulate / bf16 out."""
        if not self.bf16:
            return F.linear(x, self.w[name])
        return F.linear(x.to(BF16).float(), self.wb[name]).to(BF16)

    def _sdpa(self, q, k, v, mask, causal):
        if not self.bf16:
            return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=0.0, is_causal=causal)
        y = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask, dropout_p=0.0,
                                           is_causal=causal)
        return y.to(BF16)

    @staticmethod
    def _rms(x, w):
        x32 = x.to(torch.float32)
        var = x32.pow(2).mean(-1, keepdim=True)
        return w * (x32 * torch.rsqrt(var + 1e-6)).to(x.dtype)

    def _attn(self, i, x, cache, position_offset):
        B, T, C = x.shape
        p = f"blocks.{i}.attn."
        q = self._lin(x, p + "q_proj.weight").view(B, T, self.hq, self.D).transpose(-2, -3)
        k = self._lin(x, p + "k_proj.weight").view(B, T, self.hkv, self.D).transpose(-2, -3)
        v = self._lin(x, p + "v_proj.weight").view(B, T, self.hkv, self.D).transpose(-2, -3)
        pos = torch.arange(position_offset, position_offset + T).unsqueeze(0)
        q, k = ref_path.rope_impl(q, k, pos)
        k, v = ref_path.gqa_impl(k, v, self.hkv, self.hq)
        if isinstance(cache, list):
            # use_paged_kv_cache=False (engine.py:168-178): cache[0] is None or the
            # layer's past (K, V); the new tokens are concatenated to it and the
            # result becomes the layer's past (attn.py:174-186, 330-331, 437-440)
            past = cache[0]
            past_len = 0 if past is None else past[0].size(2)
            if past is not None:
                k, v = torch.cat([past[0], k], dim=2), torch.cat([past[1], v], dim=2)
            cache[0] = (k, v)
        else:
            past_len = cache.append(k, v)
            k, v = cache.get_kv()
        mask, causal = None, True
        if past_len > 0:
            mask = ref_path.build_cache_causal_mask(T, k.size(2), past_len, x.device)
            causal = False
        y = self._sdpa(q, k, v, mask, causal)
        y = y.transpose(-2, -3).reshape(B, T, C)
        return self._lin(y, p + "c_proj.weight")

    def forward(self, idx, caches, position_offset):
        x = F.embedding(idx, self.w["wte.weight"])
        for i in range(self.L):
            p = f"blocks.{i}."
            x = x + self._attn(i, self._rms(x, self.w[p + "ln_1.weight"]), caches[i], position_offset)
            h = self._rms(x, self.w[p + "ln_2.weight"])
            m = self._lin(F.silu(self._lin(h, p + "mlp.gate_proj.weight")) * self._lin(h, p + "mlp.up_proj.weight"),
                          p + "mlp.down_proj.weight")
            x = x + m
        x = self._rms(x, self.w["lnf.weight"])
        if not self.bf16:
            return F.linear(x, self.w["wte.weight"])
        return F.linear(x.to(BF16).float(), self.wb["wte.weight"]).to(BF16)  # tied lm_head (gpt.py:61-63)

    def new_caches(self, batch: int, block_size: int, page_size: int = 128, tuple_cache: bool = False):
        """One reference LayerPagedKVCache per layer (cache.py:54-97), or with
        ``tuple_cache`` one [past] holder per layer for the concatenating path."""
        if tuple_cache:
            return [[None] for _ in range(self.L)]
        dt = BF16 if self.bf16 else torch.float32
        return [ref_path.LayerPagedKVCache(batch, self.hq, self.D, block_size, page_size, "cpu", dt)
                for _ in range(self.L)]

    @torch.no_grad()
    def generate_greedy(self, prompt: torch.Tensor, max_new_tokens: int, block_size: int, page_size: int = 128,
                        max_steps_timed: int | None = None, tuple_cache: bool = False):
        """engine.py:144-228 with temperature 1, top_k 1 (argmax); ``tuple_cache``
        runs use_paged_kv_cache=False. Returns (tokens [B, T + n], decode
        tokens/s, logits of every step)."""
        B, T = prompt.shape
        caches = self.new_caches(B, block_size, page_size, tuple_cache)
        logits = self.forward(prompt, caches, 0)
        tokens = [prompt]
        step_logits = [logits[:, -1].clone()]
        cur = T
        t0 = time.perf_counter()
        steps = 0
        for _ in range(max_new_tokens):
            nxt = torch.argmax(logits[:, -1].float(), dim=-1)
            tokens.append(nxt[:, None])
            cur += 1
            steps += 1
            logits = self.forward(nxt[:, None], caches, cur - 1)
            step_logits.append(logits[:, -1].clone())
            if max_steps_timed is not None and steps >= max_steps_timed:
                break
        dt = time.perf_counter() - t0
        return torch.cat(tokens, 1), B * steps / dt, step_logits
