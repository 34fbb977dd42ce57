"""Autoregressive engine over the gfx950 decode path.

Restates ``InferenceEngine`` (tinytron/inference/engine.py:16-261): the same
constructor arguments, ``generate`` signature, prefill -> sample -> write
token -> one-token model call loop (engine.py:195-225), EOS handling and the
same statistics (decode tokens/s = B * decode steps / decode wall time,
engine.py:236-243). Added: ragged prompts (``prompt_lens``), KV caches that
hold H_kv heads, a paged pool with a seeded random page table, and fp8 KV.

Each step's model call is unchanged: ``model(next[B, 1], use_cache=True,
past_key_values=cache, position_offset=...)``; positions come from the
cache's per-sequence lengths, so there is no host synchronisation in the
loop (the reference syncs once per layer at attn.py:395).

With ``use_graphs=True`` the one-token model call is captured in HIP graphs
after the first decode step and replayed for the rest, which removes the
per-kernel launch cost; ``False`` launches every step eagerly. By default
(``None``) the engine times the second and third decode steps eagerly from
one synchronisation, and replays graphs only when the host needs at least
GRAPH_HOST_RATIO of those steps' GPU time to issue them: the fused bf16 step
issues 7 or 8 launches per layer, about as fast as a fast host issues them,
and the module-by-module step about 30.
The caches keep their lengths in two device buffers that swap every step, so
two graphs are captured, one per buffer parity. The attention launch bound is
fixed at the largest sequence capacity for the whole decode loop, so the
captured split size and grid stay valid as lengths grow (the kernels read
the actual lengths on the device). Sampling and the token write stay outside
the graphs, so every sampling mode works unchanged.
"""
from __future__ import annotations

import time

import torch

from .cache import PagedKVCache
from .model import GPT, ModelConfig
from .sampler import sample_next_token, sample_next_token_with_log_prob


# Launch mode of the default engine: replay graphs when issuing two eager
# steps takes the host at least this fraction of their GPU time. The ratio of
# a GPU-bound host is host / GPU time; a host-bound one reads ~0.97-0.99 (the
# GPU's time then is the host's plus the last kernels). Measured at C5 on a
# host issuing at 0.9-1.0x of the GPU: eager 31.3 k tokens/s against 30.3 k
# replayed (the two captures inside the loop); a host well below the GPU's
# pace gains from replay (26.8 k eager against 28.4 k replayed).
GRAPH_HOST_RATIO = 0.97


class DecodeGraphs:
    """Two captured one-token model calls (one per length-buffer parity)."""

    def __init__(self, model: GPT, cache: PagedKVCache, batch_size: int, position: int, uniform: bool,
                 device: torch.device):
        self.cache = cache
        self.static_in = torch.zeros(batch_size, 1, dtype=torch.long, device=device)
        self.graphs = {}
        self.logits = {}
        state = cache.host_state()
        pool = torch.cuda.graph_pool_handle()
        try:
            for k in range(2):
                parity = cache.parity()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool):
                    logits, _ = model(self.static_in, use_cache=True, past_key_values=cache,
                                      position_offset=(position + k) if uniform else 0)
                self.graphs[parity] = g
                self.logits[parity] = logits
        finally:
            cache.set_host_state(state)         # capture ran no kernel: undo its host-side advance

    def step(self, next_token: torch.Tensor) -> torch.Tensor:
        """One decode model call by replay; returns the logits [B, 1, V] it wrote."""
        self.cache.check_room(1)
        parity = self.cache.parity()
        self.static_in.copy_(next_token.view(-1, 1))
        self.graphs[parity].replay()
        self.cache.advance_host(1)
        return self.logits[parity]


class InferenceEngine:
    def __init__(self, model_config: ModelConfig, checkpoint_path: str | None = None, device: str = "cuda",
                 dtype: torch.dtype = torch.bfloat16, use_paged_kv_cache: bool = True, kv_cache_page_size: int = 128,
                 kv_cache_dtype: torch.dtype | None = None, paged_pool: bool = False, page_seed: int = 1337,
                 model: GPT | None = None, use_graphs: bool | None = None):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the tinytron_amd engine runs on the GPU (no CPU fallback)")
        if self.device.index is None:
            torch.cuda.set_device(0)
            self.device = torch.device("cuda:0")
        else:
            torch.cuda.set_device(self.device)
        if not use_paged_kv_cache and kv_cache_dtype is not None:
            raise ValueError("a kv_cache_dtype needs the paged KV cache (use_paged_kv_cache=True)")
        self.use_paged_kv_cache = use_paged_kv_cache
        self.model_config = model_config
        self.kv_cache_page_size = kv_cache_page_size
        self.kv_cache_dtype = kv_cache_dtype
        self.paged_pool = paged_pool
        self.page_seed = page_seed
        self.use_graphs = use_graphs
        self.dtype = dtype
        self.model = model if model is not None else GPT(model_config, device=self.device, dtype=dtype)
        if checkpoint_path:
            state = torch.load(checkpoint_path, map_location=self.device, weights_only=True)
            self.model.load_state_dict(state)
        self.model.eval()

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: int | None = None, top_p: float | None = None, eos_token_id: int | None = None,
                 return_stats: bool = False, return_logprobs: bool = False, prompt_lens=None):
        """engine.py:144-261. ``prompt_lens`` (optional, [B]) marks ragged
        prompts inside a right-padded ``input_ids``; the returned tokens are
        right-padded with 0 after each row's own end (prompt_lens[b] + decode
        steps) and ``stats["lengths"]`` gives each length."""
        if input_ids.dim() != 2:
            raise ValueError(f"input_ids must be [B, T], got shape={tuple(input_ids.shape)}")
        prompt = input_ids.to(self.device)
        batch_size, prompt_len = prompt.shape
        lens = [prompt_len] * batch_size if prompt_lens is None else [int(x) for x in prompt_lens]
        if len(lens) != batch_size or min(lens) < 1 or max(lens) > prompt_len:
            raise ValueError("prompt_lens must give 1 <= len <= T for every sequence")
        total_len = max(lens) + max_new_tokens
        if total_len > self.model_config.block_size:
            raise ValueError(
                f"Requested total sequence length {total_len} exceeds block_size {self.model_config.block_size}")
        tokens = torch.zeros(batch_size, total_len, dtype=prompt.dtype, device=self.device)
        tokens[:, :prompt_len] = prompt
        paged = self.use_paged_kv_cache
        if paged:
            cache = PagedKVCache.from_model_config(
                self.model_config, batch_size=batch_size, page_size=self.kv_cache_page_size, device=self.device,
                dtype=self.dtype, kv_cache_dtype=self.kv_cache_dtype,
                seq_capacity=[n + max_new_tokens for n in lens], paged_pool=self.paged_pool,
                page_seed=self.page_seed)
            cache.set_pending_new_lens(lens)
        else:
            # engine.py:168-178: the per-layer (k, v) tuples grown by concatenation; one batch-wide length
            if min(lens) != prompt_len:
                raise ValueError("ragged prompts (prompt_lens) need the paged KV cache (use_paged_kv_cache=True)")
            cache = None
        lens_t = torch.tensor(lens, device=self.device)

        prefill_tokens = int(sum(lens))
        prefill_t0 = time.perf_counter()
        logits, cache = self.model(prompt, use_cache=True, past_key_values=cache, position_offset=0,
                                   logits_index=lens_t - 1)
        if paged:
            cache.set_pending_new_lens(None)
        next_logits = logits[:, -1, :]
        torch.cuda.synchronize(self.device)
        prefill_t1 = time.perf_counter()

        decode_steps = 0
        token_log_probs = []
        # step j's tokens go to column j of one buffer (a plain copy per step) and to their
        # places lens[b] + j in `tokens` by one scatter after the loop
        generated = torch.empty(batch_size, max(max_new_tokens, 1), dtype=tokens.dtype, device=self.device)
        uniform = len(set(lens)) == 1
        graphs = None
        # the tuple cache's tensors change every step: it launches eagerly. The
        # paged caches replay graphs when asked (use_graphs=True), launch
        # eagerly when told not to (False), and by default (None) decide after
        # the third decode step: replay when the host took at least GRAPH_HOST_RATIO of
        # the GPU's time to issue eager steps 1 and 2 (the GPU waits on the
        # host), else stay eager (replay would only add the two captures and
        # the replays' own cost to the loop).
        use_graphs = paged and bool(self.use_graphs)
        auto = paged and self.use_graphs is None
        self.last_decode_launch = "graphs" if use_graphs else "eager"
        self.last_decode_issue = None  # (host, GPU) seconds of eager steps 1 and 2 when the default decided
        if paged:
            cache.set_static_max_len(max(lens) + max_new_tokens)
        decode_t0 = time.perf_counter()
        for step in range(max_new_tokens):
            if return_logprobs:
                next_token, next_log_prob = sample_next_token_with_log_prob(next_logits, temperature, top_k, top_p)
                token_log_probs.append(next_log_prob)
            else:
                next_token = sample_next_token(next_logits, temperature, top_k, top_p)
            generated[:, step] = next_token
            decode_steps += 1
            if eos_token_id is not None and torch.all(next_token == eos_token_id):
                break
            position = (lens[0] + step) if uniform else 0
            if graphs is None and use_graphs and step >= 1 and max_new_tokens - step >= 3:
                graphs = DecodeGraphs(self.model, cache, batch_size, position, uniform, self.device)
            if graphs is not None:
                logits = graphs.step(next_token)
            elif auto and step in (1, 2):
                # steps 1 and 2 eager, timed from one synchronisation: the host's
                # issue time against the GPU time of the same work
                if step == 1:
                    torch.cuda.synchronize(self.device)
                    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                    ev[0].record()
                    h0 = time.perf_counter()
                logits, cache = self.model(next_token.unsqueeze(-1), use_cache=True, past_key_values=cache,
                                           position_offset=position)
                if step == 2:
                    host_s = time.perf_counter() - h0
                    ev[1].record()
                    ev[1].synchronize()
                    gpu_s = ev[0].elapsed_time(ev[1]) * 1e-3
                    self.last_decode_issue = (host_s, gpu_s)
                    use_graphs = host_s >= GRAPH_HOST_RATIO * gpu_s
                    self.last_decode_launch = "graphs" if use_graphs else "eager"
            else:
                logits, cache = self.model(next_token.unsqueeze(-1), use_cache=True, past_key_values=cache,
                                           position_offset=position)
            next_logits = logits[:, -1, :]
        if decode_steps:
            cols = lens_t.unsqueeze(1) + torch.arange(decode_steps, device=self.device)
            tokens.scatter_(1, cols, generated[:, :decode_steps])
        torch.cuda.synchronize(self.device)
        decode_t1 = time.perf_counter()
        if paged:
            cache.set_static_max_len(None)

        out_len = max(lens) + decode_steps
        tokens = tokens[:, :out_len]
        if not uniform:  # row b ends at lens[b] + decode_steps; what follows is pad 0, not stale prompt padding
            ends = (lens_t + decode_steps).unsqueeze(1)
            tokens.masked_fill_(torch.arange(out_len, device=self.device).unsqueeze(0) >= ends, 0)
        if not return_stats and not return_logprobs:
            return tokens
        extras = {}
        prefill_time = max(prefill_t1 - prefill_t0, 1e-9)
        decode_time = max(decode_t1 - decode_t0, 1e-9)
        decode_tokens = int(batch_size * decode_steps)
        if return_stats:
            extras.update({
                "prefill_tokens_per_sec": prefill_tokens / prefill_time,
                "decode_tokens_per_sec": decode_tokens / decode_time if decode_steps > 0 else 0.0,
                "prefill_tokens": float(prefill_tokens),
                "decode_tokens": float(decode_tokens),
                "lengths": [n + decode_steps for n in lens],
            })
        if return_logprobs:
            log_probs = (torch.stack(token_log_probs, dim=1) if token_log_probs
                         else torch.empty(batch_size, 0, dtype=torch.float32, device=self.device))
            extras.update({
                "prompt_len": float(prompt_len),
                "decode_steps": float(decode_steps),
                "token_log_probs": log_probs,
                "response_mask": torch.ones_like(log_probs, dtype=torch.float32),
            })
        return tokens, extras
