#!/usr/bin/env python
"""Decode-step benchmark on one MI355X.

A step is one pass of the hot path over one batch: RoPE + KV append of one new
token per sequence and GQA split-K decode attention over each sequence's
L_b + 1 cached tokens. bf16 caches run it as one fused launch pair
(tt_decode_attn_append_*); fp8 caches (and --step-path two) as
tt_rope_append_* followed by tt_gqa_decode_attn_*.
Inputs are synthetic (seed 1337) and resident in HBM before the timed region.

Headline workload (config C3, the metric's batch-64 case): ragged paged bf16
decode attention, B = 64, 32 q heads / 8 KV heads, D = 128, L_b ~ U[128,
16384], page size 16, page table = seeded random permutation of the physical
pages. The same line carries nested records for C2 (uniform contiguous, B
32, ctx 4096), C4 (fp8-e4m3 cache, B 128, ctx U[1024, 32768]), c5a (one layer
of the C5 model mid-decode, D 64), C1 (the reference's CPU-sized model,
greedy decode) and e2e (C5 through the engine). --config selects the
headline config; --e2e-only runs C5 end to end alone.

value = algorithmic bytes per step / time per step (GB/s, 1 GB = 1e9 B), with
algorithmic bytes = unique K/V bytes read (+ fp8 scales) + q/out/new-token/page
table I/O. The roofline object covers the decode-attention operator in the
partition the KV cache picks for the workload's lengths (C3 and c5a: the paired
kernel, one launch; C2: the per-segment kernel; C4: the balanced stream kernel
and its merge kernel) timed alone with HIP events on the stream it runs on. CPU baselines time the reference's own op sequence (torch
on the host: rope_impl, gqa_impl, the H_q-expanded LayerPagedKVCache, mask,
SDPA; for C1 / C5 the whole model and generate loop) on bounded samples of
the same workloads, with the host's CPU model and thread count recorded.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
METRIC = "decode-attn HBM GB/s (% of peak) + greedy decode tokens/sec at batch 64"

CONFIGS = {
    "c2": dict(name="C2 uniform contiguous bf16 decode attention", batch=32, hq=32, hkv=8, head_dim=128,
               lo=4096, hi=4096, page=16, paged=False, fp8=False),
    "c3": dict(name="C3 ragged paged bf16 GQA decode step", batch=64, hq=32, hkv=8, head_dim=128,
               lo=128, hi=16384, page=16, paged=True, fp8=False),
    "c4": dict(name="C4 ragged paged fp8-e4m3 GQA decode step", batch=128, hq=32, hkv=8, head_dim=128,
               lo=1024, hi=32768, page=16, paged=True, fp8=True),
    # one layer's attention of the C5 model mid-decode (prompts U[64, 2048] + 128 generated tokens)
    "c5a": dict(name="C5 per-layer ragged paged bf16 GQA decode step (D 64)", batch=64, hq=32, hkv=8, head_dim=64,
                lo=192, hi=2176, page=16, paged=True, fp8=False),
}
# CPU-baseline sample per config: all sequences, or a seeded subset where the
# reference layout (4x the unique K/V) of every sequence would not fit the budget
CPU_SAMPLE = {"c2": None, "c3": None, "c4": 16, "c5a": None}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--step-path", choices=["auto", "fused", "two"], default="auto",
                   help="decode step as one launch pair (RoPE + append inside the attention kernel) or as the "
                        "RoPE + append kernel then attention; auto: fused")
    p.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    p.add_argument("--nested", default="c2,c4,c5a",
                   help="comma-separated configs measured after the headline one and reported in nested records "
                        "('' for none)")
    p.add_argument("--seed", type=int, default=1337)
    p.add_argument("--split-tokens", type=int, default=None,
                   help="decode attention partition: 0 balanced, -1 one workgroup per (sequence, KV head), "
                        "-2 one workgroup per (rank pair, KV head), 128-1024 fixed splits; default: what the KV "
                        "cache picks for the workload's lengths")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of timed CPU-baseline work per config")
    p.add_argument("--no-c1", action="store_true", help="skip config C1 (the reference's CPU-sized model)")
    p.add_argument("--no-e2e", action="store_true", help="skip the end-to-end greedy decode (config 5)")
    p.add_argument("--e2e-steps", type=int, default=256)
    p.add_argument("--e2e-only", action="store_true", help="run only the end-to-end decode and print its record")
    p.add_argument("--no-eager-compare", action="store_true",
                   help="skip the second end-to-end run that replays the step from HIP graphs and checks its tokens")
    return p.parse_args()


C1 = dict(num_layer=6, hidden_size=512, num_attention_heads=8, num_key_value_heads=2, vocab_size=32000,
          intermediate_size=2048, init_std=0.02, prompt=128, steps=64, page=128)
C5 = dict(num_layer=24, hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, vocab_size=32000,
          intermediate_size=6144, init_std=0.02, batch=64, lo=64, hi=2048, page=16)


def log(msg: str) -> None:
    """Progress line on stderr (the JSON result alone goes to stdout)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def host_threads(torch) -> int:
    """Threads for the CPU baselines: the CPUs this process may run on, capped by
    OMP_NUM_THREADS when set (the GPU box gives a 16-CPU share)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    torch.set_num_threads(n)
    return n


def host_info(torch) -> dict:
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "visible_cpus": len(os.sched_getaffinity(0)), "logical_cpus": os.cpu_count(),
            "threads_used": host_threads(torch)}


def e2e_c5(args, torch):
    """Greedy decode through the engine (config C5: 24 layers, d 2048, batch 64), tokens/s as
    engine.py:236-243 defines it, plus the reference op sequence on the host
    for a bounded sample of the same batch."""
    from tinytron_amd import ops
    from tinytron_amd.engine import InferenceEngine
    from tinytron_amd.model import GPT, ModelConfig

    steps = args.e2e_steps
    g = torch.Generator().manual_seed(args.seed)
    B = C5["batch"]
    lens = torch.randint(C5["lo"], C5["hi"] + 1, (B,), generator=g).tolist()
    prompt = torch.randint(0, C5["vocab_size"], (B, max(lens)), generator=g)
    cfg = ModelConfig(num_layer=C5["num_layer"], hidden_size=C5["hidden_size"],
                      num_attention_heads=C5["num_attention_heads"], num_key_value_heads=C5["num_key_value_heads"],
                      vocab_size=C5["vocab_size"], intermediate_size=C5["intermediate_size"], init_std=C5["init_std"],
                      block_size=max(lens) + steps, seed=args.seed)
    model = GPT(cfg, device="cuda", dtype=torch.bfloat16)
    eng = InferenceEngine(cfg, device="cuda", dtype=torch.bfloat16, kv_cache_page_size=C5["page"], paged_pool=True,
                          model=model)
    eng.generate(prompt[:, :16], 4, top_k=1)  # warm kernels and the allocator
    torch.cuda.synchronize()
    tokens, stats = eng.generate(prompt, steps, top_k=1, prompt_lens=lens, return_stats=True)
    tps = stats["decode_tokens_per_sec"]
    launch = eng.last_decode_launch
    issue = eng.last_decode_issue  # host issue and GPU time of eager steps 1 and 2 (the launch-mode decision)
    forced = {}
    if not args.no_eager_compare:  # both launch modes forced, same tokens checked
        for mode in (False, True):
            eng.use_graphs = mode
            t_m, s_m = eng.generate(prompt, steps, top_k=1, prompt_lens=lens, return_stats=True)
            if not torch.equal(tokens, t_m):
                raise RuntimeError("graph-replayed and eager decodes diverged")
            forced["graphs" if mode else "eager"] = round(s_m["decode_tokens_per_sec"], 1)
        eng.use_graphs = None
    # the reference's kind of batch: every prompt of the ragged batch's mean length (the caches then
    # pick the per-segment attention partition, one launch per layer's attention)
    uni_len = int(round(sum(lens) / B))
    _, uni_stats = eng.generate(prompt[:, :uni_len], steps, top_k=1, return_stats=True)
    # the same decode with an fp8-e4m3 KV cache (per-(token, head) scales, written by the
    # fused step's append; the same launches per layer as bf16)
    fp8_eng = InferenceEngine(cfg, device="cuda", dtype=torch.bfloat16, kv_cache_page_size=C5["page"], paged_pool=True,
                              kv_cache_dtype=torch.float8_e4m3fn, model=model)
    fp8_tokens, fp8_stats = fp8_eng.generate(prompt, steps, top_k=1, prompt_lens=lens, return_stats=True)
    gen = torch.stack([tokens[b, lens[b]:lens[b] + steps] for b in range(B)])
    gen8 = torch.stack([fp8_tokens[b, lens[b]:lens[b] + steps] for b in range(B)])
    del fp8_eng
    n_params = sum(p.numel() for p in model.parameters())
    mean_ctx = sum(lens) / B + steps / 2
    kv_bytes = C5["num_layer"] * 2 * B * mean_ctx * C5["num_key_value_heads"] * (C5["hidden_size"] // C5["num_attention_heads"]) * 2
    step_bytes = (n_params - C5["vocab_size"] * C5["hidden_size"]) * 2 + C5["vocab_size"] * C5["hidden_size"] * 2 + kv_bytes
    bound = B / (step_bytes / (PEAK_HBM_GBS * 1e9))
    out = {
        "workload": "C5 greedy decode through the engine: 24 L, d 2048, 32/8 heads, D 64, V 32000, bf16 "
                    "random-init weights, B 64, prompts U[64, 2048], paged KV page 16",
        "decode_tokens_per_sec": round(tps, 1),
        "decode_launch": launch,
        "decode_issue_ms_per_step": None if issue is None else {
            "host": round(issue[0] * 500.0, 3), "gpu": round(issue[1] * 500.0, 3),
            "note": "eager steps 1 and 2 timed from one synchronisation: host clock around their issue, HIP events "
                    "around their GPU work (per step; the engine replays graphs only when host >= 0.97 x gpu)"},
        "decode_tokens_per_sec_eager": forced.get("eager"),
        "decode_tokens_per_sec_graphs": forced.get("graphs"),
        "decode_path": "fused bf16 decode step (7 launches per layer: RoPE + append inside the attention launch, "
                       "one launch in the paired partition the caches pick for this batch, gate|up and SwiGLU in one "
                       "launch) + one-launch sampler, launched as the engine's "
                       "default picks after the third step (decode_launch: eager when the host issues steps in less "
                       "than 0.97x their GPU time, else HIP-graph replay with the two captures inside the timed "
                       "window); decode_tokens_per_sec_eager / _graphs force each mode (same tokens, checked)",
        "attention_partition": {ops.SPLIT_PER_SEGMENT: "per segment", ops.SPLIT_PAIRED: "paired (rank pairs)",
                                0: "balanced"}[ops.pick_split(lens, C5["num_key_value_heads"],
                                                              C5["hidden_size"] // C5["num_attention_heads"],
                                                              "bf16")],
        "decode_steps": int(stats["decode_tokens"] // B),
        "decode_tokens_per_sec_uniform_prompts": round(uni_stats["decode_tokens_per_sec"], 1),
        "uniform_prompts": f"all {B} prompts of {uni_len} tokens (the ragged batch's mean; the reference's engine "
                           "takes one prompt length): the attention takes the per-segment partition, one launch",
        "decode_tokens_per_sec_fp8_kv": round(fp8_stats["decode_tokens_per_sec"], 1),
        "fp8_kv_first_token_agreement": round(float((gen8[:, 0] == gen[:, 0]).float().mean()), 4),
        "prefill_tokens_per_sec_fp8_kv": round(fp8_stats["prefill_tokens_per_sec"], 1),
        "prefill_tokens_per_sec": round(stats["prefill_tokens_per_sec"], 1),
        "params": n_params,
        "hbm_bound_tokens_per_sec": round(bound, 1),
        "frac_of_hbm_bound": round(tps / bound, 4),
        "cpu_baseline": None,
        "sampler": sampler_timing(torch),
    }
    cpu_job = None
    if not args.no_cpu_baseline:
        sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
        ctx = int(round(sum(lens) / B + steps / 2))

        def cpu_job():
            out["sampler"]["cpu_baseline"] = sampler_cpu_baseline(torch)
            return e2e_cpu_baseline(sd, cfg, ctx, torch)
    del eng, model
    torch.cuda.empty_cache()
    return out, cpu_job


def sampler_timing(torch, iters=50):
    """Microseconds per call of the one-launch sampler on C5's logits
    ([64, 32000] bf16), HIP events on the stream it runs on."""
    from tinytron_amd import ops

    logits = _sampler_logits(torch).cuda()
    st = {name: timed_steps(torch, fn, iters, 5) for name, fn in (
        ("greedy_us", lambda: ops.sample_tokens(logits, top_k=1)),
        ("top_k50_top_p0.9_T0.8_us", lambda: ops.sample_tokens(logits, 0.8, 50, 0.9, 1, 0)),
        ("top_p0.9_logprob_us", lambda: ops.sample_tokens(logits, 1.0, None, 0.9, 1, 0, return_logprob=True)))}
    out = {"logits": "[64, 32000] bf16", "statistic": "median of per-call HIP event gaps"}
    out.update({name: round(s["median_ms"] * 1e3, 2) for name, s in st.items()})
    return out


def _sampler_logits(torch):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(C5["batch"], C5["vocab_size"], generator=g) * 3).to(torch.bfloat16)


def sampler_cpu_baseline(torch, iters=20):
    """The reference's sampling op sequence (filter_logits + softmax +
    multinomial, sampler.py:6-48, restated in oracle.ref_path) on the host, per
    call on the same logits as sampler_timing."""
    from oracle.ref_path import filter_logits

    threads = host_threads(torch)
    logits = _sampler_logits(torch)

    def per_call_us(t, k, p):
        torch.multinomial(torch.softmax(filter_logits(logits, t, k, p), dim=-1), 1)
        t0 = time.perf_counter()
        for _ in range(iters):
            torch.multinomial(torch.softmax(filter_logits(logits, t, k, p), dim=-1), 1)
        return round((time.perf_counter() - t0) / iters * 1e6, 1)

    return {"greedy_us": per_call_us(1.0, 1, None), "top_k50_top_p0.9_T0.8_us": per_call_us(0.8, 50, 0.9),
            "unit": "us per call", "cores": threads, "kind": "port",
            "sample": f"{iters} calls per setting on the same [64, 32000] bf16 logits, torch on the host"}


def e2e_cpu_baseline(sd, cfg, ctx, torch, budget_s=10.0, max_steps=32):
    """The reference's op sequence (oracle.ref_model, fp32 on the host, as the
    reference runs without a GPU) on C5's decode shape: batch 64, every layer's
    reference-layout cache (H_q-expanded LayerPagedKVCache) filled, untimed, to
    ctx tokens -- the mean context of C5's decode (mean prompt length + half the
    steps) -- then n_steps greedy decode steps timed (after one untimed step).
    Decode time does not depend on the cached values, and the reference's one
    batch-wide length cannot express ragged prompts, so a uniform batch at the
    mean length stands in for the ragged one. Steps run until budget_s of
    them is spent (at most max_steps)."""
    from oracle.ref_model import RefGPT

    threads = host_threads(torch)
    B = C5["batch"]
    ref = RefGPT(sd, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads)
    caches = ref.new_caches(B, ctx + max_steps + 2, page_size=C5["page"])
    g = torch.Generator().manual_seed(0)
    tile = torch.randn(1, ref.hq, 64, ref.D, generator=g)  # a random 64-token pattern, repeated
    pattern = tile.repeat(1, 1, (ctx + 63) // 64, 1)[:, :, :ctx].expand(B, -1, -1, -1)
    for c in caches:
        c._k_flat[:, :, :ctx].copy_(pattern)
        c._v_flat[:, :, :ctx].copy_(pattern)
        c.current_length = ctx
    tok = torch.randint(0, cfg.vocab_size, (B, 1), generator=g)
    with torch.no_grad():
        logits = ref.forward(tok, caches, ctx)  # untimed first step
        t0 = time.perf_counter()
        n_steps = 0
        while n_steps < max_steps and (n_steps == 0 or time.perf_counter() - t0 < budget_s):
            tok = torch.argmax(logits[:, -1].float(), dim=-1)[:, None]
            logits = ref.forward(tok, caches, ctx + 1 + n_steps)
            n_steps += 1
        wall = time.perf_counter() - t0
    del ref, caches
    return {"value": round(B * n_steps / wall, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"batch {B} (the C5 batch) at a uniform context of {ctx} tokens (C5's mean decode context: "
                      f"mean prompt + half of the decode steps), every layer's H_q-expanded LayerPagedKVCache "
                      f"filled untimed; {n_steps} greedy decode steps timed after one untimed step, fp32 on the "
                      f"host through the reference op sequence (the reference has no ragged batches)",
            "seconds": round(wall, 2)}


def c1_record(args, torch):
    """Config C1 (the reference's CPU-runnable case: 6 L, d 512, 8/2 heads, V
    32000, fp32, prompt 128, 64 greedy steps, contiguous cache): the engine on
    the GPU (fp32, the CPU path's arithmetic) and the reference's op sequence on
    the host with the paged cache and with the tuple-concat cache."""
    from tinytron_amd.engine import InferenceEngine
    from tinytron_amd.model import GPT, ModelConfig

    cfg = ModelConfig(num_layer=C1["num_layer"], hidden_size=C1["hidden_size"],
                      num_attention_heads=C1["num_attention_heads"], num_key_value_heads=C1["num_key_value_heads"],
                      vocab_size=C1["vocab_size"], intermediate_size=C1["intermediate_size"], init_std=C1["init_std"],
                      block_size=C1["prompt"] + C1["steps"], seed=args.seed)
    model = GPT(cfg, device="cpu", dtype=torch.float32)  # seeded init on the CPU, then moved
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to("cuda")
    prompt = torch.randint(0, C1["vocab_size"], (1, C1["prompt"]), generator=torch.Generator().manual_seed(args.seed))
    eng = InferenceEngine(cfg, device="cuda", dtype=torch.float32, kv_cache_page_size=C1["page"], model=model)
    eng.generate(prompt, 4, top_k=1)
    torch.cuda.synchronize()
    tokens, stats = eng.generate(prompt, C1["steps"], top_k=1, return_stats=True)
    # use_paged_kv_cache=False: the reference's per-layer (k, v) tuples grown by concatenation
    eng_t = InferenceEngine(cfg, device="cuda", dtype=torch.float32, use_paged_kv_cache=False, model=model)
    eng_t.generate(prompt, 4, top_k=1)
    torch.cuda.synchronize()
    tokens_t, stats_t = eng_t.generate(prompt, C1["steps"], top_k=1, return_stats=True)
    out = {"workload": "C1: 6 L, d 512, 8/2 heads, D 64, V 32000, fp32 weights ~N(0, 0.02) seed 1337, batch 1, "
                       "prompt 128, 64 greedy steps, contiguous KV cache",
           "decode_tokens_per_sec": round(stats["decode_tokens_per_sec"], 1),
           "decode_tokens_per_sec_tuple_cache": round(stats_t["decode_tokens_per_sec"], 1),
           "tuple_cache_tokens_equal": bool(torch.equal(tokens.cpu(), tokens_t.cpu())),
           "decode_path": "module path in fp32 (d 512 takes no fused kernels): RoPE + append + attention in one "
                          "launch pair per layer, graph-replayed steps; decode_tokens_per_sec_tuple_cache: "
                          "use_paged_kv_cache=False (the tuple-concat cache held in a growing store, eager steps)"}
    del eng, eng_t, model
    tokens = tokens.cpu()

    def cpu_job():
        """The whole C1 workload on the host (runs after every GPU leg): fills
        out['cpu_baseline'] and out['greedy_tokens_equal_cpu']."""
        from oracle.ref_model import RefGPT

        threads = host_threads(torch)
        ref = RefGPT(sd, cfg.num_layer, cfg.num_attention_heads, cfg.num_key_value_heads)
        res = {}
        for name, tuple_cache in (("paged", False), ("tuple_concat", True)):
            ref_tokens, tps, _ = ref.generate_greedy(prompt, 4, cfg.block_size, page_size=C1["page"],
                                                     tuple_cache=tuple_cache)  # warm-up
            ref_tokens, tps, _ = ref.generate_greedy(prompt, C1["steps"], cfg.block_size, page_size=C1["page"],
                                                     tuple_cache=tuple_cache)
            res[name] = (tps, ref_tokens)
        out["greedy_tokens_equal_cpu"] = bool(torch.equal(tokens, res["paged"][1]))
        out["cpu_baseline"] = {
            "value": round(res["paged"][0], 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "value_tuple_concat_cache": round(res["tuple_concat"][0], 2),
            "sample": "the whole C1 workload: fp32 on the host through the reference op sequence with "
                      "LayerPagedKVCache (value) and with use_paged_kv_cache=False's concatenated K/V "
                      "(value_tuple_concat_cache)"}

    return out, (None if args.no_cpu_baseline else cpu_job)


def build_workload(cfg, seed, torch, ops):
    dev = torch.device("cuda")
    B, hq, hkv, D, P = cfg["batch"], cfg["hq"], cfg["hkv"], cfg["head_dim"], cfg["page"]
    g = torch.Generator().manual_seed(seed)
    if cfg["lo"] == cfg["hi"]:
        ctx = torch.full((B,), cfg["lo"], dtype=torch.int64)
    else:
        ctx = torch.randint(cfg["lo"], cfg["hi"] + 1, (B,), generator=g)
    total = ctx + 1  # tokens attended after the append
    gd = torch.Generator(device=dev).manual_seed(seed)
    if cfg["paged"]:
        need = (total + P - 1) // P
        n_phys = int(need.sum())
        perm = torch.randperm(n_phys, generator=g).to(torch.int32)
        max_pages = int(need.max())
        table = torch.full((B, max_pages), -1, dtype=torch.int32)
        off = 0
        for b in range(B):
            n = int(need[b])
            table[b, :n] = perm[off:off + n]
            off += n
        page_table = table.to(dev)
        numel = n_phys * hkv * P * D
        strides = (0, hkv * P * D, P * D)
        capacity = max_pages * P
        num_pages = n_phys
    else:
        cap = int(math.ceil(int(total.max()) / P) * P)
        pages = cap // P
        page_table = None
        numel = B * hkv * pages * P * D
        strides = (hkv * pages * P * D, P * D, pages * P * D)
        capacity = cap
        num_pages = 0
    kind = "fp8" if cfg["fp8"] else "bf16"
    if cfg["fp8"]:
        k_store = torch.empty(numel, dtype=torch.uint8, device=dev)
        v_store = torch.empty(numel, dtype=torch.uint8, device=dev)
        chunk = 1 << 24  # rows of D per chunk
        rows = numel // D
        k_scale, v_scale = ops.fp8_scales(rows, dev)  # one array, K and V scales of each 16 rows in one line
        for dst, sc in ((k_store, k_scale), (v_store, v_scale)):
            for r0 in range(0, rows, chunk):
                r1 = min(rows, r0 + chunk)
                x = torch.randn(r1 - r0, D, generator=gd, device=dev, dtype=torch.bfloat16).float()
                s = x.abs().amax(dim=-1) / 448.0
                codes = torch.where(s[:, None] > 0, x / torch.where(s > 0, s, 1.0)[:, None], 0.0)
                dst[r0 * D:r1 * D] = codes.to(ops.FP8_DTYPE).view(torch.uint8).reshape(-1)
                sc[ops.fp8_scale_index(torch.arange(r0, r1, device=dev))] = s
                del x, codes
    else:
        k_store = torch.randn(numel, generator=gd, device=dev, dtype=torch.bfloat16)
        v_store = torch.randn(numel, generator=gd, device=dev, dtype=torch.bfloat16)
        k_scale = v_scale = None
    layout = ops.KVLayout(k=k_store, v=v_store, strides=strides, num_heads=hkv, head_dim=D, page_size=P,
                          capacity=capacity, kind=kind, page_table=page_table, num_pages=num_pages,
                          k_scale=k_scale, v_scale=v_scale)
    q_in = torch.randn(B, 1, hq, D, generator=gd, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    k_in = torch.randn(B, 1, hkv, D, generator=gd, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    v_in = torch.randn(B, 1, hkv, D, generator=gd, device=dev, dtype=torch.bfloat16).transpose(1, 2)
    table_rows = int(total.max()) + 1
    rope = ops.build_rope_table(table_rows, D, dtype=torch.bfloat16, device=dev)
    return dict(ctx=ctx, total=total, layout=layout, q_in=q_in, k_in=k_in, v_in=v_in, rope=rope,
                positions=ctx.to(torch.int32).to(dev), seq_lens=total.to(torch.int32).to(dev),
                max_len=int(total.max()))


def algorithmic_bytes(cfg, total):
    """Bytes the step must move at minimum: K/V of every attended token (+ fp8
    scales), page-table entries, q in / out, lengths, the new token's K/V."""
    B, hq, hkv, D, P = cfg["batch"], cfg["hq"], cfg["hkv"], cfg["head_dim"], cfg["page"]
    e = 1 if cfg["fp8"] else 2
    tokens = int(total.sum())
    kv = tokens * hkv * D * e * 2
    scales = tokens * hkv * 4 * 2 if cfg["fp8"] else 0
    pages = int(((total + P - 1) // P).sum()) * 4 if cfg["paged"] else 0
    q_out = B * hq * D * 2 * 2
    new_kv = B * hkv * D * (2 + e) * 2
    attn_bytes = kv + scales + pages + q_out + B * 4
    step_bytes = attn_bytes + B * hq * D * 2 * 2 + new_kv  # + rope q in/out
    return step_bytes, attn_bytes, tokens


def _gather_sequence(cfg, wl, torch, b):
    """Sequence b's cached K/V as bf16 [1, H_kv, L, D] on the host (fp8: dequantised)."""
    layout = wl["layout"]
    hkv, D, P = cfg["hkv"], cfg["head_dim"], cfg["page"]
    L = int(wl["ctx"][b])
    pos = torch.arange(L, device="cuda")
    if layout.page_table is not None:
        phys = layout.page_table[b].long()[pos // P]
        base = phys * layout.strides[1] + (pos % P) * D
    else:
        base = b * layout.strides[0] + (pos // P) * layout.strides[1] + (pos % P) * D
    heads = torch.arange(hkv, device="cuda") * layout.strides[2]
    idx = base[:, None, None] + heads[None, :, None] + torch.arange(D, device="cuda")[None, None, :]
    if cfg["fp8"]:
        from tinytron_amd import ops

        sidx = ops.fp8_scale_index((base[:, None] + heads[None, :]) // D)
        k = (layout.k[idx].view(torch.float8_e4m3fn).float() * layout.k_scale[sidx][..., None]).to(torch.bfloat16)
        v = (layout.v[idx].view(torch.float8_e4m3fn).float() * layout.v_scale[sidx][..., None]).to(torch.bfloat16)
    else:
        k, v = layout.k[idx], layout.v[idx]
    return k.permute(1, 0, 2).unsqueeze(0).cpu(), v.permute(1, 0, 2).unsqueeze(0).cpu()


def cpu_baseline(cfg, wl, torch, budget_s, sample=None, seed=1337, max_steps=64):
    """Reference op sequence on the host (oracle.ref_path.decode_attention_step:
    rope_impl, gqa_impl, H_q-expanded LayerPagedKVCache append / get_kv, mask,
    SDPA) in torch bf16, consecutive decode steps (each appends a token, as the
    reference's loop does) until the time budget is spent. Uniform lengths run
    as one batch (the reference's own batch-wide length); ragged batches run one
    sequence at a time (batch-1 caches), over all sequences or a seeded sample."""
    from oracle import ref_path

    threads = host_threads(torch)
    hq, hkv, D, P = cfg["hq"], cfg["hkv"], cfg["head_dim"], cfg["page"]
    rep = hq // hkv
    e = 1 if cfg["fp8"] else 2
    B = cfg["batch"]
    uniform = cfg["lo"] == cfg["hi"]
    total_time, total_bytes, tokens, steps_run = 0.0, 0, 0, 0
    if uniform:
        L = int(wl["ctx"][0])
        cache = ref_path.LayerPagedKVCache(B, hq, D, L + 2 + max_steps, P, torch.device("cpu"), torch.bfloat16)
        for b in range(B):  # append sequence by sequence into the batched store (untimed setup)
            k, v = _gather_sequence(cfg, wl, torch, b)
            cache._k_flat[b:b + 1, :, :L].copy_(k.repeat_interleave(rep, dim=1))
            cache._v_flat[b:b + 1, :, :L].copy_(v.repeat_interleave(rep, dim=1))
        cache.current_length = L
        q, kn, vn = wl["q_in"].cpu(), wl["k_in"].cpu(), wl["v_in"].cpu()
        ref_path.decode_attention_step(q, kn, vn, cache, hkv, position=L)  # warm-up (appends one token)
        while steps_run < max_steps and (steps_run == 0 or total_time < budget_s):
            Lt = L + 1 + steps_run
            t0 = time.perf_counter()
            y = ref_path.decode_attention_step(q, kn, vn, cache, hkv, position=Lt)
            total_time += time.perf_counter() - t0
            assert y.shape == (B, hq, 1, D)
            total_bytes += B * (Lt + 1) * hkv * D * e * 2
            tokens += B * (Lt + 1)
            steps_run += 1
        del cache
        what = (f"the whole batch of {B} as one reference batch (uniform length), {steps_run} consecutive decode "
                f"steps")
    else:
        seqs = list(range(B))
        if sample is not None and sample < B:
            g = torch.Generator().manual_seed(seed)
            seqs = sorted(torch.randperm(B, generator=g)[:sample].tolist())
        for b in seqs:
            L = int(wl["ctx"][b])
            k, v = _gather_sequence(cfg, wl, torch, b)
            cache = ref_path.LayerPagedKVCache(1, hq, D, L + 2 + max_steps, P, torch.device("cpu"), torch.bfloat16)
            cache.append(k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1))
            del k, v
            q, kn, vn = wl["q_in"][b:b + 1].cpu(), wl["k_in"][b:b + 1].cpu(), wl["v_in"][b:b + 1].cpu()
            ref_path.decode_attention_step(q, kn, vn, cache, hkv, position=L)  # warm-up (appends one token)
            share, spent, step = budget_s / len(seqs), 0.0, 0
            while step < max_steps and (step == 0 or spent < share):
                Lt = L + 1 + step
                t0 = time.perf_counter()
                y = ref_path.decode_attention_step(q, kn, vn, cache, hkv, position=Lt)
                spent += time.perf_counter() - t0
                assert y.shape == (1, hq, 1, D)
                total_bytes += (Lt + 1) * hkv * D * e * 2 + ((Lt + 1) * hkv * 8 if cfg["fp8"] else 0)
                tokens += Lt + 1
                step += 1
                steps_run += 1
            total_time += spent
            del cache
        what = (f"{len(seqs)} of the {B} sequences" + (" (seeded sample)" if len(seqs) < B else "")
                + f", one at a time, {steps_run} decode steps in all")
    return {
        "value": round(total_bytes / total_time / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{what} ({tokens} cached tokens attended) through the reference op sequence (rope_impl, gqa_impl, "
                   f"H_q-expanded LayerPagedKVCache append/get_kv, mask, SDPA) in torch bf16 on the host; bytes "
                   f"counted as for the GPU (unique K/V)"
                   + ("; fp8 cache dequantised to bf16, the reference has no fp8" if cfg["fp8"] else "")),
        "seconds": round(total_time, 3),
    }


def measured_traffic(config: str):
    """HBM bytes per decode-attention launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this workload (copy-calibrated), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"decode_attn_{config}.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(float(line.split(":")[1]))
    except OSError:
        return None
    return None


def timed_steps(torch, fn, steps, warmup, min_warm_s=0.1):
    """GPU time of `steps` calls of fn on torch's current stream (the stream
    the library's kernels are launched on), after `warmup` untimed calls and
    more until at least min_warm_s of them have run (clocks and caches
    settled). Two timed passes of `steps` calls each:
      - window: one event before the first call and one after the last, so
        that nothing but the steps themselves is enqueued between them; the
        window mean is the per-step figure reported (mean_ms);
      - per step: one event after every call, so that step i's time is the gap
        between events i and i + 1 (median, min, max). Each event is a marker
        packet between two steps, which costs the stream a few microseconds
        per step: these figures bound the window mean from above and show the
        spread (a stall inside the window shows as a max far above the median).
    """
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    steps = max(int(steps), 1)
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record()
    for _ in range(steps):
        fn()
    w1.record()
    torch.cuda.synchronize()
    mean = w0.elapsed_time(w1) / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    mid = steps // 2
    median = per[mid] if steps % 2 else 0.5 * (per[mid - 1] + per[mid])
    return {"mean_ms": mean, "median_ms": median, "min_ms": per[0], "max_ms": per[-1], "warmup_calls": n}


def spread(st):
    """Timing record (µs) of a timed_steps result."""
    return {"window_mean_us": round(st["mean_ms"] * 1e3, 2), "per_step_median_us": round(st["median_ms"] * 1e3, 2),
            "per_step_min_us": round(st["min_ms"] * 1e3, 2), "per_step_max_us": round(st["max_ms"] * 1e3, 2),
            "warmup_calls": st["warmup_calls"]}


def run_config(name, args, torch, ops):
    """Time one attention config on the GPU: the decode step (RoPE + append
    inside the attention launch(es), bf16 and fp8 caches), the two-launch step,
    and the attention operator alone, each over args.steps steps (a window of
    back-to-back steps between two HIP events on the stream the kernels run on,
    then a pass with per-step events for the spread) after a warm-up of at
    least args.warmup steps and 100 ms. Returns the record and the
    workload (kept for the CPU baseline, which runs after every GPU leg)."""
    cfg = CONFIGS[name]
    wl = build_workload(cfg, args.seed, torch, ops)
    B, hq, D = cfg["batch"], cfg["hq"], cfg["head_dim"]
    layout = wl["layout"]
    q_rot = torch.empty(B, hq, 1, D, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(B, hq, D, dtype=torch.bfloat16, device="cuda")
    ws = ops.Workspace("cuda")
    # the partition the KV cache picks for these lengths (LayerPagedKVCache._attention_split): one
    # workgroup per (sequence, KV head) when all lengths are equal and B * H_kv fills the GPU, one per
    # (rank pair, KV head) for a ragged batch whose pairs fill the CUs evenly, else the balanced one
    split = args.split_tokens if args.split_tokens is not None else \
        ops.pick_split(wl["total"].tolist(), cfg["hkv"], D, "fp8" if cfg["fp8"] else "bf16")
    per_segment = split == ops.SPLIT_PER_SEGMENT
    paired = split == ops.SPLIT_PAIRED
    # as the KV cache does: the length order uploaded once (every step shifts all lengths alike)
    order = torch.tensor(ops.length_order(wl["total"].tolist()), dtype=torch.int32, device="cuda") if paired else None
    lens_out = torch.empty_like(wl["positions"])
    fused = args.step_path != "two"

    def two_launch_step():
        ops.rope_append(wl["q_in"], wl["k_in"], wl["v_in"], wl["rope"], wl["positions"], layout, q_out=q_rot)
        ops.decode_attention(q_rot.view(B, hq, D), layout, wl["seq_lens"], wl["max_len"], out=out,
                             split_tokens=split, workspace=ws, length_order=order)

    def step():
        # the fused decode step: RoPE + append of the new token inside the attention launch(es)
        if split > 0 or not fused:
            two_launch_step()
            return
        ops.decode_attention_append(wl["rope"], wl["positions"], layout, wl["max_len"], q=wl["q_in"][:, :, 0],
                                    k=wl["k_in"][:, :, 0], v=wl["v_in"][:, :, 0], lens_out=lens_out, out=out,
                                    workspace=ws, split_tokens=split, length_order=order)

    def attn_only():
        ops.decode_attention(q_rot.view(B, hq, D), layout, wl["seq_lens"], wl["max_len"], out=out,
                             split_tokens=split, workspace=ws, length_order=order)

    # each timed region gets its own warm-up: a kernel's first launch loads its code
    # object (~0.6 ms), which untimed warm-up keeps out of the per-step figures
    st_step = timed_steps(torch, step, args.steps, args.warmup)
    st_two = timed_steps(torch, two_launch_step, args.steps, args.warmup)  # RoPE + append, then attention
    st_attn = timed_steps(torch, attn_only, args.steps, args.warmup)  # the dominant operator alone (q rotated above)
    ms, two_ms, attn_ms = st_step["mean_ms"], st_two["mean_ms"], st_attn["mean_ms"]
    step_bytes, attn_bytes, tokens = algorithmic_bytes(cfg, wl["total"])
    value = step_bytes / (ms * 1e-3) / 1e9
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    rec = {
        "value": round(value, 2),
        "unit": "GB/s",
        "ms_per_step": round(ms, 5),
        "ms_per_step_two_launches": round(two_ms, 5),
        "per_step": {"step": spread(st_step), "two_launch_step": spread(st_two), "attention": spread(st_attn),
                     "statistic": "ms_per_step, value and roofline.avg_us: mean over one event-bracketed window of "
                                  "back-to-back steps; per_step_*: a second pass with an event after every step"},
        "pct_of_peak_hbm": round(100.0 * value / PEAK_HBM_GBS, 2),
        "dtype": "fp8-e4m3 cache, bf16 q/out" if cfg["fp8"] else "bf16",
        "config": {
            "workload": cfg["name"],
            "batch": B, "q_heads": hq, "kv_heads": cfg["hkv"], "head_dim": D,
            "context": [cfg["lo"], cfg["hi"]], "page_size": cfg["page"], "paged": cfg["paged"],
            "cached_tokens": tokens,
            "split_tokens": ("per segment (-1: one workgroup per (sequence, KV head), merged in LDS; all lengths "
                             "equal)" if per_segment
                             else "paired (-2: the sequences ordered by length on the host, one workgroup per KV "
                             "head and rank pair (p, B - 1 - p), merged in LDS)" if paired
                             else split or "balanced (equal 32-token tiles per wave)"),
            "parallelism": "single GPU",
            "step_path": ("one launch: RoPE + append inside the per-segment attention kernel "
                          "(decode_segment_append_kernel)" if fused and per_segment
                          else "one launch: RoPE + append inside the paired attention kernel "
                          "(decode_paired_append_kernel)" if fused and paired
                          else "one launch pair: RoPE + append inside the attention split kernel "
                          "(decode_stream_append_kernel + decode_merge_kernel)" if fused and not split
                          else "rope_append_kernel, then the attention kernels"),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("decode attention (decode_segment_kernel)" if per_segment
                       else "decode attention (decode_paired_kernel)" if paired
                       else "decode attention (decode_stream_kernel + decode_merge_kernel)" if not split
                       else "decode attention (decode_split_kernel + decode_combine_kernel)"),
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(name),
            "traffic_source": f"profiles/decode_attn_{name}.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                              "scaled by a 256 MiB copy)",
            "avg_us": round(attn_ms * 1e3, 2),
            "algorithmic_bytes": attn_bytes,
        },
        "cpu_baseline": None,
    }
    del layout, q_rot, out, ws
    return rec, wl


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported in this build "
              "(the multi-GPU decode layout is a design note, not a measured path)", file=sys.stderr)
        return 2
    import torch

    from tinytron_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no CPU fallback)", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.e2e_only:
        rec, job = e2e_c5(args, torch)
        if job is not None:
            rec["cpu_baseline"] = job()
        print(json.dumps({"e2e": rec}), flush=True)
        return 0

    # a plain copy of known size, for scaling rocprof FETCH/WRITE counters
    calib = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
    calib_dst = torch.empty_like(calib)
    calib_dst.copy_(calib)
    del calib, calib_dst

    # every GPU leg first, then the host-only CPU baselines, so that no timed GPU
    # region follows seconds of host-only work
    names = [args.config] + [n for n in args.nested.split(",") if n and n != args.config]
    recs, workloads = {}, {}
    for name in names:
        recs[name], workloads[name] = run_config(name, args, torch, ops)
        log(f"{name}: step {recs[name]['ms_per_step'] * 1e3:.1f} us, attention {recs[name]['roofline']['avg_us']} us "
            f"({recs[name]['roofline']['frac']:.4f} of peak)")
    head = recs[args.config]
    result = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "ms_per_step_two_launches": head["ms_per_step_two_launches"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic",
        "pct_of_peak_hbm": head["pct_of_peak_hbm"],
        "config": head["config"],
        "roofline": head["roofline"],
        "per_step": head["per_step"],
        "cpu_baseline": None,
        "host": host_info(torch),
    }
    for name in names[1:]:
        result[name] = recs[name]
    cpu_jobs = []
    if not args.no_c1:
        result["c1"], job = c1_record(args, torch)
        cpu_jobs.append(job)
        log(f"c1: {result['c1']['decode_tokens_per_sec']} tokens/s")
    if not args.no_e2e:
        result["e2e"], job = e2e_c5(args, torch)
        log(f"e2e: {result['e2e']['decode_tokens_per_sec']} tokens/s")
        if job is not None:
            cpu_jobs.append(lambda j=job: result["e2e"].__setitem__("cpu_baseline", j()))
    if not args.no_cpu_baseline:
        for name in names:
            target = result if name == args.config else result[name]
            target["cpu_baseline"] = cpu_baseline(CONFIGS[name], workloads[name], torch, args.cpu_seconds,
                                                  sample=CPU_SAMPLE.get(name), seed=args.seed)
            log(f"{name} cpu baseline: {target['cpu_baseline']['value']} GB/s")
            del workloads[name]
            torch.cuda.empty_cache()
        for job in cpu_jobs:
            if job is not None:
                job()
                log("cpu baseline done")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
