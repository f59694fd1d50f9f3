#!/usr/bin/env python3
"""Benchmark of the MI355X verify hot path on one GPU.

Headline (one JSON line on stdout): paged verify attention of one Qwen3-8B-shaped layer (32 q / 8 kv heads,
head_dim 128, bf16, 256-token pages) at batch 64 with verify lengths uniform in {1..8} (tokens padded to a multiple
of 8 with a padding row on the zero pad block) and contexts uniform in [2800, 3200]; max_seqlen_k = 4096 as the
verify graphs pass it. value = algorithmic HBM bytes (every visible K/V row once + q + out) / time per layer.

Also measured: the fused speculative sampler (64 rows x 8 verified positions, V = 151,936, fp32 logits ~ N(0, 9),
top-k 64), against the one read of the [512, V] logits it must make; and the torch-CPU restatement of the same
attention (the oracle, the reference's CPU path) on the host cores as a reported baseline.

Also: a whole verify round of 36 Qwen3-8B-shaped layers (random bf16 weights) captured as a HIP graph, with the
logits and the fused accept, against its HBM floor (weights + K/V + logits).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-baseline on|off] [--sampler on|off]
                       [--verify-round on|off] [--copy-probe on|off]
"""
import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
METRIC = "verify-attn µs/layer & HBM GB/s (% of 8 TB/s) at B=64, 8 q, 3k ctx"

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (one counter per run) at the commit
# beside each entry, each scaled by what the counter reads for the 1 GiB copy probe (FETCH_SIZE x 1.99995,
# WRITE_SIZE x 1.0); the runs and their numbers are in profiles/hbm_traffic_pmc_verify_attention_and_spec_accept.md.
# Re-measure after a kernel change.
MEASURED_TRAFFIC = {
    "verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200": 789_697_462,              # head-major caches, 628323f
    "verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200_token_major": 789_712_493,  # 628323f
    "verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200_kv_interleaved": 789_712_021,  # 628323f
    "spec_accept_b64_k7_v151936_fp32_topk64": 320_037_489,                              # 628323f
    "markov_draw_b64_v151936_bf16_rank64": 40_235_723,                                  # f8d0a8b
}
MEASURED_AT = "628323f"   # the headline (attention) entry


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_gpu(fn, steps: int, warmup: int):
    """Average ms per call of fn over `steps` calls after `warmup`, bracketed by HIP events on the current
    stream (the stream the kernels are launched on) and device synchronisations on both sides."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def host_info() -> dict:
    """What the CPU baselines ran on: the processor model, the cores this process may use, torch's version and
    thread count."""
    import torch
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(),
            "usable_cores": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "torch": torch.__version__, "torch_threads": torch.get_num_threads()}


def time_cpu(fn, budget_s: float = 15.0, max_runs: int = 10):
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < max_runs and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def attention_bench(args, dev):
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import attention as nattn

    log("[bench] building the batch-64 verify-attention workload")
    case = wl.config_c3()
    max_k = 4096
    kv, qo = case.kv_bytes(), case.qo_bytes()
    flops = case.flops()
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    # The reference's token-major layout (model_runner.py:160), the library's head-major layout (each (block, kv
    # head) one contiguous run in K and one in V), then K and V interleaved (each (block, kv head)'s keys and then
    # values one run): the same values through the same kernel.
    # Every layout is on the device before any is timed, and one untimed pass of the first leg brings the GPU to
    # its working clock: a leg that starts after the host has kept the GPU idle (building and copying a layout)
    # runs its first milliseconds slow, which its warm-up launches alone do not cover. Each leg then runs its
    # warm-up launches and its timed launches as usual, back to back with the others.
    layouts_dev = {"token_major": case.to(dev), "head_major": case.head_major().to(dev),
                   "kv_interleaved": case.kv_interleaved(dev)}

    def stepper(g, out):
        def step():
            nattn._paged_attention(g.q, g.k_cache, g.v_cache, g.block_tables, g.cu_seqlens_q, g.cu_seqlens_k, None,
                                   0, len(case.q_lens), g.max_seqlen_q, max_k, g.scale, True, out=out, workspace=ws)
        return step

    outs = {layout: torch.empty_like(g.q) for layout, g in layouts_dev.items()}
    settle = stepper(layouts_dev["token_major"], outs["token_major"])
    for _ in range(args.warmup + args.steps):
        settle()
    torch.cuda.synchronize()
    timed = {}
    for layout in ("token_major", "head_major", "kv_interleaved"):
        ms = time_gpu(stepper(layouts_dev[layout], outs[layout]), args.steps, args.warmup)
        gbs = (kv + qo) / (ms * 1e-3) / 1e9
        log(f"[bench] attention ({layout} cache): {ms * 1e3:.1f} us/layer, {gbs:.0f} GB/s = "
            f"{100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s")
        timed[layout] = (ms, gbs)
    hip_out = outs["kv_interleaved"].float().cpu()   # the last timed output (every layout gives the same bits)
    del layouts_dev, outs
    ms, gbs = timed["head_major"]
    layouts = {}
    for layout, desc in (("token_major", "token_major [blocks, 256, 8, 128] (the reference's)"),
                         ("kv_interleaved", "kv_interleaved: K and V views of [blocks, 8, 2, 256, 128] memory")):
        l_ms, l_gbs = timed[layout]
        layouts[layout] = {"workload": "verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200", "kv_layout": desc,
                           "us": round(l_ms * 1e3, 2), "GBs": round(l_gbs, 1), "frac": round(l_gbs / HBM_PEAK_GBS, 4),
                           "traffic": MEASURED_TRAFFIC[f"verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200_{layout}"]}
    return case, ms, kv + qo, gbs, flops, layouts, hip_out


def launch_bound_bench(args, dev):
    """The batch-8 shape (contexts 900-1200): too small to fill the chip; reported, not a target. Its kernel
    (about 16 us) is as short as one eager call's host work, so the launches are captured as a HIP graph of 20, as a
    serving loop captures its verify steps, and the graph is replayed."""
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import attention as nattn
    case = wl.config_c2()
    g = case.head_major().to(dev)
    out = torch.empty_like(g.q)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=dev)

    def step():
        nattn._paged_attention(g.q, g.k_cache, g.v_cache, g.block_tables, g.cu_seqlens_q, g.cu_seqlens_k, None, 0,
                               len(case.q_lens), g.max_seqlen_q, 4096, g.scale, True, out=out, workspace=ws)

    step()   # eagerly first: the split merge's counters are created outside the capture
    torch.cuda.synchronize()
    inner = 20
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            step()
    ms = time_gpu(graph.replay, max(10, args.steps // inner), max(2, args.warmup // inner)) / inner
    b = case.kv_bytes() + case.qo_bytes()
    return {"workload": "verify_attention_qwen3_8b_b8_ctx900_1200", "kv_layout": "head_major",
            "us": round(ms * 1e3, 2), "timing": f"HIP graph of {inner} launches, per launch",
            "GBs": round(b / (ms * 1e-3) / 1e9, 1), "bytes": b}


def sampler_bench(args, dev):
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import spec_sampler as ns

    def draft_probs(lg, t, k, p):
        # top-64 softmax of the draft logits (every row has top_k 64, temperature 1)
        s = lg / t[:, None, None]
        kth = s.topk(64, dim=-1).values[..., -1:]
        return torch.softmax(s.masked_fill(s < kth, float("-inf")), dim=-1)

    log("[bench] building the 64 x 8 x 151936 sampler workload")
    case = wl.sampler_case(64, 7, 151936, draft_probs_fn=draft_probs)
    g = case.to(dev)
    st = ns.SamplingTensors(g.temperatures, g.top_k, g.top_p, case.max_top_k, case.has_top_p, True)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)  # counters start at zero

    def step():
        ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, None, g.uniforms, g.noise, workspace=ws)

    # one untimed pass first: building the workload on the host left the GPU idle (see the attention legs)
    for _ in range(args.warmup + args.steps):
        step()
    torch.cuda.synchronize()
    ms = time_gpu(step, max(10, args.steps // 2), max(3, args.warmup // 2))
    T, V = case.logits.shape
    alg = T * V * 4
    gbs = alg / (ms * 1e-3) / 1e9
    n, tail = step_out = ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st, None, g.uniforms, g.noise,
                                                   workspace=ws)
    torch.cuda.synchronize()
    del step_out
    log(f"[bench] fused sampler: {ms * 1e3:.1f} us, {gbs:.0f} GB/s = {100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s")

    # the production dtype of the target logits (bf16: half the bytes) and the greedy accept over the same rows
    lg16 = g.logits.to(torch.bfloat16)

    def step16():
        ns.spec_accept_with_draws(lg16, g.q, g.drafts, st, None, g.uniforms, g.noise, workspace=ws)

    ms16 = time_gpu(step16, max(10, args.steps // 2), max(3, args.warmup // 2))
    lg3 = g.logits.view(64, 8, V)

    def greedy():
        ns.accept_greedy(lg3, g.drafts)

    msg = time_gpu(greedy, max(10, args.steps // 2), max(3, args.warmup // 2))
    # top-p 0.9 and temperature 0.7 on every row (the nucleus path and the IEEE division by the temperature)
    st_p = ns.SamplingTensors(torch.full_like(g.temperatures, 0.7), g.top_k, torch.full_like(g.top_p, 0.9),
                              case.max_top_k, True, True)

    def step_p():
        ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st_p, None, g.uniforms, g.noise, workspace=ws)

    msp = time_gpu(step_p, max(10, args.steps // 2), max(3, args.warmup // 2))
    # the reference's default sampling (SamplingParams: temperature 1, top_k 0, top_p 1): no truncation, so p is
    # the softmax over the whole vocabulary and each row's race runs over all of it (p, q and noise rows)
    st_d = ns.SamplingTensors(g.temperatures, torch.zeros_like(g.top_k), g.top_p, 0, False, False)

    def step_d():
        ns.spec_accept_with_draws(g.logits, g.q, g.drafts, st_d, None, g.uniforms, g.noise, workspace=ws)

    msd = time_gpu(step_d, max(10, args.steps // 2), max(3, args.warmup // 2))
    alg_d = alg + 3 * 64 * V * 4
    # the same accept with q as DSpark candidate rows (top-64 + 64 = 128 entries per draft row) instead of dense
    from nvs_amd.layers.markov import CandidateRows
    top = g.q.topk(128, dim=-1)
    rows = CandidateRows(top.indices.to(torch.int32).contiguous(), top.values.contiguous())

    def step_c():
        ns.spec_accept_with_draws(g.logits, rows, g.drafts, st, None, g.uniforms, g.noise, workspace=ws)

    msc = time_gpu(step_c, max(10, args.steps // 2), max(3, args.warmup // 2))
    same = [torch.equal(x, y) for x, y in zip(ns.spec_accept_with_draws(g.logits, rows, g.drafts, st, None, g.uniforms,
                                                                        g.noise, workspace=ws), (n, tail))]
    log(f"[bench] fused sampler on bf16 logits: {ms16 * 1e3:.1f} us; top-p 0.9 + temperature 0.7: "
        f"{msp * 1e3:.1f} us; greedy accept (fp32): {msg * 1e3:.1f} us; q as candidate rows: {msc * 1e3:.1f} us "
        f"(same decisions: {all(same)}); no top-k (the reference's default): {msd * 1e3:.1f} us, "
        f"{100 * alg_d / (msd * 1e-3) / 1e9 / HBM_PEAK_GBS:.1f}% of 8 TB/s")
    variants = {
        "topp0.9_temp0.7": {"us": round(msp * 1e3, 2), "GBs": round(alg / (msp * 1e-3) / 1e9, 1)},
        "bf16_logits": {"us": round(ms16 * 1e3, 2), "GBs": round(alg / 2 / (ms16 * 1e-3) / 1e9, 1),
                        "algorithmic_bytes": alg // 2},
        "candidate_rows_q": {"us": round(msc * 1e3, 2), "GBs": round(alg / (msc * 1e-3) / 1e9, 1),
                             "candidates": 128, "same_decisions_as_dense_q": all(same)},
        "no_topk_default_sampling": {"us": round(msd * 1e3, 2), "GBs": round(alg_d / (msd * 1e-3) / 1e9, 1),
                                     "algorithmic_bytes": alg_d,
                                     "bytes_are": "every logit once, plus each row's race over its p, q and noise "
                                                  "rows"},
        "greedy_fp32": {"us": round(msg * 1e3, 2), "GBs": round(alg / (msg * 1e-3) / 1e9, 1),
                        "algorithmic_bytes": alg, "kernel": "argmax_kernel + greedy_finalize_kernel"},
    }
    out = {"workload": "spec_accept_b64_k7_v151936_fp32_topk64", "us": round(ms * 1e3, 2), "variants": variants,
           "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": alg,
           "traffic": MEASURED_TRAFFIC["spec_accept_b64_k7_v151936_fp32_topk64"],
           "kernel": "select_kernel<f32, accept> (one launch per call)",
           "mean_accepted": round(float(n.float().mean()), 3)}
    if args.cpu_baseline == "on":
        out["cpu_baseline"] = sampler_cpu_baseline(case, n.cpu(), tail.cpu())
    return out


def sampler_cpu_baseline(case, n_gpu, tail_gpu):
    """The torch-CPU restatement of the reference's sampler path (oracle: probs_from_logits then
    accept_random, the two calls of SpeculativeDecoder._accept) over the whole 64 x 8 x 151,936 case on the host
    cores, with the GPU run's uniforms and noise; its decisions are compared with the fused kernel's."""
    import torch

    from oracle import spec_sampler as ref
    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))

    def run():
        return ref.accept_from_logits(case.logits, case.q, case.drafts, case.temperatures, case.top_k, case.top_p,
                                      case.max_top_k, case.has_top_p, None, case.uniforms, case.noise)

    n_cpu, tail_cpu = run()
    same = bool(torch.equal(n_cpu, n_gpu) and torch.equal(tail_cpu, tail_gpu))
    sec, runs = time_cpu(run)
    T, V = case.logits.shape
    gbs = T * V * 4 / sec / 1e9
    log(f"[bench] sampler cpu baseline: {sec * 1e3:.1f} ms per call on {torch.get_num_threads()} threads "
        f"(same decisions as the GPU: {same})")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "host": host_info(),
            "sample": f"the whole 64 x 8 x 151,936 fp32 case (probs_from_logits + accept_random, same draws), "
                      f"median of {runs} runs: {sec * 1e3:.1f} ms per call", "ms_per_call": round(sec * 1e3, 2),
            "same_decisions_as_gpu": same}


def draft_block_bench(args, dev):
    """The draft model's block attention (the decode branch run by DFlashDrafter, speculative.py:268-275): 64 rows
    of 7 block queries each, non-causal over their whole context (2,807-3,207 keys, the same 3k contexts as the
    verify layer plus the block), Qwen3-8B-shaped heads, fixed-length mode."""
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import attention as nattn
    lq = 7
    _, k_lens = wl.random_lengths(64, (1, 8), (2800 + lq, 3200 + lq), seed=1)
    case = wl.verify_attention_case([lq] * 64, k_lens, 32, 8, 128, pad_tokens_to=1)
    g = case.head_major().to(dev)
    ctx = torch.tensor(k_lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(g.q)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)

    def step():
        nattn._paged_attention(g.q, g.k_cache, g.v_cache, g.block_tables, None, None, ctx, lq, 64, lq, 4096,
                               g.scale, False, out=out, workspace=ws)

    ms = time_gpu(step, args.steps, args.warmup)
    b = case.kv_bytes() + case.qo_bytes()
    gbs = b / (ms * 1e-3) / 1e9
    log(f"[bench] draft-block attention (Lq 7, non-causal): {ms * 1e3:.1f} us, {gbs:.0f} GB/s = "
        f"{100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s")
    return {"workload": "draft_block_attention_qwen3_8b_b64_lq7_noncausal_ctx2807_3207", "kv_layout": "head_major",
            "us": round(ms * 1e3, 2),
            "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": b}


def graph_timed(fn, args, reps: int = 10) -> float:
    """ms per call of fn as it runs inside a verify graph: reps calls captured in one HIP graph (after one eager
    call on a side stream), the graph replayed and timed by time_gpu."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    return time_gpu(graph.replay, max(10, args.steps // 4), 3) / reps


def rows_bench(args, dev):
    """The hot path's other entry points on their own, each timed per call inside a HIP graph (graph_timed):
    the KV store of a batch-64 verify layer (296 tokens, 8 kv heads, value a strided view of the fused qkv, head-
    major cache), and over 64 rows x 8 positions x 151,936 fp32 logits ~N(0, 3^2) with top-k 64: probs_from_logits,
    truncate_logits, the race of sample() over [64, V], and accept_random on dense p and q (the unfused path)."""
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import attention as nattn
    from nvs_amd.layers import spec_sampler as ns
    gen = torch.Generator(device=dev).manual_seed(11)
    rows = {}

    def report(name, ms, nbytes, what):
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows[name] = {"us": round(ms * 1e3, 2), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "bytes": nbytes, "bytes_are": what}
        log(f"[bench] {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s = {100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s")

    # a1: store_kvcache, 296 tokens into a head-major cache of 786 blocks
    n_tok, hkv, d, blocks = 296, 8, 128, 786
    qkv = torch.randn(n_tok, (32 + 2 * hkv) * d, generator=gen, device=dev).to(torch.bfloat16)
    key = qkv[:, 32 * d:(32 + hkv) * d].view(n_tok, hkv, d)
    value = qkv[:, (32 + hkv) * d:].view(n_tok, hkv, d)
    kc = wl.head_major_empty(blocks, 256, hkv, d, dtype=torch.bfloat16, device=dev).zero_()
    vc = wl.head_major_empty(blocks, 256, hkv, d, dtype=torch.bfloat16, device=dev).zero_()
    slots = torch.randperm(blocks * 256, generator=gen, device=dev)[:n_tok].to(torch.int32)
    ms = graph_timed(lambda: nattn.store_kvcache(key, value, kc, vc, slots), args)
    report("a1_store_kvcache", ms, 2 * 2 * n_tok * hkv * d * 2, "K and V rows read and written")
    del kc, vc

    # a5: probs_from_logits and truncate_logits over [64, 8, V] fp32
    B, k, V = 64, 7, 151936
    logits = (torch.randn(B, k + 1, V, generator=gen, device=dev) * 3).contiguous()
    st = ns.SamplingTensors(torch.ones(B, device=dev), torch.full((B,), 64, dtype=torch.int64, device=dev),
                            torch.ones(B, device=dev), 64, False, True)
    ms = graph_timed(lambda: ns.probs_from_logits(logits, st), args)
    report("a5_probs_from_logits", ms, 2 * logits.numel() * 4, "logits read, probabilities written (fp32)")
    ms = graph_timed(lambda: ns.truncate_logits(logits, st), args)
    report("a5_truncate_logits", ms, 2 * logits.numel() * 4, "scaled logits read, truncated logits written")

    # a6: the race of sample() over [64, V]
    p = ns.probs_from_logits(logits, st)
    noise = torch.empty(B, V, device=dev).exponential_(1.0, generator=gen).clamp_min_(1e-10)
    weights = p[:, 0].contiguous()
    ms = graph_timed(lambda: ns.race(weights, noise), args)
    report("a6_race", ms, 2 * B * V * 4, "weights and noise read")

    # a7: accept_random on dense p [512, V] and q [64, 7, V]
    q = torch.softmax(torch.randn(B, k, V, generator=gen, device=dev) * 3, dim=-1)
    drafts = torch.randint(0, V, (B, k), generator=gen, device=dev)
    uniforms = torch.rand(B, k, generator=gen, device=dev)
    ms = graph_timed(lambda: ns.accept_random_with_draws(p, q, drafts, None, uniforms, noise), args)
    report("a7_accept_random_dense", ms, 3 * B * V * 4, "each row's race reads its p row, q row and noise row")
    del logits, p, q
    torch.cuda.empty_cache()
    return rows


def qk_rope_bench(args, dev):
    """The fused q/k RMSNorm + rotary + KV store of one batch-64 verify layer (296 tokens, 32/8 heads), against
    the same sequence as separate torch ops on the GPU (norm q, norm k, rotate both, index the caches)."""
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd.layers import qk_norm_rope as nrope
    case = wl.qk_rope_case(296).to(dev)
    q, k, v = case.split()
    q_out = torch.empty_like(q)

    def fused():
        nrope.qk_norm_rope_store(case.positions, q, k, v, case.q_norm_weight, case.k_norm_weight, case.eps,
                                 case.table, case.k_cache, case.v_cache, case.slot_mapping, q_out=q_out)

    def rms(x, w):
        xf = x.to(torch.float32, copy=True)
        xf.mul_(torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + case.eps))
        return xf.to(x.dtype).mul_(w)

    def rot(x, cos, sin):
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    live = torch.nonzero(case.slot_mapping >= 0).flatten()
    slots = case.slot_mapping[live].long()
    kc = case.k_cache.view(-1, case.num_kv_heads, case.head_dim)
    vc = case.v_cache.view(-1, case.num_kv_heads, case.head_dim)

    def torch_ops():
        cos, sin = case.table[case.positions].unsqueeze(1).chunk(2, dim=-1)
        qr = rot(rms(q, case.q_norm_weight), cos, sin)
        kr = rot(rms(k, case.k_norm_weight), cos, sin)
        kc.index_copy_(0, slots, kr.index_select(0, live))
        vc.index_copy_(0, slots, v.index_select(0, live))
        return qr

    # both run as they would inside the verify graphs: 20 calls captured in one HIP graph, timed per call
    reps = 20

    def graphed(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        return graph

    g_fused, g_torch = graphed(fused), graphed(torch_ops)
    ms = time_gpu(g_fused.replay, max(10, args.steps // 4), 3) / reps
    ms_torch = time_gpu(g_torch.replay, max(10, args.steps // 4), 3) / reps
    b = case.bytes_moved()
    log(f"[bench] q/k norm + rope + store: {ms * 1e3:.2f} us fused, {ms_torch * 1e3:.2f} us as torch ops "
        f"(graph replay)")
    return {"workload": "qk_norm_rope_store_qwen3_8b_296_tokens", "us": round(ms * 1e3, 2),
            "us_torch_ops": round(ms_torch * 1e3, 2), "bytes": b, "GBs": round(b / (ms * 1e-3) / 1e9, 1),
            "timing": "HIP graph of 20 calls, per call", "kernel": "qk_norm_rope_store_kernel (one launch)"}


def markov_bench(args, dev):
    """DSpark's propose sampling (the draft side of a round): 7 Markov rows at batch 64 over V = 151,936 bf16
    draft logits, top-k 20 (84 candidates), temperature 1. Each row adds the Markov bias of the token drawn
    before it: a rank-64 head, embedding gather + GEMM by torch in both versions. Ours: one nvs_markov_draw per
    row, the bias added inside it, writing candidate rows. Against the same rows as the reference's torch ops
    (speculative.py:163-184): the add, topk, the truncated softmax, the race, and the scatter into a zeroed
    [64, 7, V] fp32 q. Both are captured as HIP graphs and replayed, as the reference replays its sampling graphs,
    with the noise drawn outside them."""
    import torch
    import torch.nn.functional as F

    from nvs_amd.layers import markov as nm
    from nvs_amd.layers import spec_sampler as ns

    B, k, V, r, top_k = 64, 7, 151936, 64, 20
    g = torch.Generator(device=dev).manual_seed(21)
    logits = torch.randn(B, k, V, device=dev, generator=g).mul_(3.0).to(torch.bfloat16)
    w1 = torch.randn(V, r, device=dev, generator=g, dtype=torch.bfloat16).mul_(0.1)
    w2 = torch.randn(V, r, device=dev, generator=g, dtype=torch.bfloat16).mul_(0.1)
    anchors = torch.randint(0, V, (B,), device=dev, generator=g)
    st = ns.SamplingTensors(torch.ones(B, device=dev), torch.full((B,), top_k, dtype=torch.int64, device=dev),
                            torch.ones(B, device=dev), top_k, False, True)
    C = nm.num_candidates(top_k, True, V)
    noise = torch.empty(B, k, C, device=dev).exponential_(1.0, generator=g).clamp_min_(1e-10)

    def bias(prev):
        return F.linear(F.embedding(prev, w1), w2)

    drafts = torch.empty(B, k, dtype=torch.int64, device=dev)

    def ours():
        nm.markov_rows(logits, anchors, st, bias, noise, drafts, C)

    q_dense = torch.empty(B, k, V, device=dev)
    drafts_t = torch.empty(B, k, dtype=torch.int64, device=dev)

    def torch_rows():
        q_dense.zero_()
        prev = anchors
        for row in range(k):
            values, ids = (logits[:, row] + bias(prev)).topk(C, dim=-1)
            s = values.float()
            kth = s[:, top_k - 1:top_k]
            probs = torch.softmax(s.masked_fill(s < kth, float("-inf")), dim=-1)
            prev = ids.gather(-1, (probs / noise[:, row]).argmax(-1, keepdim=True)).squeeze(-1)
            q_dense[:, row].scatter_(-1, ids, probs)
            drafts_t[:, row] = prev

    # one row of our draw alone (bias given, added inside), and the torch bias alone
    b0 = bias(anchors)
    ids0 = torch.empty(B, C, dtype=torch.int32, device=dev)
    probs0 = torch.empty(B, C, device=dev)
    draws0 = torch.empty(B, dtype=torch.int64, device=dev)

    def draw_only():
        nm.markov_draw(logits[:, 0], st, C, noise[:, 0], ids0, probs0, draws0, bias=b0)

    def draws_in_a_round():   # the 7 draws of a round back to back (one per Markov row), as a propose graph has them
        for row in range(k):
            nm.markov_draw(logits[:, row], st, C, noise[:, row], ids0, probs0, draws0, bias=b0)

    def bias_only():
        bias(anchors)

    def graphed(fn):
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph.replay

    steps, warm = max(10, args.steps // 4), max(3, args.warmup // 4)
    ms = time_gpu(graphed(ours), steps, warm)
    ms_t = time_gpu(graphed(torch_rows), steps, warm)
    ms_d1 = time_gpu(graphed(draw_only), steps, warm)          # a one-kernel graph: includes its replay overhead
    ms_d = time_gpu(graphed(draws_in_a_round), steps, warm) / k
    ms_b = time_gpu(graphed(bias_only), steps, warm)
    same = bool(torch.equal(drafts, drafts_t))
    replayed = drafts.clone()
    ours()                     # eager, on the same inputs: the graph's replays must have drawn the same tokens
    same = same and bool(torch.equal(drafts, replayed))
    alg = 2 * B * V * 2        # one read of a row's bf16 logits and of its bf16 bias per draw
    log(f"[bench] DSpark propose sampling (7 Markov rows, B 64, V 151936 bf16, 84 candidates, HIP graphs): "
        f"{ms * 1e3:.1f} us vs {ms_t * 1e3:.1f} us as torch ops with dense q (same drafts, graph and eager: {same}); "
        f"one draw "
        f"{ms_d * 1e3:.2f} us in a graph of the round's 7 draws ({alg / (ms_d * 1e-3) / 1e9:.0f} GB/s with its bias; "
        f"{ms_d1 * 1e3:.2f} us as a graph of its own), Markov head GEMM {ms_b * 1e3:.2f} us")
    return {"workload": "markov_rows_b64_k7_v151936_bf16_topk20_rank64", "us": round(ms * 1e3, 2),
            "torch_ops_dense_q_us": round(ms_t * 1e3, 2), "same_drafts": same, "draw_us": round(ms_d * 1e3, 2),
            "draw_us_single_graph": round(ms_d1 * 1e3, 2),
            "draw_GBs": round(alg / (ms_d * 1e-3) / 1e9, 1), "markov_head_gemm_us": round(ms_b * 1e3, 2),
            "candidates": C, "q_bytes_dense": B * k * V * 4, "q_bytes_candidates": B * k * C * 8,
            "draw_algorithmic_bytes": alg, "draw_traffic": MEASURED_TRAFFIC["markov_draw_b64_v151936_bf16_rank64"],
            "kernel": "markov_draw_kernel (one launch per Markov row; the row's last segment merges)"}


def verify_round_bench(args, dev):
    """A whole verify round (the round-level workload): 36 Qwen3-8B-shaped layers over the batch-64 verify batch
    (the attention workload's rows, one forward captured as a HIP graph on the reference's (row slots, tokens)
    shape), the bf16 logits of the verified tokens, and the fused accept (top-k 64, temperature 1) on them.
    Floor: the weights (15.14 GB) + 36 layers of K/V + the logits written once and read once, at 8 TB/s."""
    import torch

    import nvs_amd.workloads as wl
    from nvs_amd import verify_round as vr
    from nvs_amd.layers import spec_sampler as ns

    log("[bench] building the 36-layer Qwen3-8B verify round (random bf16 weights, paged KV per layer)")
    shape = vr.QWEN3_8B
    batch = vr.random_verify_batch(64)
    target = vr.Qwen3VerifyTarget(shape, batch.num_blocks, device=dev)
    graphs = vr.VerifyGraphs(target, max_batch_size=512, query_len=8, max_model_len=4096)
    rows, tokens = graphs.shape_for(batch.num_tokens)
    graphs.capture([tokens])
    B, k, V, T = len(batch.q_lens), 7, shape.vocab_size, batch.num_tokens
    lens = torch.tensor(batch.q_lens, dtype=torch.int64, device=dev)
    st = ns.SamplingTensors(torch.ones(B, device=dev), torch.full((B,), 64, dtype=torch.int64, device=dev),
                            torch.ones(B, device=dev), 64, False, True)
    # drafts that the target partly accepts (some rows all, some up to a cut, some none), so the round's accept
    # runs its acceptance, bonus and residual branches; the random drafter is a top-64 softmax of N(0, 9) logits
    log("[bench] drafting a partly accepted round (one forward per draft position)")
    rd = wl.partly_accepted_drafts(graphs, batch, st, k)
    drafts, q = rd.drafts, rd.q
    gen = torch.Generator(device=dev).manual_seed(12)
    hidden = graphs.run_drafts(batch, drafts)

    def whole():
        h = graphs.run_drafts(batch, drafts)
        return ns.accept_from_logits(target.compute_logits(h), q, drafts, st, lens, gen)

    def forward_only():
        graphs.graphs[tokens].replay()

    def tail_only():
        ns.accept_from_logits(target.compute_logits(hidden), q, drafts, st, lens, gen)

    def greedy_round():   # temperature 0: the argmax accept on the same logits (spec_sampler.py:161-169)
        h = graphs.run_drafts(batch, drafts)
        return ns.accept_greedy_varlen(target.compute_logits(h), drafts, lens)

    steps, warm = max(5, args.steps // 10), max(2, args.warmup // 5)
    ms = time_gpu(whole, steps, warm)
    ms_fwd = time_gpu(forward_only, steps, warm)
    ms_tail = time_gpu(tail_only, steps, warm)
    ms_greedy = time_gpu(greedy_round, steps, warm)
    n_accept, _ = whole()
    n_greedy, _ = greedy_round()
    weights = shape.streamed_weight_bytes()
    kv = shape.num_layers * batch.kv_bytes(shape.num_kv_heads, shape.head_dim)
    logits = 2 * T * V * 2
    floor_ms = (weights + kv + logits) / (HBM_PEAK_GBS * 1e9) * 1e3
    log(f"[bench] verify round: {ms:.3f} ms (forward graph {ms_fwd:.3f} ms, logits + accept {ms_tail:.3f} ms); "
        f"HBM floor {floor_ms:.3f} ms = {100 * floor_ms / ms:.1f}% of the floor's speed; greedy round {ms_greedy:.3f} ms")
    return {"workload": "verify_round_qwen3_8b_36_layers_b64_varlen_q1_8_ctx2800_3200_topk64",
            "ms_per_round": round(ms, 4), "forward_graph_ms": round(ms_fwd, 4),
            "logits_and_accept_ms": round(ms_tail, 4), "greedy_round_ms": round(ms_greedy, 4),
            "floor_ms": round(floor_ms, 4),
            "frac_of_floor": round(floor_ms / ms, 4),
            "floor_bytes": {"weights": weights, "kv": kv, "logits_write_and_read": logits},
            "graph_shape": {"row_slots": rows, "tokens": tokens, "verified_tokens": T},
            "mean_accepted": round(float(n_accept.float().mean()), 3),
            "mean_accepted_greedy": round(float(n_greedy.float().mean()), 3),
            "bonus_rows": int((n_accept == lens - 1).sum()), "rows": B,
            "drafts": "partly accepted: per row all verified drafts, a prefix, or none follow the target's argmax "
                      "(q = the target's own probabilities there); the rest drawn from a top-64 random drafter"}


def copy_probe(args, dev):
    """A plain 1 GiB device-to-device copy: the HBM rate a streaming kernel can reach on this box, and, under
    rocprofv3 --pmc, the known-size kernel that scales FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = time_gpu(lambda: dst.copy_(src), max(5, args.steps // 10), 2)
    gbs = 2 * n / (ms * 1e-3) / 1e9
    log(f"[bench] 1 GiB copy: {ms * 1e3:.1f} us, {gbs:.0f} GB/s read+write")
    return {"bytes_read": n, "bytes_written": n, "us": round(ms * 1e3, 2), "GBs_read_plus_write": round(gbs, 1)}


def cpu_baseline(case, hip_out):
    """The torch-CPU restatement of the reference's paged attention (oracle), in fp32 on the host cores, over the
    whole batch-64 layer (inputs converted to fp32 before timing). Also the numerics beside it: the GPU output
    against the CPU path over every row, and both against the fp64 brute force on the layer's first four rows."""
    import numpy as np
    import torch

    from oracle import attention as ref
    torch.set_num_threads(max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))))
    q = case.q.float()
    kc = case.k_cache.float()
    vc = case.v_cache.float()
    rows = case.rows
    got = {}

    def run():
        got["t32"] = ref.paged_attention_t32(q, kc, vc, case.block_tables, rows, case.scale, True)

    sec, runs = time_cpu(run)
    gbs = (case.kv_bytes() + case.qo_bytes()) / sec / 1e9
    log(f"[bench] cpu baseline: {sec * 1e3:.1f} ms/layer on {torch.get_num_threads()} threads")
    # fp64 brute force on the first four rows, their pages gathered into a compact cache
    bs = case.k_cache.shape[1]
    sub = rows[:4]
    pages = [(lk + bs - 1) // bs for _, _, lk in sub]
    blocks = sorted({int(b) for r, n in enumerate(pages) for b in case.block_tables[r, :n]})
    remap = {b: i for i, b in enumerate(blocks)}
    tables = torch.zeros(len(sub), max(pages), dtype=torch.int32)
    for r, n in enumerate(pages):
        tables[r, :n] = torch.tensor([remap[int(b)] for b in case.block_tables[r, :n]], dtype=torch.int32)
    want = ref.paged_attention_f64(case.q, case.k_cache[blocks], case.v_cache[blocks], tables, sub, case.scale,
                                   True)
    toks = np.concatenate([np.arange(q0, q0 + lq) for q0, lq, _ in sub])
    real = np.concatenate([np.arange(q0, q0 + lq) for q0, lq, _ in rows[:case.real_rows]])
    err_hip = float(np.abs(hip_out.numpy()[toks] - want[toks]).max())
    err_t32 = float(np.abs(got["t32"].numpy()[toks] - want[toks]).max())
    diff_all = float((hip_out[real] - got["t32"][real]).abs().max())
    log(f"[bench] attention numerics: max|GPU - fp64| {err_hip:.2e}, max|CPU fp32 - fp64| {err_t32:.2e} "
        f"(first 4 rows); max|GPU - CPU fp32| over every row {diff_all:.2e} (bound 2e-2)")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "host": host_info(),
            "sample": f"the whole batch-64 layer (same inputs as the GPU run, fp32), median of {runs} runs: "
                      f"{sec * 1e3:.1f} ms/layer", "ms_per_layer": round(sec * 1e3, 2),
            "numerics": {"max_abs_err_gpu_vs_fp64": err_hip, "max_abs_err_cpu_fp32_vs_fp64": err_t32,
                         "rows_vs_fp64": len(sub), "max_abs_diff_gpu_vs_cpu_fp32_all_rows": diff_all,
                         "bound": 2e-2}}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--sampler", choices=["on", "off"], default="on")
    ap.add_argument("--verify-round", choices=["on", "off"], default="on",
                    help="also time a whole 36-layer verify round (forward graph, logits, fused accept)")
    ap.add_argument("--copy-probe", choices=["on", "off"], default="off",
                    help="also time a plain 1 GiB device copy (the counter scale for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the verify hot path runs on one GPU's share and this library has no "
              "multi-GPU path; run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import nvs_amd  # noqa: F401
    from nvs_amd import _lib
    _lib.load()
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)

    case, ms, nbytes, gbs, flops, layouts, hip_out = attention_bench(args, dev)
    extra = {"attention_token_major": layouts["token_major"], "attention_kv_interleaved": layouts["kv_interleaved"],
             "c2": launch_bound_bench(args, dev),
             "draft_block": draft_block_bench(args, dev),
             "qk_norm_rope_store": qk_rope_bench(args, dev)}
    if args.sampler == "on":
        extra["sampler"] = sampler_bench(args, dev)
        extra["rows"] = rows_bench(args, dev)
        extra["markov_rows"] = markov_bench(args, dev)
    if args.verify_round == "on":
        extra["verify_round"] = verify_round_bench(args, dev)
    if args.copy_probe == "on":
        extra["copy_probe"] = copy_probe(args, dev)
    cpu = cpu_baseline(case, hip_out) if args.cpu_baseline == "on" else None

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200",
                   "rows": len(case.q_lens), "tokens": int(sum(case.q_lens)), "heads": "32q/8kv",
                   "head_dim": 128, "block_size": 256, "max_seqlen_k": 4096,
                   "kv_layout": "head_major: [blocks, 256, 8, 128] view of [blocks, 8, 256, 128] memory"},
        "us_per_layer": round(ms * 1e3, 2),
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC["verify_attention_qwen3_8b_b64_varlen_q1_8_ctx2800_3200"],
                     "traffic_measured_at": MEASURED_AT,
                     "bytes_per_launch": nbytes,
                     "kernel": "attn_split_kernel (batch 64 runs unsplit: one launch per paged_attention call)"},
        "mfma_tflops_useful": round(flops / (ms * 1e-3) / 1e12, 2),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
