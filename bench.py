#!/usr/bin/env python
"""Selective-KV decode benchmark on one MI355X.

Workload: a random-init Llama-3-8B-shaped model
(32 layers, dim 4096, 32 q / 8 kv heads, d 128, bf16), batch 32, 8192-token
context per row in 16-token pages drawn from a shuffled pool, layers 0-1 full
(layer 1 is the planner), a 2048-token budget (128 pages, L = 8) for layers
2-31, every decode step one hipGraph replay.  A "step" is one decode step of
the whole batch; ``value`` = batch / step time (tokens/s).

Also measured, in the same process:
  * the same engine with the selective cache off (full-cache decode);
  * per-kernel HBM roofline: the subset attention kernel (dominant: 30 launches
    per step), the planner kernel, the full-cache kernel and the standalone
    K-only scorer, each timed with HIP events on its launch stream; achieved
    GB/s from algorithmic bytes (K/V of the attended tokens once, q, o, the
    page indices, + the logits for the scorers);
  * the decode step of BASELINE config 4 end to end (Qwen2.5-7B shape, batch 4,
    64 k context), selective and full cache;
  * the decode step of BASELINE config 5 end to end (Qwen2.5-14B shape, 128 ragged rows of
    1 k-32 k tokens, per-row budgets; the layers share 8 KV caches since the full KV exceeds
    HBM), selective and full cache;
  * the reference's own speed recipe end to end (DeepSeek-R1-Distill-Qwen-1.5B shape,
    batch 64, full layers 0 1 2 14 22: three planner layers per step), selective and
    full cache at 2 k, 8 k and 16 k context;
  * a CPU baseline: the oracle's PyTorch-CPU restatement of the same math,
    composed per step from per-op timings on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "selective decode tokens/s (bs×ctx) + page-score/attn HBM GB/s vs peak"

# config 3
MODEL = "llama-3-8b"
BATCH = 32
CONTEXT = 8192
BUDGET_PAGES = 128
L_LAST = 8
FULL_LAYERS = [0, 1]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_engine(torch, steps_budget: int):
    from delta_amd.backend import LMBackend
    eng = LMBackend(dtype=torch.bfloat16, device="cuda:0", cuda_graph_decode=True)
    eng.load_model(f"random:{MODEL}", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = list(FULL_LAYERS)
    cfg.subset_cache_size = BUDGET_PAGES
    cfg.compression_ratio = 1.0
    cfg.L = L_LAST
    eng.setup_caches(max_batch_size=BATCH, max_seq_length=CONTEXT + steps_budget + 16)
    eng.prepare_synthetic_decode(CONTEXT, decode_budget=steps_budget, seed=0)
    return eng


def engine_config4(torch, warmup: int, steps: int) -> dict:
    """BASELINE config 4 end to end: a random-init Qwen2.5-7B-shaped model (28 layers, 28 q / 4
    kv heads, qkv bias, bf16), batch 4, 65536-token context, 4096-token budget (256 pages) behind
    the compression-ratio-16 gate, L = 8, layers 0-1 full, 4 K channels scaled x8 in every
    layer; one hipGraph per step, selective and full-cache decode in turn."""
    from delta_amd.backend import LMBackend
    from delta_amd import ops
    B, ctx, budget_pages = 4, 65536, 256
    extra = 2 * (warmup + steps) + 16
    eng = LMBackend(dtype=torch.bfloat16, device="cuda:0", cuda_graph_decode=True)
    eng.load_model("random:Qwen2.5-7b", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1]
    cfg.subset_cache_size = budget_pages
    cfg.compression_ratio = 16.0
    cfg.L = 8
    eng.setup_caches(max_batch_size=B, max_seq_length=ctx + extra + 16)
    eng.prepare_synthetic_decode(ctx, decode_budget=extra, seed=0, k_outlier_channels=4)
    ms = time_steps(torch, eng, warmup, steps)
    eng.enable_selective_cache = False
    eng._decode_graph = None
    ms_full = time_steps(torch, eng, warmup, steps)
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()
    return {"workload": "config4: Qwen2.5-7B-shaped decode step, B=4, 65536-token context, 4096-token budget "
                        "(256 pages, compression ratio 16, L=8), full layers [0,1], K outlier channels, "
                        "one hipGraph per step",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B / ms * 1e3, 2),
            "full_cache_ms_per_step": round(ms_full, 4), "full_cache_tokens_per_s": round(B / ms_full * 1e3, 2),
            "speedup_vs_full_cache": round(ms_full / ms, 3)}


def engine_config5(torch, warmup: int, steps: int, kv_pool: int = 8) -> dict:
    """BASELINE config 5 end to end: a random-init Qwen2.5-14B-shaped model (48 layers, 40 q / 8 kv
    heads, qkv bias, bf16), batch 128 with context lengths uniform in [1024, 32768] (the
    configuration's seeded lengths), per-row budgets of max(512, len/8) tokens recomputed from
    each row's length at every step (``LMBackend.set_subset_budget_rule``), L = 8, layers 0-1
    full, one hipGraph per step; selective
    and full-cache decode.  The full KV (~425 GB) exceeds one GPU's HBM, so the 48 layers share
    ``kv_pool`` physical caches round robin (``setup_caches(kv_cache_pool=...)``): every layer
    still reads and appends its own pages at the real shape."""
    import random
    from delta_amd.backend import LMBackend
    from delta_amd import ops
    B = 128
    rng = random.Random(0)
    lens = [rng.randint(1024, 32768) for _ in range(B)]          # as workloads.config_case(5)
    extra = 2 * (warmup + steps) + 16
    budgets = [max(1, max(512, (n + 1) // 8) // 16) for n in lens]  # at the first step (kv_len = n + 1)
    eng = LMBackend(dtype=torch.bfloat16, device="cuda:0", cuda_graph_decode=True)
    eng.load_model("random:Qwen2.5-14b", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1]
    cfg.subset_cache_size = max(512, (max(lens) + extra + 1) // 8) // 16  # the rule's largest budget
    cfg.compression_ratio = 1.0
    cfg.L = 8
    eng.setup_caches(max_batch_size=B, max_seq_length=max(lens) + extra + 16, kv_cache_pool=kv_pool)
    eng.prepare_synthetic_decode(lens, decode_budget=extra, seed=0)
    eng.set_subset_budget_rule(512, 8)
    ms = time_steps(torch, eng, warmup, steps)
    eng.enable_selective_cache = False
    eng._decode_graph = None
    ms_full = time_steps(torch, eng, warmup, steps)
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()
    return {"workload": f"config5: Qwen2.5-14B-shaped decode step, B=128, contexts U[1024, 32768] "
                        f"({sum(lens)} cached tokens), per-row budgets max(512, len/8) tokens on the device "
                        f"({sum(budgets)} pages at the first step), L=8, full layers [0,1], one hipGraph per step; the 48 "
                        f"layers share {kv_pool} KV caches round robin (the full KV exceeds HBM)",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B / ms * 1e3, 2),
            "full_cache_ms_per_step": round(ms_full, 4), "full_cache_tokens_per_s": round(B / ms_full * 1e3, 2),
            "speedup_vs_full_cache": round(ms_full / ms, 3)}


RECIPE_CONTEXTS = (2048, 8192, 16384)


def engine_recipe(torch, warmup: int, steps: int, contexts=RECIPE_CONTEXTS) -> dict:
    """The reference's own speed recipe (run_reasoni_speed_compare.sh:16-28): a random-init
    DeepSeek-R1-Distill-Qwen-1.5B-shaped model (28 layers, 12 q / 2 kv heads, qkv bias, bf16),
    batch 64, max_len 18432, subset 64 pages, compression ratio 1, full layers 0 1 2 14 22 (so
    layers 2, 14 and 22 are planners, each re-selecting the pages of the subset layers after it,
    model.py:177-196), one hipGraph per step; selective and full-cache decode at several
    contexts of the generation the recipe runs (its prompts are 4 tokens, so the context at a
    step is the step index)."""
    from delta_amd.backend import LMBackend
    from delta_amd import ops
    B, max_len, budget_pages = 64, 18432, 64
    extra = 2 * (warmup + steps) + 16
    eng = LMBackend(dtype=torch.bfloat16, device="cuda:0", cuda_graph_decode=True)
    eng.load_model("random:DeepSeek-R1-Distill-Qwen-1.5B", seed=0)
    cfg = eng.model.config
    cfg.enable_selective_cache = True
    cfg.full_cache_layers = [0, 1, 2, 14, 22]
    cfg.subset_cache_size = budget_pages
    cfg.compression_ratio = 1.0
    cfg.L = 8
    eng.setup_caches(max_batch_size=B, max_seq_length=max_len)
    roles = eng.layer_roles
    out = {"workload": "reference speed recipe: DeepSeek-R1-Distill-Qwen-1.5B-shaped decode step, B=64, "
                       "max_len 18432, 64-page budget (L=8, compression ratio 1), full layers [0,1,2,14,22] "
                       "(planners at 2, 14, 22), one hipGraph per step",
           "planner_layers": [i for i, r in enumerate(roles) if r == "plan"],
           "planner_logits_on_chip": eng._plan_on_chip(), "contexts": {}}
    for ctx in contexts:
        eng.enable_selective_cache = True
        eng.prepare_synthetic_decode(ctx, decode_budget=extra, seed=0)
        ms = time_steps(torch, eng, warmup, steps)
        eng.enable_selective_cache = False
        eng._decode_graph = None
        ms_full = time_steps(torch, eng, warmup, steps)
        out["contexts"][str(ctx)] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(B / ms * 1e3, 2),
                                     "full_cache_ms_per_step": round(ms_full, 4),
                                     "full_cache_tokens_per_s": round(B / ms_full * 1e3, 2),
                                     "speedup_vs_full_cache": round(ms_full / ms, 3)}
        log(f"  recipe ctx {ctx}: selective {ms:.3f} ms/step, full cache {ms_full:.3f} ms/step "
            f"({ms_full / ms:.2f}x)")
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()
    return out


def time_steps(torch, eng, warmup: int, steps: int) -> float:
    """ms per decode step over ``steps`` graph replays (after ``warmup`` replays)."""
    eng.decode_steps(warmup)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    eng.decode_steps(steps)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graph_timed(torch, calls, n_warm: int, replays: int = 3, passes: int = 3) -> float:
    """Average device time of one of ``calls`` (kernel launches), in us: the best of ``passes``
    timed passes of ``replays`` graph replays each (clock ramps and other processes' noise
    only ever add time).

    The launches are captured in one hipGraph and replayed, with HIP events on the replay
    stream around the replays, so host launch overhead never enters the figure (a 10 us kernel
    launched eagerly from Python is launch-bound).  The first ``n_warm`` calls run eagerly
    first (workspaces sized, code loaded)."""
    for f in calls[:n_warm]:
        f()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in calls[:n_warm]:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # under inference mode (as the engine captures): the CUDA generator's state, which the capture
    # updates in place, may have been created there
    with torch.inference_mode(), torch.cuda.graph(g):
        for f in calls:
            f()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    best = float("inf")
    for _ in range(passes):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(replays):
            g.replay()
        e.record(stream)
        torch.cuda.synchronize()
        best = min(best, s.elapsed_time(e) * 1e3 / (replays * len(calls)))
    del g
    return best


def warm_up(torch, run, seconds: float = 0.25):
    """Keep the GPU busy with ``run`` (a timed launch loop, result discarded) for ``seconds``
    before the measurements: after the host-side set-up the GPU comes back at reduced clocks,
    and the first ~20 ms of launches on fresh buffers read ~2 us slower at the config-3 subset
    shape (the steady state is what a decode loop runs at)."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        run()
    torch.cuda.synchronize()


def kernel_roofline(torch, reps: int = 60, n_rot: int = 30):
    """Time each hot-path kernel at the config-3 layer shape (graph replays, HIP events on the
    replay stream).

    Launches rotate over ``n_rot`` independent layers (own 1 GB KV cache, q and selection), as
    the 30 selective layers of a step do: no launch re-reads a working set left in the 256 MB
    MALL by the previous one, and the launches see the step's spread of cache addresses (with 4
    layers the subset launch reads ~1 us faster)."""
    from delta_amd import kernels as K
    from delta_amd.workloads import make_case
    layers, appends = [], []
    for seed in range(n_rot):
        c = make_case(batch=BATCH, hq=32, hkv=8, kv_lens=CONTEXT, dtype=torch.bfloat16, seed=seed,
                      page_order="shuffle", k=BUDGET_PAGES, L=L_LAST, device="cuda:0")
        B, hq = c.q.shape[:2]
        mp = c.max_pages
        dump = torch.empty((B, hq, mp * 16), device="cuda:0")
        lse = torch.empty((B, hq), device="cuda:0")
        K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, max_pages_per_row=mp,
                       lse=lse, logits_dump=dump)
        scores = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
        idx, ip = K.select_pages(scores, c.kv_indptr, c.block_table, c.k, c.L)
        layers.append((c, dump, lse, scores, idx, ip))
        # the decode token's (k, v) and position for the fused RoPE + append launches the step makes
        hkv_ = c.kv_cache.shape[3]
        g = torch.Generator(device="cuda:0").manual_seed(100 + seed)
        appends.append(K.DecodeAppend(
            torch.randn((B, hkv_, 128), generator=g, device="cuda:0").to(torch.bfloat16),
            torch.randn((B, hkv_, 128), generator=g, device="cuda:0").to(torch.bfloat16),
            torch.tensor([n - 1 for n in c.kv_lens], dtype=torch.int32, device="cuda:0"),
            c.kv_indptr, c.kv_indices, rope_scale=1.0, rope_theta=500000.0))
    torch.cuda.synchronize()
    c = layers[0][0]
    B, hq = c.q.shape[:2]
    hkv = c.kv_cache.shape[3]
    mp = c.max_pages
    esz = c.kv_cache.element_size()
    last = c.kv_last_page_len.cpu()
    ntok_full = sum(c.kv_lens)
    ntok_sub = sum((c.k - 1) * 16 + int(x) for x in last)
    qo = 2 * B * hq * 128 * esz
    row_kv = hkv * 128 * esz  # one token of K (or V) for all kv heads

    def timed(fn):
        return graph_timed(torch, [lambda i=i: fn(*layers[i % n_rot]) for i in range(reps)], n_rot)

    def timed_ap(fn):
        return graph_timed(torch, [lambda i=i: fn(*layers[i % n_rot], appends[i % n_rot]) for i in range(reps)],
                           n_rot)

    res = {}

    def add(name, us, nbytes, note):
        res[name] = {"us": round(us, 2), "bytes": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), "what": note}

    warm_up(torch, lambda: timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                                          c.kv_last_page_len, max_pages_per_row=mp)))
    # the fused launches also read the token's k and v and write them into its cache slot
    ap_bytes = 2 * 2 * B * hkv * 128 * esz + 2 * B * 4
    add("paged_decode_subset_kernel<ROPE>",
        timed_ap(lambda c, d, l, s, i, p, a: K.paged_decode(c.q, c.kv_cache, p, i, c.kv_last_page_len,
                                                             max_pages_per_row=c.k, subset=True, append=a)),
        ntok_sub * 2 * row_kv + qo + B * c.k * 4 + ap_bytes,
        "the launch a decode step makes in each selective layer (delta_paged_decode_subset_append): "
        "K+V of the 128 selected pages/row, q, o, page ids, the token's k/v read and appended")
    add("paged_decode_plan_kernel<ROPE>",
        timed_ap(lambda c, d, l, s, i, p, a: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                             c.kv_last_page_len, max_pages_per_row=mp, lse=l,
                                                             logits_dump=d, append=a)),
        ntok_full * 2 * row_kv + qo + B * mp * 4 + ntok_full * hq * 4 + ap_bytes,
        "the planner launch of a decode step (delta_paged_decode_append with a dump)")
    if K.paged_decode_scores_supported(B, hq, hkv, mp, True):
        # the per-token maxima are written once and read once by the page-sum kernel
        add("planner on chip <ROPE> (plan_tokmax + tokmax_score)",
            timed_ap(lambda c, d, l, s, i, p, a: K.paged_decode_scores(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                                        c.kv_last_page_len, max_pages_per_row=mp,
                                                                        lse=l, scores=s, append=a)),
            ntok_full * 2 * row_kv + qo + B * mp * 4 + ap_bytes + 2 * ntok_full * hkv * 4 + B * mp * 4,
            "the planner launch pair of a decode step with its logits on chip (delta_paged_decode_scores_append): "
            "K+V of all pages, q, o, page ids, the token's k/v, per-token maxima written and summed, scores")
    add("paged_decode_subset_kernel",
        timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, p, i, c.kv_last_page_len,
                                                       max_pages_per_row=c.k, subset=True)),
        ntok_sub * 2 * row_kv + qo + B * c.k * 4, "K+V of the 128 selected pages/row, q, o, page ids")
    add("paged_decode_full_kernel",
        timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                       c.kv_last_page_len, max_pages_per_row=mp)),
        ntok_full * 2 * row_kv + qo + B * mp * 4, "K+V of all 512 pages/row, q, o, page ids")
    add("paged_decode_plan_kernel",
        timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                       c.kv_last_page_len, max_pages_per_row=mp, lse=l,
                                                       logits_dump=d)),
        ntok_full * 2 * row_kv + qo + B * mp * 4 + ntok_full * hq * 4,
        "planner: full attention + fp32 logits dump")
    add("legacy_softmax_score_kernel",
        timed(lambda c, d, l, s, i, p: K.page_scores_from_logits(d, c.kv_indptr, c.kv_last_page_len, mp, lse=l,
                                                                  scores=s)),
        ntok_full * hq * 4 + B * mp * 4, "reads the logits dump once, writes page scores")
    add("page_score_kv (standalone scorer)",
        timed(lambda c, d, l, s, i, p: K.page_score(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                     c.kv_last_page_len, mp, scores=s)),
        ntok_full * row_kv + B * hq * 128 * esz + B * mp * 4 + B * mp * 4,
        "K read once + q + page table + scores (logits on chip where they fit, else a spilled dump)")
    add("select_pages_kernel",
        timed(lambda c, d, l, s, i, p: K.select_pages(s, c.kv_indptr, c.block_table, c.k, c.L, out_indices=i,
                                                       out_indptr=p)),
        B * mp * 4 * 2 + B * c.k * 4, "latency-bound selection (reported in us)")
    del layers, c
    torch.cuda.empty_cache()
    return res


def prefill_roofline(torch, n: int = 8192):
    """The causal paged prefill kernel on one ``n``-token prompt at the Llama-3-8B layer shape
    (32 q / 8 kv heads, bf16, shuffled pages): MFMA-bound, so reported in TFLOP/s of the two
    attention products over the causal pairs (4 * n (n + 1) / 2 * Hq * 128 flops)."""
    from delta_amd import kernels as K
    from delta_amd.workloads import make_case
    c = make_case(batch=1, hq=32, hkv=8, kv_lens=[n], dtype=torch.bfloat16, seed=0, page_order="shuffle",
                  k=4, L=2, device="cuda:0")
    q = torch.randn(n, 32, 128, device="cuda:0", dtype=torch.bfloat16)
    qo = torch.tensor([0, n], dtype=torch.int32, device="cuda:0")
    out = torch.empty_like(q)
    run = lambda: K.paged_prefill(q, c.kv_cache, qo, c.kv_indptr, c.kv_indices, c.kv_last_page_len, max_qo_len=n,
                                  out=out)
    warm_up(torch, run, 0.1)  # launches ramp from ~0.82 to ~0.62 ms over the first ~30 ms
    us = graph_timed(torch, [run] * 4, 1)
    flops = 4 * (n * (n + 1) / 2) * 32 * 128
    del c, q, out
    torch.cuda.empty_cache()
    return {"us": round(us, 2), "tokens": n, "TFLOP_s": round(flops / us / 1e6, 1), "peak_TFLOP_s": PEAK_BF16_TFLOPS,
            "frac": round(flops / us / 1e6 / PEAK_BF16_TFLOPS, 4),
            "what": f"causal prefill of one {n}-token prompt, 32q/8kv heads, bf16 (MFMA-bound)"}


def config_kernels(torch, config: int, reps: int = 12, n_rot: int = 2):
    """Planner, score, selection and subset-attention kernels at one layer of BASELINE config
    ``config`` (2, 4 or 5) at its full size, timed in graph replays over ``n_rot`` rotating layers.
    Algorithmic bytes count each row's real pages (ragged rows, per-row budgets)."""
    from delta_amd import kernels as K
    from delta_amd.workloads import config_case
    layers = []
    for r in range(n_rot):
        c = config_case(config, device="cuda:0")
        if r:  # independent K/V and q for the rotation (same shapes and page tables)
            c.kv_cache.normal_()
            c.q.normal_()
        B, hq = c.q.shape[:2]
        mp = c.max_pages
        dump = torch.empty((B, hq, mp * 16), device="cuda:0")
        lse = torch.empty((B, hq), device="cuda:0")
        K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, max_pages_per_row=mp,
                       lse=lse, logits_dump=dump)
        scores = K.page_scores_from_logits(dump, c.kv_indptr, c.kv_last_page_len, mp, lse=lse)
        idx, ip = K.select_pages(scores, c.kv_indptr, c.block_table, c.k, c.L, k_per_row=c.k_per_row)
        layers.append((c, dump, lse, scores, idx, ip))
    torch.cuda.synchronize()
    c, _, _, _, _, ip = layers[0]
    B, hq = c.q.shape[:2]
    hkv = c.kv_cache.shape[3]
    esz = c.kv_cache.element_size()
    mp = c.max_pages
    kmax = int(c.k_per_row.max()) if c.k_per_row is not None else c.k
    last = c.kv_last_page_len.cpu().tolist()
    nsel = (ip[1:] - ip[:-1]).cpu().tolist()
    npages = (c.kv_indptr[1:] - c.kv_indptr[:-1]).cpu().tolist()
    ntok_full = sum(c.kv_lens)
    ntok_sub = sum((n - 1) * 16 + l if n else 0 for n, l in zip(nsel, last))
    row_kv = hkv * 128 * esz
    qo = 2 * B * hq * 128 * esz

    def timed(fn):
        return graph_timed(torch, [lambda i=i: fn(*layers[i % n_rot]) for i in range(reps)], n_rot)

    res = {"shape": f"B={B}, {hq}q/{hkv}kv, {ntok_full} cached tokens ({min(c.kv_lens)}-{max(c.kv_lens)} per row), "
                    f"{sum(nsel)} selected pages, {str(c.kv_cache.dtype).replace('torch.', '')}"}
    warm_up(torch, lambda: timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                                          c.kv_last_page_len, max_pages_per_row=mp)))

    def add(name, us, nbytes):
        res[name] = {"us": round(us, 2), "bytes": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)}

    add("paged_decode_plan_kernel",
        timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                       c.kv_last_page_len, max_pages_per_row=mp, lse=l,
                                                       logits_dump=d)),
        ntok_full * 2 * row_kv + qo + sum(npages) * 4 + ntok_full * hq * 4)
    add("legacy_softmax_score_kernel",
        timed(lambda c, d, l, s, i, p: K.page_scores_from_logits(d, c.kv_indptr, c.kv_last_page_len, mp, lse=l,
                                                                  scores=s)),
        ntok_full * hq * 4 + B * mp * 4)
    add("select_pages_kernel",
        timed(lambda c, d, l, s, i, p: K.select_pages(s, c.kv_indptr, c.block_table, c.k, c.L,
                                                       k_per_row=c.k_per_row, out_indices=i, out_indptr=p)),
        B * mp * 4 * 2 + sum(nsel) * 4)
    add("paged_decode_subset_kernel",
        timed(lambda c, d, l, s, i, p: K.paged_decode(c.q, c.kv_cache, p, i, c.kv_last_page_len,
                                                       max_pages_per_row=kmax, subset=True)),
        ntok_sub * 2 * row_kv + qo + sum(nsel) * 4)
    add("page_score_kv (standalone scorer)",
        timed(lambda c, d, l, s, i, p: K.page_score(c.q, c.kv_cache, c.kv_indptr, c.kv_indices,
                                                     c.kv_last_page_len, mp, scores=s)),
        ntok_full * row_kv + B * hq * 128 * esz + sum(npages) * 4 + B * mp * 4)
    del layers, c
    torch.cuda.empty_cache()
    return res


def profiled_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy of known size); None when the summary does not list it."""
    path = os.path.join(ROOT, "profiles", "decode_kernels_config3_roofline.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


def copy_calibration(torch, mib: int = 256, reps: int = 8):
    """A plain device copy of known size (``mib`` MiB read + ``mib`` MiB written per launch).

    Run under ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` beside the hot-path kernels, it
    gives the factor between those counters and real bytes on this GPU."""
    n = mib * (1 << 20) // 2
    src = torch.randn(n, device="cuda:0", dtype=torch.float32).to(torch.bfloat16)
    dst = torch.empty_like(src)
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    s.record()
    for _ in range(reps):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) * 1e3 / reps
    nbytes = 2 * n * 2
    del src, dst
    torch.cuda.empty_cache()
    return {"us": round(us, 2), "bytes": nbytes, "GB_s": round(nbytes / us / 1e3, 1),
            "what": f"torch bf16 copy of {mib} MiB (read + write)"}


def cpu_model_name() -> str:
    """The host CPU's model string (/proc/cpuinfo; lscpu's "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, warm: int = 2, reps: int = 5) -> float:
    """Seconds: median of ``reps`` timed calls after ``warm`` untimed ones."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_layer_ops(torch, c, rows=None):
    """Per-op oracle timings (fp32 on the host) of one layer case, in seconds for the rows of
    ``c``: planner scorer (logits dump + del3_legacy_softmax scores), v2 selector, sparse decode
    attention over the selection, full decode attention.  Per-row budgets select row by row."""
    from oracle import delta_oracle as O
    f32 = torch.float32
    q = c.q.float()
    cache = c.kv_cache.float()
    scale = 1 / math.sqrt(128)
    B = q.shape[0]
    mp = c.max_pages
    counts = c.kv_indptr[1:] - c.kv_indptr[:-1]

    def score():
        x = O.dump_logits(q, cache, c.kv_indptr, c.kv_indices, c.kv_last_page_len, scale, mp * 16,
                          compute_dtype=f32)
        return O.legacy_softmax_page_scores(x, B, mp)

    scores = score()

    def select():
        if c.k_per_row is None:
            return O.select_pages(scores, counts, c.block_table, c.k, c.L)
        idx, ip = [], [0]
        for b in range(B):
            i, _ = O.select_pages(scores[b:b + 1], counts[b:b + 1], c.block_table[b:b + 1], int(c.k_per_row[b]),
                                  c.L)
            idx.append(i)
            ip.append(ip[-1] + i.numel())
        return torch.cat(idx), torch.tensor(ip, dtype=torch.int32)

    idx, ip = select()
    t = {"scorer": _median_time(score), "selector": _median_time(select),
         "sparse_layer": _median_time(lambda: O.paged_decode_attention(q, cache, ip, idx, c.kv_last_page_len,
                                                                       scale, compute_dtype=f32)),
         "full_layer": _median_time(lambda: O.paged_decode_attention(q, cache, c.kv_indptr, c.kv_indices,
                                                                     c.kv_last_page_len, scale, compute_dtype=f32))}
    return t


def cpu_baseline(torch, sample_rows: int = 2):
    """The oracle's PyTorch-CPU restatement of the same math (fp32, bf16/fp16 inputs upcast
    exactly), timed on this host's cores: 2 warm-ups, then the median of 5.

    ``value``: config 3 decode-step tokens/s, composed from per-op timings of ``sample_rows``
    rows of the config-3 layer (scaled to the batch) plus the dense decoder layer and lm_head at
    the full batch with random fp32 weights: 2 full layers (one the planner, with its dump,
    score and selection) + 30 subset layers + 32 dense layers + lm_head.  ``per_op`` holds the
    per-op timings at every config's real shape (configs 4 and 5 on sampled rows, scaled by
    their share of the cached tokens) and the whole selective step of configs 1 and 2 (no
    sampling)."""
    from delta_amd.workloads import config_case, make_case
    from oracle import delta_oracle as O
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t_start = time.perf_counter()

    c = make_case(batch=sample_rows, hq=32, hkv=8, kv_lens=CONTEXT, dtype=torch.float32, seed=0,
                  page_order="shuffle", k=BUDGET_PAGES, L=L_LAST)
    ops3 = _cpu_layer_ops(torch, c)
    per_row = (ops3["full_layer"] + (ops3["full_layer"] + ops3["scorer"] + ops3["selector"])
               + 30 * ops3["sparse_layer"]) / sample_rows
    dim, inter, vocab = 4096, 14336, 128256
    g = torch.Generator().manual_seed(0)
    w = {n: torch.randn(shape, generator=g) * 0.02 for n, shape in
         (("wqkv", (6144, dim)), ("wo", (dim, dim)), ("w1", (inter, dim)), ("w3", (inter, dim)),
          ("w2", (dim, inter)))}
    x = torch.randn(BATCH, dim, generator=g)

    def dense():
        h = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-5)
        qkv = h @ w["wqkv"].T
        y = x + qkv[:, :dim] @ w["wo"].T
        hn = y * torch.rsqrt((y * y).mean(-1, keepdim=True) + 1e-5)
        return y + (torch.nn.functional.silu(hn @ w["w1"].T) * (hn @ w["w3"].T)) @ w["w2"].T

    t_dense = _median_time(dense)
    del w
    lm = torch.randn(vocab, dim, generator=g) * 0.02
    t_head = _median_time(lambda: (x @ lm.T).argmax(-1))
    del lm
    step = BATCH * per_row + 32 * t_dense + t_head
    ms = lambda d: {k: round(v * 1e3, 2) for k, v in d.items()}
    per_op = {"config3": {"ms": ms({k: v * BATCH / sample_rows for k, v in ops3.items()}),
                          "rows_timed": sample_rows, "rows": BATCH}}
    # configs 1 and 2: the whole selective step of the layer (score, select, sparse attention), all rows
    for cfg in (1, 2):
        cc = config_case(cfg)
        o = _cpu_layer_ops(torch, cc)
        per_op[f"config{cfg}"] = {"ms": ms(o), "rows_timed": cc.batch, "rows": cc.batch,
                                  "selective_step_ms": round((o["scorer"] + o["selector"] + o["sparse_layer"]) * 1e3,
                                                             2)}
        del cc
    # configs 4 and 5 on sampled rows, scaled by the cached tokens they cover
    for cfg, rows in ((4, 1), (5, 2)):
        cc = config_case(cfg, batch=rows)
        o = _cpu_layer_ops(torch, cc)
        total_rows = 4 if cfg == 4 else 128
        if cfg == 5:
            import random as _r
            rng = _r.Random(0)
            all_lens = [rng.randint(1024, 32768) for _ in range(total_rows)]
            share = sum(all_lens) / sum(cc.kv_lens)
        else:
            share = total_rows / rows
        per_op[f"config{cfg}"] = {"ms": ms({k: v * share for k, v in o.items()}), "rows_timed": rows,
                                  "rows": total_rows, "scaled_by": round(share, 3)}
        del cc
    return {"value": round(BATCH / step, 3), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model_name(), "kind": "port",
            "sample": (f"oracle fp32 (PyTorch CPU), 2 warm-ups + median of 5 per op; config 3 step composed from "
                       f"{sample_rows} of {BATCH} rows of the layer scaled to the batch (full "
                       f"{ops3['full_layer'] * 1e3:.1f} ms, scorer {ops3['scorer'] * 1e3:.1f} ms, selector "
                       f"{ops3['selector'] * 1e3:.1f} ms, subset {ops3['sparse_layer'] * 1e3:.1f} ms per "
                       f"{sample_rows} rows), dense layer {t_dense * 1e3:.1f} ms and lm_head {t_head * 1e3:.1f} ms "
                       f"at batch {BATCH}: composed step {step:.2f} s"),
            "per_op": per_op, "wall_s": round(time.perf_counter() - t_start, 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-full-compare", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the kernel-level measurements at BASELINE configs 2, 4 and 5")
    ap.add_argument("--no-engine-config4", action="store_true",
                    help="skip the end-to-end decode step at BASELINE config 4")
    ap.add_argument("--engine-config4-only", action="store_true",
                    help="only the config-4 decode step (selective and full cache; for kernel traces)")
    ap.add_argument("--no-engine-config5", action="store_true",
                    help="skip the end-to-end decode step at BASELINE config 5")
    ap.add_argument("--engine-config5-only", action="store_true",
                    help="only the config-5 decode step (selective and full cache)")
    ap.add_argument("--no-engine-recipe", action="store_true",
                    help="skip the reference speed recipe's decode step (DeepSeek-R1-Distill-Qwen-1.5B shape)")
    ap.add_argument("--engine-recipe-only", action="store_true",
                    help="only the reference speed recipe's decode step, selective and full cache")
    ap.add_argument("--recipe-contexts", default=",".join(str(c) for c in RECIPE_CONTEXTS),
                    help="contexts the speed recipe's decode step is measured at (comma separated)")
    ap.add_argument("--kernel-reps", type=int, default=60)
    ap.add_argument("--configs-only", action="store_true",
                    help="only the kernel-level measurements at BASELINE configs 2, 4 and 5 (for rocprofv3 runs)")
    ap.add_argument("--configs", default="2,4,5",
                    help="which of BASELINE configs 2, 4, 5 --configs-only measures (comma separated)")
    ap.add_argument("--cpu-baseline-only", action="store_true",
                    help="only the CPU baseline (runs without a GPU)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the per-kernel roofline loop and a copy of known size (for rocprofv3 --pmc runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill kernel measurement (for rocprofv3 runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The selective decode shards by batch with no cross-GPU exchange; run --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.cpu_baseline_only:
        print(json.dumps({"cpu_baseline": cpu_baseline(torch)}), flush=True)
        return
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    torch.manual_seed(0)
    if args.engine_config4_only:
        log("engine at config 4 (Qwen2.5-7B shape, B=4, 64k context)")
        eng4 = engine_config4(torch, args.warmup, args.steps)
        log(f"  selective {eng4['ms_per_step']:.3f} ms/step ({eng4['tokens_per_s']} tokens/s), full cache "
            f"{eng4['full_cache_ms_per_step']:.3f} ms/step: {eng4['speedup_vs_full_cache']}x")
        print(json.dumps({"engine_config4": eng4}), flush=True)
        return
    if args.engine_config5_only:
        log("engine at config 5 (Qwen2.5-14B shape, B=128 ragged, per-row budgets)")
        eng5 = engine_config5(torch, args.warmup, args.steps)
        log(f"  selective {eng5['ms_per_step']:.3f} ms/step, full cache {eng5['full_cache_ms_per_step']:.3f} ms/step: "
            f"{eng5['speedup_vs_full_cache']}x")
        print(json.dumps({"engine_config5": eng5}), flush=True)
        return
    if args.engine_recipe_only:
        log("engine at the reference speed recipe (DeepSeek-R1-Distill-Qwen-1.5B shape, B=64)")
        ctxs = tuple(int(x) for x in args.recipe_contexts.split(","))
        print(json.dumps({"engine_recipe": engine_recipe(torch, args.warmup, args.steps, ctxs)}), flush=True)
        return
    if args.configs_only:
        out = {}
        for cfg in sorted({int(x) for x in args.configs.split(",")} & {2, 4, 5}):
            out[f"config{cfg}"] = config_kernels(torch, cfg, reps=args.kernel_reps // 4 or 1)
            for k, v in out[f"config{cfg}"].items():
                if isinstance(v, dict):
                    log(f"  config {cfg} {k}: {v['us']} us, {v['GB_s']} GB/s")
            torch.cuda.empty_cache()
        print(json.dumps({"kernels_other_configs": out}), flush=True)
        return
    if args.prefill_only:
        prefill = prefill_roofline(torch)
        log(f"  paged_prefill_kernel: {prefill['us']} us, {prefill['TFLOP_s']} TFLOP/s "
            f"({100 * prefill['frac']:.1f}% of bf16 MFMA peak)")
        print(json.dumps({"prefill": prefill}), flush=True)
        return
    if args.kernels_only:
        kern = kernel_roofline(torch, args.kernel_reps)
        kern["copy_calibration"] = copy_calibration(torch)
        for k, v in kern.items():
            log(f"  {k}: {v['us']} us, {v['GB_s']} GB/s")
        print(json.dumps({"kernels": kern}), flush=True)
        return
    budget = args.warmup + args.steps + 16
    if not args.no_full_compare:
        budget += args.warmup + args.steps
    log(f"building engine ({MODEL}, B={BATCH}, ctx={CONTEXT})")
    eng = build_engine(torch, budget)
    log("selective decode (hipGraph)")
    ms = time_steps(torch, eng, args.warmup, args.steps)
    tok_s = BATCH / ms * 1e3
    log(f"selective: {ms:.3f} ms/step, {tok_s:.1f} tokens/s")
    full = None
    if not args.no_full_compare:
        eng.enable_selective_cache = False
        eng._decode_graph = None
        ms_full = time_steps(torch, eng, args.warmup, args.steps)
        full = {"ms_per_step": round(ms_full, 4), "tokens_per_s": round(BATCH / ms_full * 1e3, 2)}
        log(f"full cache: {ms_full:.3f} ms/step")
    from delta_amd import ops
    ops.set_active_backend(None)
    del eng
    torch.cuda.empty_cache()
    log("kernel roofline")
    kern = kernel_roofline(torch, args.kernel_reps)
    for k, v in kern.items():
        log(f"  {k}: {v['us']} us, {v['GB_s']} GB/s ({100 * v['frac']:.1f}% of peak)")
    dom = kern["paged_decode_subset_kernel<ROPE>"]  # the launch each selective layer of a step makes
    log("prefill kernel")
    try:
        prefill = prefill_roofline(torch)
        log(f"  paged_prefill_kernel: {prefill['us']} us, {prefill['TFLOP_s']} TFLOP/s "
            f"({100 * prefill['frac']:.1f}% of bf16 MFMA peak)")
    except Exception as exc:  # reported in the line, never fatal for the headline number
        prefill = {"error": repr(exc)}
        log(f"  failed: {exc!r}")
    torch.cuda.empty_cache()
    others = None
    if not args.no_other_configs:
        others = {}
        for cfg in (2, 4, 5):
            log(f"kernels at config {cfg}")
            try:
                others[f"config{cfg}"] = config_kernels(torch, cfg)
                for k, v in others[f"config{cfg}"].items():
                    if isinstance(v, dict):
                        log(f"  {k}: {v['us']} us, {v['GB_s']} GB/s ({100 * v['frac']:.1f}% of peak)")
            except Exception as exc:  # reported in the line, never fatal for the headline number
                others[f"config{cfg}"] = {"error": repr(exc)}
                log(f"  failed: {exc!r}")
            torch.cuda.empty_cache()
    eng4 = None
    if not args.no_engine_config4:
        log("engine at config 4 (Qwen2.5-7B shape, B=4, 64k context)")
        try:
            eng4 = engine_config4(torch, args.warmup, args.steps)
            log(f"  selective {eng4['ms_per_step']:.3f} ms/step ({eng4['tokens_per_s']} tokens/s), full cache "
                f"{eng4['full_cache_ms_per_step']:.3f} ms/step: {eng4['speedup_vs_full_cache']}x")
        except Exception as exc:  # reported in the line, never fatal for the headline number
            eng4 = {"error": repr(exc)}
            log(f"  failed: {exc!r}")
        torch.cuda.empty_cache()
    eng5 = None
    if not args.no_engine_config5:
        log("engine at config 5 (Qwen2.5-14B shape, B=128 ragged, per-row budgets)")
        try:
            eng5 = engine_config5(torch, args.warmup, args.steps)
            log(f"  selective {eng5['ms_per_step']:.3f} ms/step ({eng5['tokens_per_s']} tokens/s), full cache "
                f"{eng5['full_cache_ms_per_step']:.3f} ms/step: {eng5['speedup_vs_full_cache']}x")
        except Exception as exc:  # reported in the line, never fatal for the headline number
            eng5 = {"error": repr(exc)}
            log(f"  failed: {exc!r}")
        torch.cuda.empty_cache()
    recipe = None
    if not args.no_engine_recipe:
        log("engine at the reference speed recipe (DeepSeek-R1-Distill-Qwen-1.5B shape, B=64)")
        try:
            recipe = engine_recipe(torch, args.warmup, args.steps)
        except Exception as exc:  # reported in the line, never fatal for the headline number
            recipe = {"error": repr(exc)}
            log(f"  failed: {exc!r}")
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle)")
        try:
            cpu = cpu_baseline(torch)
            log(f"  cpu: {cpu['value']} tokens/s on {cpu['cores']} cores")
        except Exception as exc:  # reported in the line, never fatal for the headline number
            cpu = {"error": repr(exc)}
            log(f"  failed: {exc!r}")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights, N(0,1) K/V, random current tokens",
        "config": {"workload": "config3: Llama-3-8B-shaped decode step, B=32, 8192-token context, "
                               "2048-token budget (128 pages, L=8), full layers [0,1], one hipGraph per step",
                   "batch": BATCH, "context": CONTEXT, "budget_pages": BUDGET_PAGES, "page_size": 16},
        "roofline": {"bound": "hbm", "achieved": dom["GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": dom["frac"], "traffic": profiled_traffic("paged_decode_subset_kernel<ROPE>"),
                     "algorithmic_bytes": dom["bytes"],
                     "kernel": "paged_decode_subset_kernel<ROPE> (delta_paged_decode_subset_append, the launch "
                               "of every selective layer in a decode step)"},
        "cpu_baseline": cpu,
        "full_cache": full,
        "speedup_vs_full_cache": round(tok_s / full["tokens_per_s"], 3) if full else None,
        "kernels": kern,
        "prefill": prefill,
        "kernels_other_configs": others,
        "engine_config4": eng4,
        "engine_config5": eng5,
        "engine_recipe": recipe,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
