"""Decode throughput of the int8 Qwen3-0.6B-shaped step at batch 64 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one "step"): 64 sequences each decode one token; contexts 256 + U[0, 128] tokens in a
paged KV pool of 16-token blocks (random permuted block tables, N(0,1) bf16 contents); a 28-layer
Qwen3-0.6B-architecture model with random N(0, 0.02) bf16 weights, every decoder linear int8 per
output channel, tied bf16 LM head. A step is what the runner does per engine step: build the flat
batch and attention metadata on the host, upload it (pinned, non-blocking), run the forward, the
LM head on the 64 sampled rows, greedy argmax, and the one device->host sync. The step runs as a
captured HIP graph (one replay per step, metadata uploaded to its static buffers first).

Prints ONE JSON line. ``roofline`` is for the dominant kernel, paged-attention decode (76% of the
step's bytes): algorithmic bytes per launch / its average duration, timed with HIP events on the
stream it runs on over one launch per layer (28 distinct KV pools, so the Infinity Cache cannot
serve repeats). ``cpu_baseline`` times the CPU oracle (a PyTorch restatement of the reference's
path, run on this host's cores) on the same step.
"""

from __future__ import annotations

import argparse
import json
import os
import random
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s at batch 64 (Qwen3-0.6B int8); int8 GEMV + attn HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
BATCH, CTX_LO, CTX_HI = 64, 256, 384


def attention_bytes(ctx: list[int], heads: int, kv_heads: int, dim: int) -> int:
    """Algorithmic bytes of one decode-attention launch: every context token's K and V for every
    KV head, the queries and outputs, the block-table entries read and the per-sequence ints."""
    kv = 2 * kv_heads * dim * 2 * sum(ctx)
    qo = 2 * len(ctx) * heads * dim * 2
    tables = 4 * sum(-(-c // 16) for c in ctx)
    return kv + qo + tables + 8 * len(ctx)


def time_attention(runner, sched, cfg, reps: int = 4) -> tuple[float, int]:
    """Average duration of the dominant kernel: one decode-attention launch per layer (28
    distinct KV pools) queued back to back behind a spin kernel, timed by one pair of HIP events
    on the stream the launches go to; returns (seconds per launch, algorithmic bytes per launch)."""
    import torch

    from miniserve_amd import kernels

    inp = runner.prepare(sched)
    d = inp.attn.decode
    heads, kvh, dim = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    ptok, parts = kernels.decode_splits(d.num_seqs, kvh, d.block_tables.shape[1])
    q = torch.randn(len(sched), heads, dim, device=runner.device).to(torch.bfloat16)
    out = torch.empty_like(q)
    spans = []
    for rep in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)
        e0.record()
        for kc, vc in runner.kv_caches:
            kernels.paged_attention_decode(q, kc, vc, d.block_tables, d.context_lens, d.q_rows, ptok, parts,
                                           dim**-0.5, out)
        e1.record()
        torch.cuda.synchronize()
        if rep:
            spans.append(e0.elapsed_time(e1) * 1e-3 / len(runner.kv_caches))
    ctx = [s.num_computed + 1 for s in sched]
    return sum(spans) / len(spans), attention_bytes(ctx, heads, kvh, dim)


def linear_bytes(m: int, n: int, k: int) -> int:
    """Algorithmic bytes of one int8 linear: int8 weights, bf16 scales, bf16 x in, bf16 y out."""
    return n * k + 2 * n + 2 * m * k + 2 * m * n


def time_linears(seed: int) -> list[dict]:
    """Average duration of the token-split int8 linear on the single gate_proj-shaped linear
    ([3072 x 1024], 16 tokens) and on the four decode-step linears at 64 tokens, each over enough
    distinct weight copies (> 256 MiB) that the Infinity Cache cannot serve repeats; HIP events on
    the launch stream around one pass over the copies, after a warm-up pass."""
    import torch

    from miniserve_amd import kernels

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    shapes = [("gate_proj [3072x1024], 16 tokens", 16, 3072, 1024, kernels.EPI_NONE),
              ("qkv [4096x1024] + q/k-norm/RoPE/cache, 64 tokens", 64, 4096, 1024, -1),
              ("o [1024x2048] + residual, 64 tokens", 64, 1024, 2048, kernels.EPI_RESIDUAL),
              ("gate_up [6144x1024] + norm + silu*up, 64 tokens", 64, 6144, 1024, kernels.EPI_SILU_MUL),
              ("down [1024x3072] + residual, 64 tokens", 64, 1024, 3072, kernels.EPI_RESIDUAL)]
    out = []
    for name, m, n, k, epi in shapes:
        copies = max(8, -(-(300 << 20) // (n * k)))
        ws = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device=dev, generator=g)
        sc = (torch.rand(copies, n, device=dev, generator=g) * 0.001).to(torch.bfloat16)
        x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        nw = torch.ones(k, dtype=torch.bfloat16, device=dev)
        resid = torch.randn(m, n, device=dev, generator=g).to(torch.bfloat16)
        y = torch.empty(m, n // 2 if epi == kernels.EPI_SILU_MUL else n, dtype=torch.bfloat16, device=dev)
        if epi == -1:
            heads, kvh = 16, 8
            pos = torch.arange(m, device=dev) + 300
            cos = torch.randn(4096, 128, device=dev)
            sin = torch.randn(4096, 128, device=dev)
            slots = torch.arange(m, device=dev)
            kc = torch.zeros(m, kvh, 128, dtype=torch.bfloat16, device=dev)
            vc = torch.zeros_like(kc)

            def run(i):
                kernels.qkv_rope_cache_rows(x, ws[i], sc[i], heads, kvh, 128, nw[:128], nw[:128], 1e-6, pos, cos, sin,
                                            slots, kc, vc, norm_w=nw, eps=1e-6)
        elif epi == kernels.EPI_SILU_MUL:
            def run(i):
                kernels.int8_linear_rows(x, ws[i], sc[i], epi, norm_w=nw, eps=1e-6, out=y)
        elif epi == kernels.EPI_RESIDUAL:
            def run(i):
                kernels.int8_linear_rows(x, ws[i], sc[i], epi, residual=resid, out=y)
        else:
            def run(i):
                kernels.int8_linear_rows(x, ws[i], sc[i], out=y)
        for i in range(copies):
            run(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(5_000_000)
        e0.record()
        for i in range(copies):
            run(i)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / copies
        nbytes = linear_bytes(m, n, k)
        out.append({"linear": name, "us_per_launch": round(us, 3), "bytes_per_launch": nbytes,
                    "GB_s": round(nbytes / us / 1e3, 1), "copies": copies})
        del ws, sc
    return out


def kernel_only(mode: str, seed: int) -> int:
    """Profiling entry points: ``attention`` runs only the decode-attention timing above on the
    bench workload; ``linear`` the int8 linear timings of ``time_linears``; ``copy`` copies a
    256 MiB buffer 10 times (a kernel of known traffic, to calibrate rocprofv3's FETCH_SIZE /
    WRITE_SIZE counters)."""
    import torch

    dev = torch.device("cuda:0")
    if mode == "linear":
        for row in time_linears(seed):
            print(json.dumps(row))
        return 0
    if mode == "copy":
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).normal_()
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2, "copies": 10}))
        return 0
    from miniserve_amd import workloads
    from miniserve_amd.runner.model_runner import ModelRunner, ScheduledChunk

    cfg = workloads.QWEN3_0_6B
    batch = workloads.decode_batch(BATCH, CTX_LO, CTX_HI, seed=seed + 1, vocab=cfg["vocab_size"], spare_blocks=64)

    runner = ModelRunner.__new__(ModelRunner)
    runner.device, runner.block_size = dev, 16
    kv = torch.empty(cfg["num_hidden_layers"], 2, batch.num_blocks * 16, cfg["num_key_value_heads"], cfg["head_dim"],
                     dtype=torch.bfloat16, device=dev)
    workloads.fill_kv_pool_(kv, seed=seed + 2, on_device=True)
    runner.kv_caches = [(kv[i, 0], kv[i, 1]) for i in range(kv.shape[0])]
    sched = [ScheduledChunk([0] * c, c - 1, 1, t) for c, t in zip(batch.context_lens, batch.block_tables, strict=True)]
    secs, nbytes = time_attention(runner, sched, cfg)
    print(json.dumps({"kernel": "paged_decode_kernel", "us_per_launch": secs * 1e6, "bytes_per_launch": nbytes,
                      "GB_s": nbytes / secs / 1e9}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", choices=["attention", "linear", "copy"], help="profiling entry point (see kernel_only)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if args.kernel_only:
        return kernel_only(args.kernel_only, args.seed)

    import torch

    from miniserve_amd import kernels, workloads
    from miniserve_amd.quant.int8 import quantize_int8_
    from miniserve_amd.runner.model_runner import ModelRunner, ScheduledChunk
    from miniserve_amd.runner.sampler import sample

    dev = torch.device("cuda:0")
    cfg = workloads.QWEN3_0_6B
    t0 = time.time()
    weights = workloads.random_weights(cfg, seed=args.seed)
    model = workloads.build_model(cfg, weights, dev, max_positions=4096)
    quantize_int8_(model)
    batch = workloads.decode_batch(BATCH, CTX_LO, CTX_HI, seed=args.seed + 1, vocab=cfg["vocab_size"], spare_blocks=64)
    runner = ModelRunner(model, dev, use_graphs=True, max_model_len=4096)
    runner.allocate_kv_cache(batch.num_blocks)
    workloads.fill_kv_pool_(runner.kv_cache, seed=args.seed + 2, on_device=True)
    rng = random.Random(args.seed + 3)
    sched = []
    for c, table, tok in zip(batch.context_lens, batch.block_tables, batch.token_ids, strict=True):
        sched.append(ScheduledChunk([rng.randrange(cfg["vocab_size"]) for _ in range(c - 1)] + [tok], c - 1, 1, table))
    torch.cuda.synchronize()
    print(f"[bench] setup {time.time() - t0:.1f}s: 28-layer int8 model, {batch.num_blocks} KV blocks", file=sys.stderr)

    def eager_step() -> list[int]:
        return sample(runner.forward_logits(runner.prepare(sched))).tolist()

    def timed(fn, steps: int, warmup: int) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / steps

    eager_dt = timed(eager_step, max(3, args.steps // 4), 2)
    graph_ids = runner.execute(sched)
    if [g[0] for g in graph_ids] != eager_step():
        raise RuntimeError("captured decode step disagrees with the eager step")
    dt = timed(lambda: runner.execute(sched), args.steps, args.warmup)
    tok_s = BATCH / dt
    print(f"[bench] eager {eager_dt * 1e3:.3f} ms/step; graph {args.steps} steps: {dt * 1e3:.3f} ms/step, "
          f"{tok_s:.0f} tok/s", file=sys.stderr)

    attn_s, attn_b = time_attention(runner, sched, cfg)
    achieved = attn_b / attn_s / 1e9
    print(f"[bench] decode attention: {attn_s * 1e6:.2f} us/launch, {achieved:.0f} GB/s", file=sys.stderr)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen3-0.6B-architecture int8 decode step (28 layers, random init)",
            "batch": BATCH,
            "context": f"{CTX_LO}+U[0,{CTX_HI - CTX_LO}]",
            "sum_context": sum(batch.context_lens),
            "kv_block": 16,
            "weights": "int8 per-output-channel, bf16 activations, fp32 accumulation, tied bf16 LM head",
            "parallelism": "none",
            "hip_graph": True,
            "eager_ms_per_step": round(eager_dt * 1e3, 4),
        },
        "roofline": {
            "kernel": "paged_decode_kernel<2, 8>",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": attn_b,
            "us_per_launch": round(attn_s * 1e6, 3),
        },
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, weights, runner, sched)
    print(json.dumps(result))
    return 0


def cpu_baseline(cfg, weights, runner, sched) -> dict:
    """The CPU oracle's decode step on this host (same weights, same KV contents, same batch)."""
    import platform

    import torch

    from oracle import model as om

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    ocfg = om.Config.from_dict(cfg)
    ow = om.quantize_weights(weights, ocfg)
    okv = [(kc.cpu(), vc.cpu()) for kc, vc in runner.kv_caches]
    tables = om.tables_for(ocfg, 4096)
    step = om.prepare([(s.token_ids, s.num_computed, s.num_new, s.block_table) for s in sched], 16)
    t = time.perf_counter()
    om.run_step(ocfg, ow, okv, step, 16, tables)  # warm-up
    first = time.perf_counter() - t
    reps = max(1, min(5, int(20.0 / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        om.run_step(ocfg, ow, okv, step, 16, tables)
        times.append(time.perf_counter() - t)
    times.sort()
    med = times[len(times) // 2]
    print(f"[bench] cpu oracle: {med:.3f} s/step on {cores} threads", file=sys.stderr)
    return {
        "value": round(BATCH / med, 2),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"the full decode step (64 tokens, 28 layers, LM head, argmax), median of {reps} after 1 warm-up",
        "cpu": platform.processor() or platform.machine(),
        "torch": torch.__version__,
    }


if __name__ == "__main__":
    sys.exit(main())
