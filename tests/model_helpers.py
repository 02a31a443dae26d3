"""Model-level helpers for the GPU parity tests: the HIP model and the CPU oracle built from the same
seeded weights, one oracle step, float64 copies of the int8 model, the decode-step workload.

Importable by the test modules (pytest puts tests/ on sys.path); nothing here touches the GPU
until a function is called.
"""

from __future__ import annotations

import random

import torch

from miniserve_amd import workloads
from miniserve_amd.quant.int8 import quantize_int8_
from miniserve_amd.runner.model_runner import ModelRunner, ScheduledChunk
from oracle import model as om

DEV = torch.device("cuda:0")


def pair(cfg, seed, max_positions, num_blocks, jitter=0.1, weights=None):
    """(runner, oracle config, oracle weights, oracle KV pool, rotary tables) for one seeded model:
    the HIP model quantized on the GPU, the oracle's weights quantized on the CPU; every layer's
    int8 pack is checked bit-equal between the two."""
    if weights is None:
        weights = workloads.random_weights(cfg, seed=seed, norm_jitter=jitter)
    model = workloads.build_model(cfg, weights, DEV, max_positions)
    quantize_int8_(model)
    runner = ModelRunner(model, DEV)
    runner.allocate_kv_cache(num_blocks)
    ocfg = om.Config.from_dict(cfg)
    ow = om.quantize_weights(weights, ocfg)
    for i in range(cfg["num_hidden_layers"]):
        for name in om.QUANTIZED:
            mod = model.layers[i].get_submodule(name)
            assert torch.equal(mod.qweight.cpu(), ow[f"layers.{i}.{name}.qweight"])
            assert torch.equal(mod.scale.cpu().view(torch.int16), ow[f"layers.{i}.{name}.scale"].view(torch.int16))
    shape = (num_blocks * 16, cfg["num_key_value_heads"], cfg["head_dim"])
    okv = [(torch.zeros(shape, dtype=torch.bfloat16), torch.zeros(shape, dtype=torch.bfloat16))
           for _ in range(cfg["num_hidden_layers"])]
    return runner, ocfg, ow, okv, om.tables_for(ocfg, max_positions)


def oracle_step(ocfg, ow, okv, tables, scheduled):
    """One oracle runner step over ScheduledChunks: (logits [R, V] float32, greedy ids [R])."""
    step = om.prepare([(s.token_ids, s.num_computed, s.num_new, s.block_table) for s in scheduled], 16)
    logits, ids = om.run_step(ocfg, ow, okv, step, 16, tables)
    return logits, ids


def margins(logits: torch.Tensor) -> torch.Tensor:
    """Per row, the gap between the two largest logits."""
    top = logits.topk(2, dim=-1).values
    return top[:, 0] - top[:, 1]


def copy_pool_to_oracle(runner, okv) -> None:
    for i, (kc, vc) in enumerate(runner.kv_caches):
        okv[i][0].copy_(kc.cpu())
        okv[i][1].copy_(vc.cpu())


def config3_case(seed: int, spare_blocks: int = 0):
    """The decode-step workload on the full Qwen3-0.6B-shaped int8 model: 64 sequences, contexts
    256 + U[0, 128], permuted block tables, an N(0, 1) pool shared with the oracle."""
    cfg = workloads.QWEN3_0_6B
    batch = workloads.decode_batch(64, 256, 384, seed=seed, vocab=cfg["vocab_size"], spare_blocks=spare_blocks)
    runner, ocfg, ow, okv, tables = pair(cfg, seed=seed, max_positions=4096, num_blocks=batch.num_blocks, jitter=0.0)
    workloads.fill_kv_pool_(runner.kv_cache, seed=seed + 1)
    copy_pool_to_oracle(runner, okv)
    rng = random.Random(seed + 2)
    used = {b for t in batch.block_tables for b in t}
    spare = iter(sorted(set(range(batch.num_blocks)) - used))
    sched = []
    for c, table, tok in zip(batch.context_lens, batch.block_tables, batch.token_ids, strict=True):
        table = list(table)
        if spare_blocks and c + 3 > 16 * len(table):  # room for the next steps' tokens
            table.append(next(spare))
        hist = [rng.randrange(cfg["vocab_size"]) for _ in range(c - 1)] + [tok]
        sched.append(ScheduledChunk(hist, c - 1, 1, table))
    return runner, ocfg, ow, okv, tables, sched


def dequantized64(ow: dict[str, torch.Tensor], layers: list[int] | None = None) -> dict[str, torch.Tensor]:
    """float64 copy of the int8 model: every quantized weight as its bf16(q * s) value (only the
    given layers' weights when ``layers`` is set, plus everything outside the layers)."""
    keep = None if layers is None else {f"layers.{i}." for i in layers}
    w64 = {}
    for k, v in ow.items():
        if keep is not None and k.startswith("layers.") and not any(k.startswith(p) for p in keep):
            continue
        if k.endswith(".qweight"):
            base = k[: -len(".qweight")]
            w64[base + ".weight"] = (v.to(torch.bfloat16) * ow[base + ".scale"].unsqueeze(1)).double()
        elif not k.endswith(".scale"):
            w64[k] = v.double()
    return w64
