"""Test helpers shared by the CPU and GPU suites (importable: pytest puts tests/ on sys.path).

``oracle_run_chunk`` mirrors the reference's tests/helpers.py:27-49 (one sequence whose blocks are
0, 1, 2, ...) on top of the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from oracle import model as om
from oracle.attention import SeqChunk, build_attention_metadata


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def new_kv_caches(cfg: om.Config, num_slots: int, dtype: torch.dtype) -> list[tuple[Tensor, Tensor]]:
    shape = (num_slots, cfg.num_key_value_heads, cfg.head_dim)
    return [(torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)) for _ in range(cfg.num_hidden_layers)]


def oracle_run_chunk(
    cfg: om.Config,
    weights: dict[str, Tensor],
    kv: list[tuple[Tensor, Tensor]],
    ids: list[int],
    start: int,
    block_size: int,
    tables: tuple[Tensor, Tensor],
) -> Tensor:
    n = len(ids)
    table = list(range(cdiv(start + n, block_size)))
    slots = torch.tensor([table[p // block_size] * block_size + p % block_size for p in range(start, start + n)])
    meta = build_attention_metadata([SeqChunk(0, n, start, table)], slots, block_size)
    positions = torch.arange(start, start + n)
    with torch.inference_mode():
        hidden = om.forward(cfg, weights, torch.tensor(ids), positions, kv, meta, tables)
        return om.compute_logits(cfg, weights, hidden)


def bf16_bits_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns with round-to-nearest-even, in integer arithmetic."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def rel_l2(a: Tensor, b: Tensor) -> float:
    a64, b64 = a.double().flatten(), b.double().flatten()
    return float((a64 - b64).norm() / b64.norm().clamp_min(1e-30))
