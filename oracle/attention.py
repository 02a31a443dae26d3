"""Oracle: paged attention over a slot pool, gathered then attended (test infrastructure only).

Follows attention/backends.py of the reference:
  * ``SeqChunk``                 <- backends.py:36-47
  * ``context_slots``            <- backends.py:74-77   slot = table[p // bs] * bs + p % bs
  * ``build_attention_metadata`` <- backends.py:80-98   short rows (<= 8 new tokens) sorted by
                                    context, descending, grouped under 16,384 gathered tokens
  * ``_batched_group``           <- backends.py:101-132
  * ``_prefill_chunk``           <- backends.py:135-142
  * ``paged_attention``          <- backends.py:145-197
Also a float64 brute-force ``dense_attention`` that pins the above without any gathering tricks.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

SHORT_QUERY = 8  # backends.py:32
MAX_GATHER_TOKENS = 16384  # backends.py:33


@dataclass
class SeqChunk:
    """One scheduled sequence as attention sees it (backends.py:36-47)."""

    flat_start: int
    num_new: int
    num_cached: int
    block_table: list[int]

    @property
    def context_len(self) -> int:
        return self.num_cached + self.num_new


@dataclass
class _Group:
    q_index: Tensor  # [b, Q]
    valid_rows: Tensor | None  # [n]
    out_index: Tensor  # [n]
    ctx_slots: Tensor  # [b, L]
    mask: Tensor  # [b, Q, L]


@dataclass
class _Prefill:
    q_start: int
    q_end: int
    ctx_slots: Tensor | None
    mask: Tensor | None


@dataclass
class OracleMeta:
    slot_mapping: Tensor
    groups: list[_Group]
    prefills: list[_Prefill]


def context_slots(block_tables: Tensor, length: int, block_size: int) -> Tensor:
    """Page-table lookup for positions 0..length-1 (backends.py:74-77)."""
    pos = torch.arange(length)
    return block_tables[..., pos // block_size] * block_size + pos % block_size


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _group(chunks: list[SeqChunk], block_size: int) -> _Group:
    """backends.py:101-132: pad to the longest query and whole blocks; block 0 fills the gaps."""
    q_len = max(c.num_new for c in chunks)
    nb = _cdiv(max(c.context_len for c in chunks), block_size)
    ctx_len = nb * block_size
    tables = [c.block_table[:nb] + [0] * (nb - min(nb, len(c.block_table))) for c in chunks]
    q_index = [[c.flat_start + min(i, c.num_new - 1) for i in range(q_len)] for c in chunks]
    q_pos = [[c.num_cached + min(i, c.num_new - 1) for i in range(q_len)] for c in chunks]
    out_index = [c.flat_start + i for c in chunks for i in range(c.num_new)]
    all_valid = all(c.num_new == q_len for c in chunks)
    valid_rows = (
        None
        if all_valid
        else torch.tensor([b * q_len + i for b, c in enumerate(chunks) for i in range(c.num_new)])
    )
    slots = context_slots(torch.tensor(tables, dtype=torch.long), ctx_len, block_size)
    key_pos = torch.arange(ctx_len)
    mask = key_pos[None, None, :] <= torch.tensor(q_pos, dtype=torch.long)[:, :, None]
    return _Group(torch.tensor(q_index), valid_rows, torch.tensor(out_index), slots, mask)


def _prefill(c: SeqChunk, block_size: int) -> _Prefill:
    """backends.py:135-142: a fresh prompt is plain causal; a cached one sees tril(num_cached)."""
    if c.num_cached == 0:
        return _Prefill(c.flat_start, c.flat_start + c.num_new, None, None)
    nb = _cdiv(c.context_len, block_size)
    slots = context_slots(torch.tensor(c.block_table[:nb], dtype=torch.long), c.context_len, block_size)
    mask = torch.ones(c.num_new, c.context_len, dtype=torch.bool).tril(c.num_cached)
    return _Prefill(c.flat_start, c.flat_start + c.num_new, slots, mask)


def build_attention_metadata(
    chunks: list[SeqChunk], slot_mapping: Tensor, block_size: int
) -> OracleMeta:
    """backends.py:80-98."""
    short = sorted(
        (c for c in chunks if c.num_new <= SHORT_QUERY), key=lambda c: c.context_len, reverse=True
    )
    groups: list[_Group] = []
    current: list[SeqChunk] = []
    for c in short:
        if current and (len(current) + 1) * current[0].context_len > MAX_GATHER_TOKENS:
            groups.append(_group(current, block_size))
            current = []
        current.append(c)
    if current:
        groups.append(_group(current, block_size))
    prefills = [_prefill(c, block_size) for c in chunks if c.num_new > SHORT_QUERY]
    return OracleMeta(slot_mapping.cpu(), groups, prefills)


def paged_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    meta: OracleMeta,
    scale: float,
) -> Tensor:
    """Write K/V by slot, then gather + SDPA per group / per prefill (backends.py:145-197).

    q [T, H, D]; k, v [T, KVH, D]; caches [S, KVH, D], mutated in place. Returns [T, H, D].
    """
    k_cache.index_copy_(0, meta.slot_mapping, k)
    v_cache.index_copy_(0, meta.slot_mapping, v)
    out = torch.empty_like(q)
    heads, kv_heads, dim = q.shape[1], k.shape[1], q.shape[2]
    group = heads // kv_heads
    for g in meta.groups:
        b, q_len = g.q_index.shape
        qg = q[g.q_index].view(b, q_len, kv_heads, group, dim).permute(0, 2, 3, 1, 4)
        qg = qg.reshape(b, kv_heads, group * q_len, dim)
        kg = k_cache[g.ctx_slots].transpose(1, 2)
        vg = v_cache[g.ctx_slots].transpose(1, 2)
        if q_len == 1:
            mask = g.mask.unsqueeze(1)
        else:
            mask = g.mask.unsqueeze(1).expand(b, group, q_len, -1).reshape(b, 1, group * q_len, -1)
        og = F.scaled_dot_product_attention(qg, kg, vg, attn_mask=mask, scale=scale)
        og = og.view(b, kv_heads, group, q_len, dim).permute(0, 3, 1, 2, 4)
        og = og.reshape(b * q_len, heads, dim)
        out[g.out_index] = og if g.valid_rows is None else og[g.valid_rows]
    for p in meta.prefills:
        qp = q[p.q_start : p.q_end].transpose(0, 1).unsqueeze(0)
        if p.ctx_slots is None:
            kp, vp = k[p.q_start : p.q_end], v[p.q_start : p.q_end]
        else:
            kp, vp = k_cache[p.ctx_slots], v_cache[p.ctx_slots]
        kp = kp.repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0)
        vp = vp.repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0)
        if p.mask is None:
            op = F.scaled_dot_product_attention(qp, kp, vp, is_causal=True, scale=scale)
        else:
            op = F.scaled_dot_product_attention(qp, kp, vp, attn_mask=p.mask, scale=scale)
        out[p.q_start : p.q_end] = op[0].transpose(0, 1)
    return out


def dense_attention(
    q: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    chunks: list[SeqChunk],
    block_size: int,
    scale: float,
) -> Tensor:
    """float64 brute force: each query row of each sequence against its own context, read one
    slot at a time through the block table; query head h reads KV head h // (H / KVH).

    The caches must already hold this step's keys and values. Returns float64 [T, H, D].
    """
    heads, dim = q.shape[1], q.shape[2]
    kv_heads = k_cache.shape[1]
    group = heads // kv_heads
    out = torch.zeros(q.shape, dtype=torch.float64)
    for c in chunks:
        slots = [c.block_table[p // block_size] * block_size + p % block_size for p in range(c.context_len)]
        kc = k_cache[slots].double()  # [L, KVH, D]
        vc = v_cache[slots].double()
        for i in range(c.num_new):
            row = c.flat_start + i
            visible = c.num_cached + i + 1  # keys 0..position
            for h in range(heads):
                kh = kc[:visible, h // group]
                vh = vc[:visible, h // group]
                s = (kh @ q[row, h].double()) * scale
                p = torch.softmax(s, dim=0)
                out[row, h] = p @ vh
    return out


def default_scale(head_dim: int) -> float:
    """Qwen3Attention uses head_dim ** -0.5 (model/qwen3.py:73)."""
    return head_dim**-0.5
