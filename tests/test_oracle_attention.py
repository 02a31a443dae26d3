"""Pins the oracle's paged attention (reference attention/backends.py:74-197).

Against a float64 brute force that reads one slot at a time through the block table, plus the
invariants the reference relies on: permuted physical block placement changes nothing, and a
sequence attended in a batch equals the same sequence alone (the reference's
tests/correctness/test_engine_equivalence.py:34-39 pattern), including batches split into several
gather groups by the 16,384-token cap.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.attention import (
    MAX_GATHER_TOKENS,
    SeqChunk,
    build_attention_metadata,
    context_slots,
    dense_attention,
    paged_attention,
)


def _scenario(specs, heads, kv_heads, dim, bs, dtype, seed, num_blocks=None):
    """specs: list of (num_cached, num_new). Returns q, k, v, caches, chunks, slot_mapping."""
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    need = sum(-(-(c + n) // bs) for c, n in specs)
    num_blocks = num_blocks or need + 3
    perm = list(range(num_blocks))
    rng.shuffle(perm)
    chunks, slots, flat, used = [], [], 0, 0
    for cached, new in specs:
        nb = -(-(cached + new) // bs)
        table = perm[used : used + nb]
        used += nb
        chunks.append(SeqChunk(flat, new, cached, table))
        slots.extend(table[p // bs] * bs + p % bs for p in range(cached, cached + new))
        flat += new
    t = flat
    q = torch.randn(t, heads, dim, generator=g).to(dtype)
    k = torch.randn(t, kv_heads, dim, generator=g).to(dtype)
    v = torch.randn(t, kv_heads, dim, generator=g).to(dtype)
    kc = torch.randn(num_blocks * bs, kv_heads, dim, generator=g).to(dtype)
    vc = torch.randn(num_blocks * bs, kv_heads, dim, generator=g).to(dtype)
    return q, k, v, kc, vc, chunks, torch.tensor(slots, dtype=torch.long)


SPECS = [(37, 1), (0, 1), (15, 1), (16, 1), (5, 3), (40, 8), (0, 20), (33, 9), (3, 30)]


@pytest.mark.parametrize("bs", [4, 16])
def test_matches_float64_brute_force(bs: int) -> None:
    q, k, v, kc, vc, chunks, slots = _scenario(SPECS, 4, 2, 16, bs, torch.float64, seed=bs)
    meta = build_attention_metadata(chunks, slots, bs)
    out = paged_attention(q, k, v, kc, vc, meta, 16**-0.5)
    ref = dense_attention(q, kc, vc, chunks, bs, 16**-0.5)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)


def test_cache_write_by_slot() -> None:
    q, k, v, kc, vc, chunks, slots = _scenario(SPECS, 4, 2, 16, 16, torch.bfloat16, seed=1)
    meta = build_attention_metadata(chunks, slots, 16)
    paged_attention(q, k, v, kc, vc, meta, 0.25)
    assert torch.equal(kc[slots], k) and torch.equal(vc[slots], v)


def test_context_slots_closed_form() -> None:
    table = torch.tensor([[7, 2, 9], [1, 0, 4]])
    got = context_slots(table, 40, 16)
    for b in range(2):
        for p in range(40):
            assert int(got[b, p]) == int(table[b, p // 16]) * 16 + p % 16


def test_physical_placement_does_not_matter() -> None:
    bs = 16
    a = _scenario(SPECS, 4, 2, 16, bs, torch.bfloat16, seed=3)
    q, k, v, kc, vc, chunks, slots = a
    out1 = paged_attention(q, k, v, kc.clone(), vc.clone(), build_attention_metadata(chunks, slots, bs), 0.25)
    # Move every logical block to a new physical block, carrying its contents along.
    nblk = kc.shape[0] // bs
    move = torch.randperm(nblk, generator=torch.Generator().manual_seed(9))
    kc2, vc2 = torch.empty_like(kc), torch.empty_like(vc)
    for old in range(nblk):
        new = int(move[old])
        kc2[new * bs : (new + 1) * bs] = kc[old * bs : (old + 1) * bs]
        vc2[new * bs : (new + 1) * bs] = vc[old * bs : (old + 1) * bs]
    chunks2 = [SeqChunk(c.flat_start, c.num_new, c.num_cached, [int(move[b]) for b in c.block_table]) for c in chunks]
    slots2 = torch.tensor([int(move[int(s) // bs]) * bs + int(s) % bs for s in slots])
    out2 = paged_attention(q, k, v, kc2, vc2, build_attention_metadata(chunks2, slots2, bs), 0.25)
    assert torch.equal(out1, out2)


def test_batched_equals_alone_across_gather_groups() -> None:
    """Enough long decodes that the 16,384-token cap splits them into several groups."""
    bs = 16
    specs = [(700 + 37 * i, 1) for i in range(40)]
    assert sum(c + n for c, n in specs) > 2 * MAX_GATHER_TOKENS
    q, k, v, kc, vc, chunks, slots = _scenario(specs, 4, 2, 16, bs, torch.float64, seed=11)
    meta = build_attention_metadata(chunks, slots, bs)
    assert len(meta.groups) >= 2
    out = paged_attention(q, k, v, kc.clone(), vc.clone(), meta, 0.25)
    for i in (0, 17, 39):
        c = chunks[i]
        one = SeqChunk(0, 1, c.num_cached, c.block_table)
        alone = paged_attention(
            q[i : i + 1], k[i : i + 1], v[i : i + 1], kc.clone(), vc.clone(),
            build_attention_metadata([one], slots[i : i + 1], bs), 0.25,
        )
        torch.testing.assert_close(out[i], alone[0], atol=1e-12, rtol=1e-12)
