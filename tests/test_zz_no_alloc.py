"""The allocation-free decode attention entry point (msa_paged_attention_decode_noalloc) against the
workspace entry point (msa_paged_attention_decode), both called through the C ABI on the same
inputs: bit-identical outputs on two calls in a row, the second with a smaller batch (the scratch
keeps the first call's partials; nothing in it may leak into the second)."""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

from miniserve_amd import _native, kernels

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(num_seqs, max_ctx, heads, kv_heads, seed):
    rng = random.Random(seed)
    ctx = [rng.randint(1, max_ctx) for _ in range(num_seqs)]
    need = [-(-c // 16) for c in ctx]
    total = sum(need) + 2
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).tolist()
    width = max(need)
    tables = torch.zeros(num_seqs, width, dtype=torch.int32)
    off = 0
    for i, n in enumerate(need):
        tables[i, :n] = torch.tensor(perm[off : off + n], dtype=torch.int32)
        off += n
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(num_seqs, heads, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(total * 16, kv_heads, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(total * 16, kv_heads, 128, generator=g).to(torch.bfloat16)
    rows = torch.randperm(num_seqs, generator=g).to(torch.int32)  # each plan row has its own q/out row
    return (q.to(DEV), kc.to(DEV), vc.to(DEV), tables.to(DEV), torch.tensor(ctx, dtype=torch.int32).to(DEV),
            rows.to(DEV))


def _both(num_seqs, max_ctx, heads, kv_heads, seed):
    q, kc, vc, tables, ctx, rows = _case(num_seqs, max_ctx, heads, kv_heads, seed)
    ptok, parts = kernels.decode_splits(num_seqs, kv_heads, tables.shape[1], heads // kv_heads)
    assert parts > 1  # the split partials go through the scratch
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    args = (_ptr(q), q.stride(0), _ptr(kc), _ptr(vc), kc.shape[0], heads, kv_heads, 128, 16, _ptr(tables),
            tables.shape[1], _ptr(ctx), _ptr(rows), num_seqs, ptok, parts, 128**-0.5)
    ws_bytes = _native.query("msa_paged_attention_decode_workspace_size", num_seqs, heads, 128, parts)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    ref = torch.full_like(q, 7.0)
    got = torch.full_like(q, -7.0)
    _native.call("msa_paged_attention_decode", *args, _ptr(ref), ref.stride(0), _ptr(ws), ws_bytes, stream)
    _native.call("msa_paged_attention_decode_noalloc", *args, _ptr(got), got.stride(0), stream)
    torch.cuda.synchronize()
    return got, ref


def test_noalloc_decode_matches_the_workspace_entry_point_twice():
    got, ref = _both(12, 3000, 16, 8, seed=1)  # 96 (sequence, KV head) pairs: keys split across workgroups
    assert torch.equal(got, ref)
    got, ref = _both(5, 700, 32, 8, seed=2)  # smaller, G = 4: the first call's partials are left behind
    assert torch.equal(got, ref)
