"""GPU parity of the token-split int8 kernels (fused prologues / epilogues) and of the fused LM
head + greedy argmax, against the CPU oracle on the same seeded inputs.

Bars: linears within rel-L2 1e-2 of the oracle and within bf16 rounding of a float64 product of
the same dequantized weights; gathered rows bit-exact; greedy ids equal to the argmax of the
reference's bf16 logits except where the two best logits are within one bf16 step (a rounding
tie), and exact first-index tie-breaking on planted exact ties. Every call goes through the C ABI.
"""

from __future__ import annotations

import pytest
import torch
from helpers import rel_l2

from miniserve_amd import kernels
from oracle import int8 as oi
from oracle import layers as ol

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _bf16(shape, seed, std=1.0):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * std).to(torch.bfloat16)


def _weights(n, k, seed):
    return oi.quantize_int8(_bf16((n, k), seed, std=0.02))


def _norm_w(dim, seed):
    return (1 + 0.1 * torch.randn(dim, generator=torch.Generator().manual_seed(seed))).to(torch.bfloat16)


ROWS_SHAPES = [
    (1, 1024, 2048),
    (5, 1024, 2048),
    (16, 3072, 1024),  # the gate_proj-shaped single linear
    (64, 4096, 1024),  # qkv
    (64, 1024, 2048),  # o
    (64, 1024, 3072),  # down
    (33, 512, 256),
    (100, 1024, 1024),
    (256, 1024, 512),
    (7, 48, 64),  # n not a multiple of the 16-row tile's block, a single K chunk
    (3, 1000, 4096),  # ragged rows, the largest K the activation tile takes here
]


@pytest.mark.parametrize("m,n,k", ROWS_SHAPES)
def test_rows_linear(m, n, k):
    q, s = _weights(n, k, seed=n + k)
    x = _bf16((m, k), seed=m)
    qd, sd, xd = q.to(DEV), s.to(DEV), x.to(DEV)
    y = kernels.int8_linear_rows(xd, qd, sd)
    y2 = kernels.int8_linear_rows(xd, qd, sd)
    assert torch.equal(y, y2)  # deterministic
    ref = oi.int8_linear(x, q, s)
    exact = x.double() @ oi.dequantize(q, s, torch.bfloat16).double().T
    assert rel_l2(y.cpu(), ref) < 1e-2
    assert rel_l2(y.cpu(), exact) < 4e-3


@pytest.mark.parametrize("m,n,k", [(1, 1024, 3072), (64, 1024, 2048), (64, 1024, 3072), (37, 256, 512)])
def test_rows_residual_in_place(m, n, k):
    q, s = _weights(n, k, seed=3 * n + k)
    x = _bf16((m, k), seed=m + 1)
    r = _bf16((m, n), seed=m + 2)
    rd = r.to(DEV)
    out = kernels.int8_linear_rows(x.to(DEV), q.to(DEV), s.to(DEV), kernels.EPI_RESIDUAL, residual=rd, out=rd)
    assert out.data_ptr() == rd.data_ptr()
    ref = r + oi.int8_linear(x, q, s)
    assert rel_l2(rd.cpu(), ref) < 1e-2
    # the residual add itself is exact on the kernel's own projection
    y = kernels.int8_linear_rows(x.to(DEV), q.to(DEV), s.to(DEV)).cpu()
    assert torch.equal(rd.cpu(), r + y)


@pytest.mark.parametrize("m", [1, 16, 64, 77, 200])
@pytest.mark.parametrize("with_norm", [True, False])
def test_rows_silu_mul(m, with_norm):
    n, k = 6144, 1024
    q, s = _weights(n, k, seed=m)
    x = _bf16((m, k), seed=m + 5)
    w = _norm_w(k, seed=m + 6)
    y = kernels.int8_linear_rows(
        x.to(DEV), q.to(DEV), s.to(DEV), kernels.EPI_SILU_MUL, norm_w=w.to(DEV) if with_norm else None, eps=1e-6
    )
    h = ol.rms_norm(x, w, 1e-6) if with_norm else x
    gate, up = oi.int8_linear(h, q, s).chunk(2, dim=-1)
    ref = torch.nn.functional.silu(gate) * up
    assert y.shape == (m, n // 2)
    assert rel_l2(y.cpu(), ref) < 1e-2
    # against the two-kernel composition on the GPU: norm prologue + product + silu*up
    if with_norm:
        hd = kernels.rmsnorm(x.to(DEV), w.to(DEV), 1e-6)
        plain = kernels.int8_linear_rows(hd, q.to(DEV), s.to(DEV), kernels.EPI_SILU_MUL)
        assert torch.equal(hd.cpu(), kernels.rmsnorm(x.to(DEV), w.to(DEV), 1e-6).cpu())
        assert rel_l2(y.cpu(), plain.cpu()) < 5e-3


def _qkv_case(t, heads, kv_heads, hidden, seed, gather):
    dim = 128
    n = (heads + 2 * kv_heads) * dim
    q, s = _weights(n, hidden, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    if gather:
        table = _bf16((997, hidden), seed=seed + 2, std=0.02)  # an embedding table
        ids = torch.randint(0, 997, (t,), generator=g)
        x = table[ids]
    else:
        table, ids = None, None
        x = _bf16((t, hidden), seed=seed + 2)
    w_in = _norm_w(hidden, seed + 3)
    qw, kw = _norm_w(dim, seed + 4), _norm_w(dim, seed + 5)
    cos_t, sin_t = ol.rope_tables(dim, 4096, 1e6)
    pos = torch.randint(0, 4096, (t,), generator=g)
    nslots = 3 * t + 16
    slots = torch.randperm(nslots, generator=g)[:t]
    return q, s, table, ids, x, w_in, qw, kw, cos_t, sin_t, pos, nslots, slots


@pytest.mark.parametrize("t,heads,kv_heads,hidden,gather", [
    (64, 16, 8, 1024, False),
    (64, 16, 8, 1024, True),
    (1, 16, 8, 1024, True),
    (19, 32, 8, 4096, False),
    (130, 8, 8, 512, False),
    (5, 16, 4, 2048, True),
])
def test_qkv_rope_cache_rows(t, heads, kv_heads, hidden, gather):
    dim = 128
    q, s, table, ids, x, w_in, qw, kw, cos_t, sin_t, pos, nslots, slots = _qkv_case(t, heads, kv_heads, hidden,
                                                                                   seed=t + heads, gather=gather)
    kc = torch.zeros(nslots, kv_heads, dim, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    resid = torch.full((t, hidden), 7.0, dtype=torch.bfloat16, device=DEV) if gather else None
    src = (table if gather else x).to(DEV)
    qo = kernels.qkv_rope_cache_rows(
        src, q.to(DEV), s.to(DEV), heads, kv_heads, dim, qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV), cos_t.to(DEV),
        sin_t.to(DEV), slots.to(DEV), kc, vc, norm_w=w_in.to(DEV), eps=1e-6,
        gather=ids.to(DEV) if gather else None, x_copy=resid,
    )
    if gather:
        assert torch.equal(resid.cpu(), x)  # the embedding rows, bit for bit
    h = ol.rms_norm(x, w_in, 1e-6)
    qkv = oi.int8_linear(h, q, s)
    qr, kr, vr = qkv.split([heads * dim, kv_heads * dim, kv_heads * dim], dim=-1)
    qn = ol.rms_norm(qr.reshape(t, heads, dim), qw, 1e-6)
    kn = ol.rms_norm(kr.reshape(t, kv_heads, dim), kw, 1e-6)
    qref, kref = ol.apply_rope(qn, kn, cos_t[pos], sin_t[pos])
    assert rel_l2(qo.cpu(), qref) < 1e-2
    kcc, vcc = kc.cpu(), vc.cpu()
    assert rel_l2(kcc[slots], kref) < 1e-2
    assert rel_l2(vcc[slots], vr.reshape(t, kv_heads, dim)) < 1e-2
    untouched = torch.ones(nslots, dtype=torch.bool)
    untouched[slots] = False
    assert torch.all(kcc[untouched] == 0) and torch.all(vcc[untouched] == 0)


def test_qkv_rope_cache_rows_skips_negative_slots():
    t, heads, kv_heads, hidden, dim = 9, 16, 8, 1024, 128
    q, s, _, _, x, w_in, qw, kw, cos_t, sin_t, pos, nslots, slots = _qkv_case(t, heads, kv_heads, hidden, 4, False)
    slots = slots.clone()
    slots[::2] = -1
    kc = torch.zeros(nslots, kv_heads, dim, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    kernels.qkv_rope_cache_rows(
        x.to(DEV), q.to(DEV), s.to(DEV), heads, kv_heads, dim, qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV),
        cos_t.to(DEV), sin_t.to(DEV), slots.to(DEV), kc, vc, norm_w=w_in.to(DEV), eps=1e-6,
    )
    written = slots[slots >= 0]
    assert int((kc.cpu().abs().sum((1, 2)) > 0).sum()) == written.numel()
    assert torch.all(kc.cpu()[written].abs().sum((1, 2)) > 0)


def _lm_case(rows, vocab, k, seed):
    hidden = _bf16((rows + 3, k), seed)
    w = _bf16((vocab, k), seed + 1, std=0.02)
    nw = _norm_w(k, seed + 2)
    sel = torch.randperm(rows + 3, generator=torch.Generator().manual_seed(seed + 3))[:rows]
    return hidden, w, nw, sel


def _check_greedy(got, logits_bf16):
    """got == argmax of the bf16 logits, except where the two best are within one bf16 step."""
    ref = logits_bf16.float().argmax(-1)
    best = logits_bf16.float().max(-1).values
    pick = logits_bf16.float().gather(1, got.view(-1, 1)).flatten()
    step = best.abs() * 2.0**-7
    ok = (got == ref) | (best - pick <= step)
    assert bool(ok.all()), (got[~ok], ref[~ok])
    return int((got == ref).sum())


# (64, 151936, 1024): the decode step; up to 64 rows (16 at k = 4096) stream the weight with the rows
# in LDS. More rows take the GEMM route: 65 rows (a chunked-prefill step's samples), 130 rows, and
# 200 rows at an 8B-sized hidden width.
@pytest.mark.parametrize("rows,vocab,k", [(64, 151936, 1024), (1, 32771, 1024), (17, 5000, 256), (40, 9000, 4096),
                                          (65, 151936, 1024), (130, 9000, 1024), (200, 12000, 4096)])
def test_lm_head_argmax(rows, vocab, k):
    hidden, w, nw, sel = _lm_case(rows, vocab, k, seed=rows + vocab % 97)
    got = kernels.lm_head_argmax(hidden.to(DEV), sel.to(DEV), nw.to(DEV), 1e-6, w.to(DEV)).cpu()
    h = ol.rms_norm(hidden[sel], nw, 1e-6)
    logits = (h.double() @ w.double().T).to(torch.bfloat16)  # bf16 logits as the reference holds them
    exact = _check_greedy(got, logits)
    assert exact >= rows - max(1, rows // 16)
    # prenormed rows give the same ids
    got2 = kernels.lm_head_argmax(h.to(DEV), torch.arange(rows).to(DEV), nw.to(DEV), 1e-6, w.to(DEV),
                                  prenormed=True).cpu()
    assert torch.equal(got, got2)


# Streaming route: 1..64 rows per launch (16 at k = 4096; 70 rows at k = 96 take two launches);
# GEMM route: more rows at k % 64 == 0.
@pytest.mark.parametrize("rows,vocab,k", [(64, 151936, 1024), (5, 4099, 1024), (70, 3000, 96), (40, 9000, 4096),
                                          (65, 20000, 1024), (200, 12000, 4096)])
def test_lm_head_logits(rows, vocab, k):
    """msa_lm_head_logits: each logit within one bf16 step (plus the float32 accumulation bound
    2^-20 sum|h w|, which matters only where the sum cancels to near zero) of the float64 product of
    the same bf16 operands rounded to bf16 (the reference's bf16 logits), rel-L2 against them 1e-3;
    the argmax of the logits is exactly the id of msa_lm_head_argmax (the same products); prenormed
    rows give the same logits."""
    hidden, w, nw, sel = _lm_case(rows, vocab, k, seed=rows + vocab % 89)
    hd, wd, nwd, seld = hidden.to(DEV), w.to(DEV), nw.to(DEV), sel.to(DEV)
    got = kernels.lm_head_logits(hd, seld, nwd, 1e-6, wd).cpu()
    assert got.shape == (rows, vocab) and got.dtype == torch.float32
    h = ol.rms_norm(hidden[sel], nw, 1e-6)
    ref = (h.double() @ w.double().T).to(torch.bfloat16).float()
    assert torch.equal(got, got.to(torch.bfloat16).float())  # every value is a bf16 value
    acc_err = (h.double().abs() @ w.double().abs().T).float() * 2.0**-20
    assert bool(((got - ref).abs() <= (ref.abs() + acc_err) * 2.0**-7 + acc_err).all())
    assert rel_l2(got, ref) < 1e-3
    ids = kernels.lm_head_argmax(hd, seld, nwd, 1e-6, wd).cpu()
    assert torch.equal(got.argmax(-1), ids)
    got2 = kernels.lm_head_logits(h.to(DEV), torch.arange(rows).to(DEV), None, 0.0, wd, prenormed=True).cpu()
    assert torch.equal(got, got2)


def test_lm_head_logits_row_stride_and_clamped_rows():
    """Through the C ABI: an output row stride above vocab leaves the padding untouched; row
    indices outside [0, hidden_rows) are clamped (memory safety), as in msa_lm_head_argmax."""
    from miniserve_amd import _native

    rows, vocab, k, ld = 6, 1000, 256, 1031
    hidden, w, nw, _ = _lm_case(rows, vocab, k, seed=3)
    sel = torch.tensor([0, 8, -4, 2, 100, 5])
    out = torch.full((rows, ld), 7.0, device=DEV)
    hd, wd, nwd, seld = hidden.to(DEV), w.to(DEV), nw.to(DEV), sel.to(DEV)
    _native.call("msa_lm_head_logits", hd.data_ptr(), k, hidden.shape[0], seld.data_ptr(), rows, k, nwd.data_ptr(),
                 1e-6, wd.data_ptr(), vocab, out.data_ptr(), ld, None, 0, torch.cuda.current_stream().cuda_stream)
    got = out.cpu()
    assert bool((got[:, vocab:] == 7.0).all())
    clamped = sel.clamp(0, hidden.shape[0] - 1)
    want = kernels.lm_head_logits(hd, clamped.to(DEV), nwd, 1e-6, wd).cpu()
    assert torch.equal(got[:, :vocab], want)


@pytest.mark.parametrize("rows", [8, 100])  # the streaming route and the GEMM route
def test_lm_head_argmax_first_index_wins_ties(rows):
    vocab, k = 20000, 1024
    hidden, w, nw, sel = _lm_case(rows, vocab, k, seed=5)
    h = ol.rms_norm(hidden[sel], nw, 1e-6)
    # plant the same winning row at three vocabulary positions, spread over row blocks and tiles
    for r in range(rows):
        target = (h[r].float() * 0.5).to(torch.bfloat16)
        for v in (101 + 13 * r, 6000 + r, 19999 - r):
            w[v] = target
    got = kernels.lm_head_argmax(hidden.to(DEV), sel.to(DEV), nw.to(DEV), 1e-6, w.to(DEV)).cpu()
    assert got.tolist() == [101 + 13 * r for r in range(rows)]
