"""GPU parity of the streaming decode linear (gemv_stream.hip), which msa_int8_linear_dec takes for up
to 16 tokens when k is 2048 or 4096 and the weight has at least 384 output units (16-row tiles; for
silu * up, 8 gate + 8 up rows), against the CPU oracle on the same seeded inputs.

The kernel rounds where the reference rounds: weights dequantized to bf16(q * s), the RMSNorm
prologue as bf16(w * bf16(x * r)), float32 accumulation, bf16 outputs. Bars as for the other decode
linears: within rel-L2 2e-3 of the oracle; within bf16 output rounding of the float64 product of the
same bf16 operands; the residual add exact on the kernel's own projection; bit-identical across
calls. Shapes cover the Qwen3-8B-shaped projections (k = 4096: qkv 6144 rows, gate_up 2 x 12288
rows), k = 2048, the smallest eligible weight (384 units) and the largest unit runs, ragged last
units and 1..16 tokens. Every call goes through the C ABI.
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


def _exact_weights(q, s):
    """The dequantized weights bf16(q * s) (quant/int8.py:36) in float64."""
    return (q.to(torch.bfloat16) * s[:, None]).double()


def _exact_norm(x, w, eps):
    x64 = x.double()
    return x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + eps) * w.double()


@pytest.mark.parametrize("m,n,k,with_norm", [
    (16, 6144, 4096, True),   # 8B qkv after input_layernorm: 384 units, two per workgroup
    (1, 6144, 4096, True),
    (7, 6144, 4096, False),
    (16, 6200, 4096, False),  # ragged last unit
    (16, 8192, 2048, True),   # k = 2048
    (3, 12288, 2048, False),  # 768 units: three per workgroup
])
def test_stream_linear(m, n, k, with_norm):
    q, s = _weights(n, k, seed=n + k + m)
    x = _bf16((m, k), seed=m + 11, std=3.0 if with_norm else 1.0)
    w = _norm_w(k, seed=m + 12)
    qd, sd, xd = q.to(DEV), s.to(DEV), x.to(DEV)
    wd = w.to(DEV) if with_norm else None
    y = kernels.int8_linear_dec(xd, qd, sd, norm_w=wd, eps=1e-6)
    y2 = kernels.int8_linear_dec(xd, qd, sd, norm_w=wd, eps=1e-6)
    assert torch.equal(y, y2)  # deterministic
    h = ol.rms_norm(x, w, 1e-6) if with_norm else x
    assert rel_l2(y.cpu(), oi.int8_linear(h, q, s)) < 2e-3
    h64 = _exact_norm(x, w, 1e-6) if with_norm else x.double()
    assert rel_l2(y.cpu(), h64 @ _exact_weights(q, s).T) < (6e-3 if with_norm else 4e-3)
    if with_norm:  # against the norm kernel (the same roundings) followed by the plain product
        plain = kernels.int8_linear_dec(kernels.rmsnorm(xd, wd, 1e-6), qd, sd)
        assert rel_l2(y.cpu(), plain.cpu()) < 2e-3


@pytest.mark.parametrize("m,half,k", [
    (16, 12288, 4096),  # the 8B gate_up: 1536 units, six per workgroup
    (5, 12288, 4096),
    (16, 3100, 4096),   # 388 units, the last one ragged
    (9, 6144, 2048),
])
@pytest.mark.parametrize("with_norm", [True, False])
def test_stream_silu_mul(m, half, k, with_norm):
    n = 2 * half
    q, s = _weights(n, k, seed=m + half + k)
    x = _bf16((m, k), seed=m + 21)
    w = _norm_w(k, seed=m + 22)
    wd = w.to(DEV) if with_norm else None
    y = kernels.int8_linear_dec(x.to(DEV), q.to(DEV), s.to(DEV), kernels.EPI_SILU_MUL, norm_w=wd, eps=1e-6)
    assert y.shape == (m, half)
    h = ol.rms_norm(x, w, 1e-6) if with_norm else x
    gate, up = oi.int8_linear(h, q, s).chunk(2, dim=-1)
    assert rel_l2(y.cpu(), torch.nn.functional.silu(gate) * up) < 2e-3
    h64 = _exact_norm(x, w, 1e-6) if with_norm else x.double()
    g64, u64 = (h64 @ _exact_weights(q, s).T).chunk(2, dim=-1)
    assert rel_l2(y.cpu(), torch.nn.functional.silu(g64) * u64) < 8e-3


@pytest.mark.parametrize("m,n,k", [(16, 6144, 4096), (11, 8192, 2048), (1, 6160, 4096)])
def test_stream_residual_in_place(m, n, k):
    q, s = _weights(n, k, seed=5 * n + k)
    x = _bf16((m, k), seed=m + 31)
    r = _bf16((m, n), seed=m + 32)
    rd = r.to(DEV)
    out = kernels.int8_linear_dec(x.to(DEV), q.to(DEV), s.to(DEV), kernels.EPI_RESIDUAL, residual=rd, out=rd)
    assert out.data_ptr() == rd.data_ptr()
    assert rel_l2(rd.cpu(), r + oi.int8_linear(x, q, s)) < 2e-3
    y = kernels.int8_linear_dec(x.to(DEV), q.to(DEV), s.to(DEV)).cpu()
    assert torch.equal(rd.cpu(), r + y)  # the residual add itself is exact on the kernel's projection


def test_stream_eligibility_boundary():
    """383 units take the row-block decode kernel, 384 the streaming one: both within the bars, on
    the same rows (the first 6128 of the same weight)."""
    k, m = 4096, 12
    q, s = _weights(6144, k, seed=77)
    x = _bf16((m, k), seed=78)
    ref = oi.int8_linear(x, q, s)
    y_stream = kernels.int8_linear_dec(x.to(DEV), q.to(DEV), s.to(DEV)).cpu()
    y_dec = kernels.int8_linear_dec(x.to(DEV), q[:6128].contiguous().to(DEV), s[:6128].contiguous().to(DEV)).cpu()
    assert rel_l2(y_stream, ref) < 2e-3
    assert rel_l2(y_dec, ref[:, :6128]) < 2e-3
    assert rel_l2(y_stream[:, :6128], y_dec) < 2e-3
