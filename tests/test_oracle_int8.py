"""Pins the oracle's int8 pack and linear (reference quant/int8.py:25-37) without the reference.

Checks: an independent numpy restatement bit for bit, the closed-form invariants, exact half-way
ties (round half to even), the all-zero row, bf16 rounding of scales and of q*s, and float64 brute
force for the linear. ``test_mutants_are_caught`` plants plausible mistakes in copies of the
oracle, on the CPU, and shows that these checks reject each of them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from helpers import bf16_bits_rne, rel_l2

from oracle.int8 import dequantize, int8_linear, quantize_int8


def numpy_quantize(w_bf16: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """Independent restatement: IEEE float32 division and np.rint (half to even)."""
    w = w_bf16.float().numpy().astype(np.float32)
    amax = np.abs(w).max(axis=1)
    s32 = (np.maximum(amax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint((w / s32[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    return q, bf16_bits_rne(s32)


def _weights(rows: int, cols: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(rows, cols, generator=g) * 0.02).to(torch.bfloat16)


def _check_all(quant, w: torch.Tensor) -> None:
    q, s = quant(w)
    qn, sn = numpy_quantize(w)
    assert np.array_equal(q.numpy(), qn)
    assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), sn)
    _check_invariants(q, w)


def _check_invariants(q: torch.Tensor, w: torch.Tensor) -> None:
    w32 = w.float()
    amax = w32.abs().amax(dim=1)
    s32 = amax.clamp(min=1e-8) / 127.0
    assert int(q.abs().max()) <= 127
    nz = amax > 0
    assert torch.all(q[nz].abs().amax(dim=1) == 127)
    # float32 division can land within |w/s| * 2^-24 <= 127 * 2^-24 of a tie before rounding.
    err = (w32.double() - q.double() * s32.double()[:, None]).abs()
    assert torch.all(err <= s32.double()[:, None] * (0.5 + 1e-5))


@pytest.mark.parametrize("shape", [(3072, 1024), (96, 64), (7, 48)])
def test_matches_numpy_restatement(shape: tuple[int, int]) -> None:
    _check_all(quantize_int8, _weights(*shape, seed=sum(shape)))


def test_half_way_ties_round_to_even() -> None:
    # amax = 127 makes scale exactly 1.0, so w / s is w itself: every .5 is an exact tie.
    row = torch.tensor([[127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -126.5]], dtype=torch.bfloat16)
    q, s = quantize_int8(row)
    assert q.tolist() == [[127, 2, -2, 4, 0, 0, 2, -126]]
    assert float(s) == 1.0


def test_zero_row_and_clamp() -> None:
    w = torch.zeros(3, 32, dtype=torch.bfloat16)
    w[1, 5] = -3.0
    q, s = quantize_int8(w)
    assert torch.all(q[0] == 0) and torch.all(q[2] == 0)
    assert q[1, 5] == -127
    # scale of a zero row is 1e-8 / 127 rounded to bf16
    expect = bf16_bits_rne(np.array([np.float32(1e-8) / np.float32(127.0)], dtype=np.float32))[0]
    assert int(s[0].view(torch.int16)) & 0xFFFF == int(expect)


def test_dequantize_is_rne_of_exact_product() -> None:
    w = _weights(64, 256, seed=3)
    q, s = quantize_int8(w)
    deq = dequantize(q, s, torch.bfloat16)
    prod = q.float().numpy() * s.float().numpy()[:, None]  # exact in float32 (<= 15 bits)
    assert np.array_equal(deq.view(torch.int16).numpy().view(np.uint16), bf16_bits_rne(prod))


def test_linear_against_float64_brute_force() -> None:
    w = _weights(3072, 1024, seed=1)
    q, s = quantize_int8(w)
    x = torch.randn(16, 1024, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    y = int8_linear(x, q, s)
    assert y.dtype == torch.bfloat16 and y.shape == (16, 3072)
    deq64 = torch.from_numpy(np.array(q.numpy(), dtype=np.float64) * s.double().numpy()[:, None])
    ref = x.double() @ deq64.T
    # bf16 rounding of q*s (<= 2^-9 relative per weight) plus bf16 output rounding.
    assert rel_l2(y, ref) < 4e-3


def test_mutants_are_caught() -> None:
    """Plausible mistakes, planted in copies of the oracle, fail the checks above."""

    def half_away(w):
        w32 = w.float()
        s = w32.abs().amax(dim=1).clamp(min=1e-8) / 127.0
        v = w32 / s[:, None]
        q = (torch.sign(v) * torch.floor(v.abs() + 0.5)).clamp(-127, 127).to(torch.int8)
        return q, s.to(w.dtype)

    def no_clamp_floor(w):
        w32 = w.float()
        s = w32.abs().amax(dim=1) / 127.0
        return torch.round(w32 / s[:, None]).nan_to_num(0).clamp(-127, 127).to(torch.int8), s.to(w.dtype)

    def scale_by_255(w):
        w32 = w.float()
        s = w32.abs().amax(dim=1).clamp(min=1e-8) / 255.0
        return torch.round(w32 / s[:, None]).clamp(-127, 127).to(torch.int8), s.to(w.dtype)

    def truncated_scale(w):
        q, s = quantize_int8(w)
        s32 = w.float().abs().amax(dim=1).clamp(min=1e-8) / 127.0
        bits = (s32.view(torch.int32) >> 16).to(torch.int16)
        return q, bits.view(torch.bfloat16)

    ties = torch.tensor([[127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -126.5]], dtype=torch.bfloat16)
    assert half_away(ties)[0].tolist() != quantize_int8(ties)[0].tolist()
    zero = torch.zeros(2, 16, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        _check_all(no_clamp_floor, zero)
    for mutant in (scale_by_255, truncated_scale):
        with pytest.raises(AssertionError):
            _check_all(mutant, _weights(96, 64, seed=5))


def test_linear_mutant_transposed_scale_is_caught() -> None:
    w = _weights(48, 48, seed=7)
    q, s = quantize_int8(w)
    x = torch.randn(4, 48, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    wrong = F.linear(x, q.to(torch.bfloat16) * s.unsqueeze(0))  # scale along the wrong axis
    deq64 = torch.from_numpy(np.array(q.numpy(), dtype=np.float64) * s.double().numpy()[:, None])
    ref = x.double() @ deq64.T
    assert rel_l2(int8_linear(x, q, s), ref) < 4e-3
    assert rel_l2(wrong, ref) > 0.1
