"""Oracle: int8 weight-only quantization (test infrastructure only).

Follows quant/int8.py of the reference:
  * ``quantize_int8``  <- ``Int8Linear.__init__``  quant/int8.py:25-33
  * ``dequantize``     <- the first line of ``Int8Linear.forward``  quant/int8.py:36
  * ``int8_linear``    <- ``Int8Linear.forward``  quant/int8.py:35-37
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor


def quantize_int8(weight: Tensor) -> tuple[Tensor, Tensor]:
    """Per-output-row symmetric absmax quantization (quant/int8.py:27-32).

    scale32 = max|w_row| (clamped to >= 1e-8) / 127 in float32 (true division on the CPU),
    q = round_half_even(w / scale32) clamped to [-127, 127] as int8, and the stored scale is
    scale32 rounded to the weight's dtype (bf16 for the model).
    """
    w = weight.detach().float()
    scale = w.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    q = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return q, scale.to(weight.dtype)


def dequantize(q: Tensor, scale: Tensor, dtype: torch.dtype) -> Tensor:
    """The whole-matrix dequantization the reference runs on every call (quant/int8.py:36)."""
    return q.to(dtype) * scale.to(dtype).unsqueeze(1)


def int8_linear(x: Tensor, q: Tensor, scale: Tensor) -> Tensor:
    """y = x @ bf16(q * s)^T in x's dtype (quant/int8.py:35-37)."""
    return F.linear(x, dequantize(q, scale, x.dtype))
