"""Oracle: the ops that border the linears and attention (test infrastructure only).

Follows model/layers.py of the reference:
  * ``rms_norm``       <- ``RMSNorm.forward``            model/layers.py:18-22
  * ``rope_tables``    <- ``RotaryEmbedding.build``      model/layers.py:43-50
  * ``rotate_half``    <- ``rotate_half``                model/layers.py:56-58
  * ``apply_rope``     <- ``apply_rope``                 model/layers.py:61-65
  * ``swiglu``         <- ``SwiGLU.forward``             model/layers.py:76-79
"""

from __future__ import annotations

from collections.abc import Callable

import torch
import torch.nn.functional as F
from torch import Tensor


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """float32 normalize, cast back to x's dtype, THEN multiply by the weight (layers.py:19-22)."""
    dtype = x.dtype
    x32 = x.to(torch.float32)
    x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return weight * x32.to(dtype)


def rope_tables(head_dim: int, max_positions: int, theta: float) -> tuple[Tensor, Tensor]:
    """float32 cos/sin tables ``[max_positions, head_dim]`` (layers.py:43-50)."""
    exponents = torch.arange(0, head_dim, 2, dtype=torch.int64).float()
    inv_freq = 1.0 / (theta ** (exponents / head_dim))
    t = torch.arange(max_positions, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: Tensor) -> Tensor:
    """Dimension i pairs with i + head_dim/2 (layers.py:56-58)."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """cos/sin ``[T, head_dim]`` are cast to q's dtype before use (layers.py:61-65)."""
    cos = cos.unsqueeze(1).to(q.dtype)
    sin = sin.unsqueeze(1).to(q.dtype)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def swiglu(x: Tensor, gate_up: Callable[[Tensor], Tensor], down: Callable[[Tensor], Tensor]) -> Tensor:
    """down(silu(gate) * up) with gate/up from one fused projection, gate rows first (layers.py:76-79)."""
    gate, up = gate_up(x).chunk(2, dim=-1)
    return down(F.silu(gate) * up)
