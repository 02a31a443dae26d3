"""The building blocks of a Qwen3 layer (reference: src/miniserve/model/layers.py).

RMSNorm runs as a HIP kernel; RoPE is applied inside the fused q/k-norm + RoPE + KV-write kernels
of ``Qwen3Attention`` from the float32 tables built here; SwiGLU with int8 projections runs
silu(gate) * up in the epilogue of the gate_up kernel and the residual add in the epilogue of the
down kernel.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from miniserve_amd import kernels
from miniserve_amd.quant.int8 import Int8Linear


class RMSNorm(nn.Module):
    """x / rms(x) * weight, normalized in float32 and cast to bf16 before the weight multiply
    (layers.py:10-22)."""

    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return kernels.rmsnorm(x, self.weight, self.eps)


class RotaryEmbedding(nn.Module):
    """Precomputed float32 cos/sin tables indexed by each token's own position (layers.py:25-53).

    Dimension i pairs with i + head_dim/2. The tables are built once with the reference's float32
    formula on the host (so they match it bit for bit) and kept on the device.
    """

    cos: Tensor
    sin: Tensor

    def __init__(self, head_dim: int, max_positions: int, theta: float) -> None:
        super().__init__()
        self.head_dim, self.max_positions, self.theta = head_dim, max_positions, theta
        self.register_buffer("cos", torch.empty(0), persistent=False)
        self.register_buffer("sin", torch.empty(0), persistent=False)

    def build(self, device: torch.device) -> None:
        exponents = torch.arange(0, self.head_dim, 2, dtype=torch.int64).float()
        inv_freq = 1.0 / (self.theta ** (exponents / self.head_dim))
        t = torch.arange(self.max_positions, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos = emb.cos().to(device)
        self.sin = emb.sin().to(device)

    def forward(self, positions: Tensor) -> tuple[Tensor, Tensor]:
        return self.cos[positions], self.sin[positions]


class SwiGLU(nn.Module):
    """down(silu(gate(x)) * up(x)), gate and up fused into one projection (layers.py:68-79)."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.gate_up_proj: nn.Module = nn.Linear(hidden_size, 2 * intermediate_size, bias=False)
        self.down_proj: nn.Module = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: Tensor, residual: Tensor | None = None) -> Tensor:
        """Returns down(...) or, when ``residual`` is given, residual + down(...)."""
        if isinstance(self.gate_up_proj, Int8Linear):
            act = self.gate_up_proj(x, epilogue=kernels.EPI_SILU_MUL)
        else:
            gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
            act = F.silu(gate) * up
        if isinstance(self.down_proj, Int8Linear):
            if residual is None:
                return self.down_proj(act)
            return self.down_proj(act, epilogue=kernels.EPI_RESIDUAL, residual=residual)
        out: Tensor = self.down_proj(act)
        return out if residual is None else residual + out
