"""Weight-only INT8 linears (reference: src/miniserve/quant/int8.py).

Same storage as the reference -- ``qweight`` int8 ``[out, in]`` row-major and ``scale`` ``[out]``
in the weight dtype (bf16), with scale = max|w_row| / 127 and q = round_half_even(w / scale) --
but the pack runs as one HIP kernel on the GPU, bit-identical to quant/int8.py:27-32, and the
forward never materializes the dequantized matrix: the HIP kernel dequantizes each weight in
registers to the same bf16(q * s) value and multiplies on MFMA tiles.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from miniserve_amd import kernels


class Int8Linear(nn.Module):
    """Drop-in for quant/int8.py:21-37: ``Int8Linear(weight)``; ``forward(x) -> [..., out]``."""

    qweight: Tensor
    scale: Tensor

    def __init__(self, weight: Tensor) -> None:
        super().__init__()
        if not weight.is_cuda:
            raise RuntimeError("Int8Linear packs on the GPU: move the weight to the MI355X first")
        if weight.dtype != torch.bfloat16:
            raise RuntimeError(f"Int8Linear supports bf16 weights (got {weight.dtype})")
        q, s = kernels.int8_quantize(weight)
        self.register_buffer("qweight", q)
        self.register_buffer("scale", s)
        self.out_features, self.in_features = weight.shape

    def forward(self, x: Tensor, epilogue: int = kernels.EPI_NONE, residual: Tensor | None = None) -> Tensor:
        """y = x @ bf16(qweight * scale)^T; ``epilogue`` fuses SwiGLU's silu(gate) * up or a
        residual add into the same kernel (used by this package's Qwen3 layers)."""
        return kernels.int8_linear(x, self.qweight, self.scale, epilogue, residual)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, int8 per-row"


def quantize_int8_(model: nn.Module) -> int:
    """Swap every decoder-layer linear for Int8Linear in place (quant/int8.py:40-60).

    The embedding / LM head stay bf16. Returns the number of weight bytes saved.
    """
    saved = 0
    for layer in model.layers:  # type: ignore[attr-defined]
        for parent, name in (
            (layer.self_attn, "qkv_proj"),
            (layer.self_attn, "o_proj"),
            (layer.mlp, "gate_up_proj"),
            (layer.mlp, "down_proj"),
        ):
            linear = getattr(parent, name)
            q = Int8Linear(linear.weight)
            saved += linear.weight.numel() * linear.weight.element_size()
            saved -= q.qweight.numel() + q.scale.numel() * q.scale.element_size()
            setattr(parent, name, q)
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return saved
