"""Logits to tokens (reference: src/miniserve/runner/sampler.py).

Only greedy decoding is on the hot path (sampler.py:59): ``argmax`` over the float32 logits,
first index among equal maxima, staying on the GPU so that the caller syncs once per step.
"""

from __future__ import annotations

from typing import Any

from torch import Tensor


def sample(logits: Tensor, params: list[Any] | None = None, generators: list[Any] | None = None) -> Tensor:
    """logits [R, vocab] -> token ids [R]. Non-greedy sampling parameters are not supported."""
    if params is not None:
        for p in params:
            if not getattr(p, "greedy", True):
                raise NotImplementedError("only greedy sampling is implemented on the MI355X path")
    return logits.argmax(dim=-1)
