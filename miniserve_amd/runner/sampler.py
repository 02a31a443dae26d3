"""Logits to tokens: greedy, temperature, top-k and top-p, batched with per-request settings
(reference: src/miniserve/runner/sampler.py), on the HIP sampling kernel.

Same functions and signatures as the reference. The reference sorts every row of the vocabulary
for top-k / top-p; here one kernel per call finds the k-th largest value and the nucleus cut by
radix selection (no sort, no [R, V] index tensor) and, for ``sample``, runs the exponential race
``argmax(probs / noise)`` in the same pass. The Exp(1) noise is drawn exactly as the reference
draws it (torch's ``exponential_``, a per-row generator for seeded requests), so a seeded request
samples from the same noise.

``params`` entries only need the reference's ``SamplingParams`` attributes: ``temperature``,
``top_k``, ``top_p`` and ``greedy``.
"""

from __future__ import annotations

from typing import Any, Sequence

import torch
from torch import Tensor

from miniserve_amd import kernels
from miniserve_amd.utils import to_device


def apply_top_k_top_p(logits: Tensor, top_k: Tensor, top_p: Tensor) -> Tensor:
    """Set every logit outside a row's top-k and top-p nucleus to -inf (sampler.py:12-27).

    top_k: [R] (vocab size = disabled), top_p: [R] (1.0 = disabled). logits: float32 [R, vocab].
    """
    k = top_k.to(device=logits.device, dtype=torch.int32).contiguous()
    p = top_p.to(device=logits.device, dtype=torch.float32).contiguous()
    return kernels.top_k_top_p_mask(logits.float().contiguous(), k, p)


def _filters(params: Sequence[Any], vocab: int, dev: torch.device) -> tuple[Tensor | None, Tensor | None]:
    if not any(0 < p.top_k < vocab or p.top_p < 1.0 for p in params):
        return None, None
    top_k = to_device([p.top_k if 0 < p.top_k < vocab else vocab for p in params], dev, torch.int32)
    top_p = to_device([p.top_p for p in params], dev, torch.float32)
    return top_k, top_p


def compute_probs(logits: Tensor, params: Sequence[Any]) -> Tensor:
    """Probabilities after temperature, top-k and top-p, each row with its request's settings
    (sampler.py:30-40)."""
    vocab = logits.shape[-1]
    dev = logits.device
    temps = to_device([max(p.temperature, 1e-5) for p in params], dev, torch.float32)
    top_k, top_p = _filters(params, vocab, dev)
    return kernels.sampling_probs(logits.float().contiguous(), temps, top_k, top_p)


def exponential_noise(
    shape: tuple[int, int], generators: Sequence[torch.Generator | None], device: torch.device
) -> Tensor:
    """Exp(1) noise per row; rows with their own generator (a seeded request) use it
    (sampler.py:43-52)."""
    noise = torch.empty(shape, device=device).exponential_()
    for i, g in enumerate(generators):
        if g is not None:
            noise[i].exponential_(generator=g)
    return noise.clamp_(min=torch.finfo(noise.dtype).tiny)


def sample(logits: Tensor, params: Sequence[Any], generators: Sequence[torch.Generator | None]) -> Tensor:
    """logits [R, vocab] -> token ids [R], staying on the GPU (sampler.py:55-69)."""
    logits = logits.float().contiguous()
    dev = logits.device
    rows, vocab = logits.shape
    greedy = to_device([1 if p.greedy else 0 for p in params], dev, torch.uint8)
    if all(p.greedy for p in params):
        return kernels.sample_ids(logits, None, None, None, greedy, None)
    temps = to_device([max(p.temperature, 1e-5) for p in params], dev, torch.float32)
    top_k, top_p = _filters(params, vocab, dev)
    noise = exponential_noise((rows, vocab), generators, dev)
    return kernels.sample_ids(logits, temps, top_k, top_p, greedy, noise)
