"""Verify speculative drafts so that the output distribution is exactly the target model's
(reference: src/miniserve/spec/rejection.py), on the HIP kernels.

Same functions, signatures and semantics as the reference: ``verify_greedy`` accepts drafts
while they equal the target's own argmax and returns the target's pick after the run (a
correction or the bonus token); ``verify_sampled`` accepts draft d_i with probability
min(1, p_i(d_i) / q_i(d_i)) (q one-hot for a deterministic proposer) and samples the replacement
from normalize(max(0, p - q)) -- or the bonus token from p -- by the exponential race on the
caller's noise. The per-position argmax runs on the sampling kernel (first index on ties, as
``argmax``); acceptance and the residual sample run in one kernel per call, one workgroup per
sequence, without materializing the residual distribution.
"""

from __future__ import annotations

import torch
from torch import Tensor

from miniserve_amd import kernels


def verify_greedy(target_logits: Tensor, drafts: Tensor, num_drafts: Tensor) -> tuple[Tensor, Tensor]:
    """target_logits [B, K+1, V], drafts [B, K], num_drafts [B] -> (accepted [B], next_token [B])
    (spec/rejection.py:27-40)."""
    b, k1, v = target_logits.shape
    rows = target_logits.reshape(b * k1, v).float().contiguous()
    greedy = torch.ones(b * k1, dtype=torch.uint8, device=rows.device)
    target = kernels.sample_ids(rows, None, None, None, greedy, None).view(b, k1)
    return kernels.verify_greedy_ids(target, drafts.long(), num_drafts.long())


def verify_sampled(
    target_probs: Tensor,
    drafts: Tensor,
    num_drafts: Tensor,
    draft_probs: Tensor | None,
    uniform: Tensor,
    noise: Tensor,
) -> tuple[Tensor, Tensor]:
    """Rejection sampling (spec/rejection.py:43-79): target_probs [B, K+1, V]; drafts [B, K];
    num_drafts [B]; draft_probs [B, K, V] or None; uniform [B, K] ~ U(0,1); noise [B, V] ~ Exp(1)."""
    return kernels.verify_sampled(target_probs, drafts.long(), num_drafts.long(), draft_probs, uniform, noise)
