"""Pins the verification oracle (oracle/rejection.py) on the reference's own cases
(tests/unit/test_sampling.py:73-126): greedy acceptance of the matching prefix with the target's
correction or bonus token, and rejection sampling that reproduces the target distribution
exactly (chi-square, p = 0.001) for a deterministic proposer and for a random draft model."""

from __future__ import annotations

import torch
from test_oracle_sampler import CHI2_DF4_P001, chi_square

from oracle import rejection as orj


def test_verify_greedy_accepts_the_matching_prefix() -> None:
    target = torch.full((1, 4, 10), -5.0)
    for pos, tok in enumerate([4, 2, 9, 1]):
        target[0, pos, tok] = 5.0
    acc, nxt = orj.verify_greedy(target, torch.tensor([[4, 2, 7]]), torch.tensor([3]))
    assert (int(acc[0]), int(nxt[0])) == (2, 9)
    acc, nxt = orj.verify_greedy(target, torch.tensor([[4, 2, 9]]), torch.tensor([3]))
    assert (int(acc[0]), int(nxt[0])) == (3, 1)
    acc, nxt = orj.verify_greedy(target, torch.tensor([[4, 2, 9]]), torch.tensor([1]))  # one real draft
    assert (int(acc[0]), int(nxt[0])) == (1, 2)


def test_rejection_sampling_keeps_the_target_distribution() -> None:
    g = torch.Generator().manual_seed(0)
    b, v = 20_000, 5
    p = torch.tensor([[0.1, 0.4, 0.2, 0.25, 0.05], [0.3, 0.1, 0.1, 0.2, 0.3]])
    target = p.unsqueeze(0).expand(b, 2, v).contiguous()
    drafts = torch.full((b, 1), 3)
    acc, nxt = orj.verify_sampled(target, drafts, torch.ones(b, dtype=torch.long), None, torch.rand(b, 1, generator=g),
                                  torch.empty(b, v).exponential_(generator=g))
    first = torch.where(acc == 1, drafts[:, 0], nxt)
    assert chi_square(torch.bincount(first, minlength=v).double(), p[0].double()) < CHI2_DF4_P001
    second = nxt[acc == 1]
    assert chi_square(torch.bincount(second, minlength=v).double(), p[1].double()) < CHI2_DF4_P001
    q = torch.tensor([0.3, 0.1, 0.3, 0.1, 0.2])
    drafts = torch.multinomial(q, b, replacement=True, generator=g).unsqueeze(1)
    acc, nxt = orj.verify_sampled(target, drafts, torch.ones(b, dtype=torch.long), q.expand(b, 1, v).contiguous(),
                                  torch.rand(b, 1, generator=g), torch.empty(b, v).exponential_(generator=g))
    first = torch.where(acc == 1, drafts[:, 0], nxt)
    assert chi_square(torch.bincount(first, minlength=v).double(), p[0].double()) < CHI2_DF4_P001
