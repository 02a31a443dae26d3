"""Pins the sampling oracle (oracle/sampler.py) before it judges the HIP sampler.

* The reference's own unit cases (tests/unit/test_sampling.py:22-70): greedy is argmax; top_k=1
  and a tiny top_p reduce to greedy; the exact masks of [1, 4, 3, 2, 0] for k=2 and for p=0.8;
  the sampled distribution matches the softmax (chi-square); temperature sharpens / flattens.
* Brute force in float64 on small vocabularies: keep the k largest values (ties with the k-th
  kept), then drop the smallest kept values while their cumulative probability stays <= 1 - p,
  never the largest -- compared mask for mask wherever no cumulative sum lies within 1e-6 of the
  cut (ties in the sort order make those undecidable).
* A planted mistake (top-p cut on the descending order) is caught by the brute force.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampler as osm

CHI2_DF4_P001 = 18.47


def chi_square(counts: torch.Tensor, probs: torch.Tensor) -> float:
    expected = probs * counts.sum()
    return float(((counts - expected) ** 2 / expected).sum())


def test_reference_masks() -> None:
    logits = torch.tensor([[1.0, 4.0, 3.0, 2.0, 0.0]])
    kept = osm.apply_top_k_top_p(logits, torch.tensor([2]), torch.tensor([1.0])) > float("-inf")
    assert kept.tolist() == [[False, True, True, False, False]]
    kept = osm.apply_top_k_top_p(logits, torch.tensor([5]), torch.tensor([0.8])) > float("-inf")
    assert kept.tolist() == [[False, True, True, False, False]]


def test_greedy_top_k_1_and_tiny_top_p() -> None:
    logits = torch.randn(4, 100, generator=torch.Generator().manual_seed(0))
    noise = torch.empty(4, 100).exponential_(generator=torch.Generator().manual_seed(1))
    ones = torch.ones(4)
    greedy = torch.tensor([True, False, False, False])
    k = torch.tensor([100, 1, 100, 1])
    p = torch.tensor([1.0, 1.0, 1e-6, 1e-6])
    assert torch.equal(osm.sample(logits, ones, k, p, greedy, noise), logits.argmax(-1))


def brute_force_cut(z: np.ndarray, k: int, p: float, tol: float = 1e-6) -> tuple[np.ndarray, np.ndarray]:
    """float64 kept mask of one row, and the tokens whose cumulative probability lies within
    ``tol`` of the top-p cut (their side of it depends on summation rounding), in vocab order."""
    v = len(z)
    order = np.argsort(z, kind="stable")  # ascending
    zs = z[order]
    kth = zs[v - k] if 0 < k < v else zs[0]
    keep = zs >= kth
    e = np.where(keep, np.exp(zs - zs.max()), 0.0)
    cum = np.cumsum(e / e.sum())
    near = keep & (np.abs(cum - (1.0 - p)) <= tol) if p < 1.0 else np.zeros(v, dtype=bool)
    drop = cum <= 1.0 - p
    drop[-1] = False
    keep &= ~drop
    mask = np.zeros(v, dtype=bool)
    mask[order] = keep
    boundary = np.zeros(v, dtype=bool)
    boundary[order] = near
    return mask, boundary


def brute_force_mask(z: np.ndarray, k: int, p: float) -> tuple[np.ndarray, bool]:
    """float64 kept mask of one row and whether the top-p cut is decidable (no cumulative sum
    within 1e-6 of 1 - p)."""
    mask, boundary = brute_force_cut(z, k, p)
    return mask, not bool(boundary.any())


@pytest.mark.parametrize("seed", range(6))
def test_masks_against_float64_brute_force(seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    rows, vocab = 64, 37
    logits = torch.randn(rows, vocab, generator=g, dtype=torch.float64) * 2
    k = torch.randint(1, vocab + 1, (rows,), generator=g)
    p = torch.rand(rows, generator=g, dtype=torch.float64) * 0.9 + 0.05
    got = osm.apply_top_k_top_p(logits, k, p) > float("-inf")
    checked = 0
    for r in range(rows):
        mask, ok = brute_force_mask(logits[r].numpy(), int(k[r]), float(p[r]))
        if ok:
            assert np.array_equal(got[r].numpy(), mask), r
            checked += 1
    assert checked >= rows // 2


def test_planted_descending_cut_is_caught() -> None:
    """A restatement that accumulates the nucleus from the largest value down drops different
    tokens: the brute force tells them apart."""
    logits = torch.tensor([[0.0, 1.0, 2.0, 3.0, 4.0, 5.0]], dtype=torch.float64)
    mask, ok = brute_force_mask(logits[0].numpy(), 6, 0.5)
    assert ok
    desc = logits[0].sort(descending=True)
    cum = desc.values.softmax(-1).cumsum(-1)
    wrong = torch.zeros(6, dtype=torch.bool)
    wrong[desc.indices[cum <= 0.5]] = True  # keeps only what lies strictly inside p
    assert not np.array_equal(wrong.numpy(), mask)
    got = osm.apply_top_k_top_p(logits, torch.tensor([6]), torch.tensor([0.5], dtype=torch.float64)) > float("-inf")
    assert np.array_equal(got[0].numpy(), mask)


def test_sampling_matches_the_softmax_distribution() -> None:
    g = torch.Generator().manual_seed(0)
    rows = 50_000
    logits = torch.tensor([[0.5, 1.5, -1.0, 0.0, 1.0]]).repeat(rows, 1)
    noise = torch.empty(rows, 5).exponential_(generator=g)
    tokens = osm.sample(logits, torch.ones(rows), None, None, torch.zeros(rows, dtype=torch.bool), noise)
    counts = torch.bincount(tokens, minlength=5).double()
    assert chi_square(counts, logits[0].double().softmax(-1)) < CHI2_DF4_P001


def test_temperature_changes_the_distribution() -> None:
    logits = torch.tensor([[2.0, 1.0, 0.0]])
    sharp = osm.compute_probs(logits, torch.tensor([0.5]), None, None)
    flat = osm.compute_probs(logits, torch.tensor([2.0]), None, None)
    assert sharp[0, 0] > logits.softmax(-1)[0, 0] > flat[0, 0]
