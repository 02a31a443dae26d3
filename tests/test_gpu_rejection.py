"""GPU parity of the speculative-decoding verification kernels against the verification oracle
on the same probabilities, uniforms and noise; the reference's own cases on the GPU.

Bars: accepted counts identical; next tokens identical wherever the best two scores of the
sampled distribution differ by more than 1e-4 relative; greedy verification exact."""

from __future__ import annotations

import pytest
import torch
from test_oracle_sampler import CHI2_DF4_P001, chi_square

from miniserve_amd.spec import rejection as hrj
from oracle import rejection as orj

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_verify_greedy_reference_case_and_random():
    target = torch.full((1, 4, 10), -5.0)
    for pos, tok in enumerate([4, 2, 9, 1]):
        target[0, pos, tok] = 5.0
    acc, nxt = hrj.verify_greedy(target.to(DEV), torch.tensor([[4, 2, 7]], device=DEV), torch.tensor([3], device=DEV))
    assert (int(acc[0]), int(nxt[0])) == (2, 9)
    g = torch.Generator().manual_seed(1)
    b, k, v = 40, 6, 5000
    logits = torch.randn(b, k + 1, v, generator=g)
    picks = logits.argmax(-1)
    drafts = picks[:, :k].clone()
    cut = torch.randint(0, k + 1, (b,), generator=g)
    for i in range(b):  # corrupt one draft at a random position (or none)
        if int(cut[i]) < k:
            drafts[i, int(cut[i])] = (drafts[i, int(cut[i])] + 1) % v
    nd = torch.randint(0, k + 1, (b,), generator=g)
    acc, nxt = hrj.verify_greedy(logits.to(DEV), drafts.to(DEV), nd.to(DEV))
    racc, rnxt = orj.verify_greedy(logits, drafts, nd)
    assert torch.equal(acc.cpu(), racc) and torch.equal(nxt.cpu(), rnxt)


@pytest.mark.parametrize("with_q", [False, True])
def test_verify_sampled_matches_the_oracle(with_q):
    g = torch.Generator().manual_seed(2 + with_q)
    b, k, v = 48, 5, 151936
    tp = torch.softmax(torch.randn(b, k + 1, v, generator=g) * 2, dim=-1)
    drafts = torch.randint(0, v, (b, k), generator=g)
    drafts[::2] = tp[::2, :k].argmax(-1)  # likely accepted drafts on half the rows
    nd = torch.randint(1, k + 1, (b,), generator=g)
    q = torch.softmax(torch.randn(b, k, v, generator=g) * 2, dim=-1) if with_q else None
    u = torch.rand(b, k, generator=g)
    noise = torch.empty(b, v).exponential_(generator=g)
    acc, nxt = hrj.verify_sampled(tp.to(DEV), drafts.to(DEV), nd.to(DEV), q.to(DEV) if q is not None else None,
                                  u.to(DEV), noise.to(DEV))
    racc, rnxt = orj.verify_sampled(tp, drafts, nd, q, u, noise)
    assert torch.equal(acc.cpu(), racc)
    checked = 0
    for i in range(b):
        a = int(racc[i])
        p = tp[i, a]
        if a < int(nd[i]):
            at = min(a, k - 1)
            dist = (p - q[i, at]).clamp(min=0) if q is not None else p.clone().index_fill_(0, drafts[i, at:at + 1], 0.0)
        else:
            dist = p
        s = (dist / dist.sum()) / noise[i]
        top2 = s.double().topk(2).values
        if float(top2[0] - top2[1]) > 1e-4 * float(top2[0]):
            assert int(nxt[i]) == int(rnxt[i]), i
            checked += 1
    assert checked >= b * 3 // 4


def test_rejection_sampling_keeps_the_target_distribution_on_gpu():
    g = torch.Generator(device=DEV).manual_seed(0)
    b, v = 100_000, 5
    p = torch.tensor([[0.1, 0.4, 0.2, 0.25, 0.05], [0.3, 0.1, 0.1, 0.2, 0.3]], device=DEV)
    target = p.unsqueeze(0).expand(b, 2, v).contiguous()
    drafts = torch.full((b, 1), 3, device=DEV)
    acc, nxt = hrj.verify_sampled(target, drafts, torch.ones(b, dtype=torch.long, device=DEV), None,
                                  torch.rand(b, 1, generator=g, device=DEV),
                                  torch.empty(b, v, device=DEV).exponential_(generator=g))
    first = torch.where(acc == 1, drafts[:, 0], nxt).cpu()
    assert chi_square(torch.bincount(first, minlength=v).double(), p[0].cpu().double()) < CHI2_DF4_P001
    second = nxt[acc == 1].cpu()
    assert chi_square(torch.bincount(second, minlength=v).double(), p[1].cpu().double()) < CHI2_DF4_P001


def test_verify_sampled_converts_its_inputs():
    """float64 probabilities, uniforms and noise and non-contiguous int64 drafts: every operand the
    wrapper converts stays alive until the kernel has read it, so the result equals the call on
    float32 contiguous copies (and the oracle's on the same values)."""
    g = torch.Generator().manual_seed(7)
    b, k, v = 33, 4, 30000
    tp = torch.softmax(torch.randn(b, k + 1, v, generator=g, dtype=torch.float64) * 2, dim=-1)
    q = torch.softmax(torch.randn(b, k, v, generator=g, dtype=torch.float64) * 2, dim=-1)
    drafts_t = torch.randint(0, v, (k, b), generator=g)
    drafts_t[:, ::2] = tp[::2, :k].argmax(-1).T
    drafts = drafts_t.T  # [b, k], not contiguous
    assert not drafts.is_contiguous()
    nd = torch.randint(1, k + 1, (2 * b,), generator=g)[::2]  # strided too
    u = torch.rand(b, k, generator=g, dtype=torch.float64)
    noise = torch.empty(b, v, dtype=torch.float64).exponential_(generator=g)
    acc, nxt = hrj.verify_sampled(tp.to(DEV), drafts.to(DEV), nd.to(DEV), q.to(DEV), u.to(DEV), noise.to(DEV))
    tp32, q32, u32, n32 = tp.float(), q.float(), u.float(), noise.float()
    acc2, nxt2 = hrj.verify_sampled(tp32.to(DEV), drafts.contiguous().to(DEV), nd.contiguous().to(DEV), q32.to(DEV),
                                    u32.to(DEV), n32.to(DEV))
    assert torch.equal(acc.cpu(), acc2.cpu()) and torch.equal(nxt.cpu(), nxt2.cpu())
    racc, _ = orj.verify_sampled(tp32, drafts.contiguous(), nd.contiguous(), q32, u32, n32)
    assert torch.equal(acc.cpu(), racc)
