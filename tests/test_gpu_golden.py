"""GPU parity of the HIP path against the committed golden fixtures of tests/golden/ (written by
tests/golden/make_golden.py with numpy, float64 brute force and transformers' float64 Qwen3;
nothing here runs the oracle).

Bars: int8 packing bit-exact; slots exact; linears within rel-L2 1e-2 (4e-3 for the single
linear); attention within rel-L2 1e-2; the tiny int8 Qwen3's logits within rel-L2 1e-2 of the
float64 model at every step and greedy ids equal except where the float64 top-2 margin is below
2e-2 (a bf16-rounding tie).
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import numpy as np
import pytest
import torch
from helpers import rel_l2

from miniserve_amd import kernels, workloads
from miniserve_amd.attention import backends as hb
from miniserve_amd.quant.int8 import quantize_int8_
from miniserve_amd.runner.model_runner import ModelRunner, ScheduledChunk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_pack_fixture_on_device():
    g = load("int8_pack.npz")
    w = bf16(g["w_bits"]).to(DEV)
    q, s = kernels.int8_quantize(w)
    assert np.array_equal(q.cpu().numpy(), g["q"])
    assert np.array_equal(bits(s), g["scale_bits"])


def test_linear_fixture_on_device():
    g = load("int8_linear.npz")
    q, s = kernels.int8_quantize(bf16(g["w_bits"]).to(DEV))
    assert np.array_equal(q.cpu().numpy(), g["q"]) and np.array_equal(bits(s), g["scale_bits"])
    x = bf16(g["x_bits"]).to(DEV)
    y = kernels.int8_linear(x, q, s)
    assert y.shape == (5, 24)
    assert rel_l2(y.cpu(), torch.from_numpy(g["y"])) < 4e-3


def test_attention_fixture_on_device():
    g = load("paged_attention.npz")
    kc, vc, q = bf16(g["k_bits"]).to(DEV), bf16(g["v_bits"]).to(DEV), bf16(g["q_bits"]).to(DEV)
    chunks, flat = [], 0
    for (cached, new), row in zip(g["cached_new"].tolist(), g["tables"].tolist(), strict=True):
        chunks.append(hb.SeqChunk(flat, new, cached, [b for b in row if b >= 0]))
        flat += new
    slots = torch.from_numpy(g["slots"]).to(DEV)
    k, v = kc[slots].clone(), vc[slots].clone()  # this step's keys are already in the pool
    k_before, v_before = kc.clone(), vc.clone()
    meta = hb.build_attention_metadata(chunks, slots, 16)
    out = hb.paged_attention(q, k, v, kc, vc, meta, float(g["scale"]))
    assert torch.equal(kc, k_before) and torch.equal(vc, v_before)  # the writes hit exactly these slots
    assert rel_l2(out.cpu(), torch.from_numpy(g["out"])) < 1e-2


def test_qwen3_tiny_fixture_on_device():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    g = load("qwen3_tiny.npz")
    cfg = json.loads(str(g["config"]))
    raw = mg.tiny_model_weights(cfg, int(g["seed"]))
    assert mg.weights_digest(raw) == str(g["digest"]), "the seeded weight generator changed"
    model = workloads.build_model(cfg, {k: bf16(v) for k, v in raw.items()}, DEV, max_positions=256)
    quantize_int8_(model)
    for i, layer in enumerate(model.layers):
        for name in mg.LINEARS:
            mod = layer.get_submodule(name)
            q, s, _ = mg.pack_int8(raw[f"layers.{i}.{name}.weight"])
            assert np.array_equal(mod.qweight.cpu().numpy(), q) and np.array_equal(bits(mod.scale), s)
    runner = ModelRunner(model, DEV)
    runner.allocate_kv_cache(4)
    seqs = [mg.prompt_ids(n, s, cfg["vocab_size"]) for n, s in mg.PROMPTS]
    tables = [[0, 1], [3, 2]]
    starts = [0, 0]
    for step in range(mg.DECODE_STEPS + 1):
        sched = [ScheduledChunk(list(s), st, len(s) - st, t) for s, st, t in zip(seqs, starts, tables, strict=True)]
        inp = runner.prepare(sched)
        logits = runner.forward_logits(inp).cpu()
        assert rel_l2(logits, torch.from_numpy(g["logits"][step])) < 1e-2, step
        ids = runner.forward_greedy(inp).cpu()
        margin = g["top2_margin"][step]
        for a, b, m in zip(ids.tolist(), g["next_ids"][step].tolist(), margin.tolist(), strict=True):
            assert a == b or m < 2e-2, (step, a, b, m)
        starts = [len(s) for s in seqs]
        for s, nxt in zip(seqs, g["next_ids"][step].tolist(), strict=True):
            s.append(int(nxt))  # teacher-forced with the float64 model's greedy ids
