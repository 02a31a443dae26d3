"""Pins the CPU oracle against the committed golden fixtures of tests/golden/.

The fixtures were written by tests/golden/make_golden.py from computations that share nothing
with the oracle: a numpy restatement of the int8 pack (quant/int8.py:27-32), float64 brute force
for the linear and for paged attention through block tables (attention/backends.py:145-197), and
``transformers.Qwen3ForCausalLM`` in float64 for a tiny int8 Qwen3. A plausible slip in the
oracle -- a transposed scale, a wrong KV head for a query head, an off-by-one block index, a
missing norm -- moves its results far outside these bars.
"""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import numpy as np
import torch
from helpers import rel_l2

from oracle import model as om
from oracle.attention import SeqChunk, build_attention_metadata, context_slots, paged_attention
from oracle.int8 import dequantize, int8_linear, quantize_int8

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def golden_module():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_int8_pack_fixture() -> None:
    g = load("int8_pack.npz")
    q, s = quantize_int8(bf16(g["w_bits"]))
    assert np.array_equal(q.numpy(), g["q"])
    assert np.array_equal(bits(s), g["scale_bits"])
    assert np.array_equal(bits(dequantize(q, s, torch.bfloat16)), g["deq_bits"])


def test_int8_linear_fixture() -> None:
    g = load("int8_linear.npz")
    q, s = quantize_int8(bf16(g["w_bits"]))
    assert np.array_equal(q.numpy(), g["q"]) and np.array_equal(bits(s), g["scale_bits"])
    y = int8_linear(bf16(g["x_bits"]), q, s)
    assert y.shape == (5, 24) and y.dtype == torch.bfloat16
    assert rel_l2(y, torch.from_numpy(g["y"])) < 4e-3
    w = dequantize(q, s, torch.bfloat16).double()  # bf16(q * s), then the product in float64
    y64 = torch.nn.functional.linear(bf16(g["x_bits"]).double(), w)
    torch.testing.assert_close(y64, torch.from_numpy(g["y"]), atol=1e-12, rtol=1e-10)


def _attention_case(g: dict[str, np.ndarray], dtype: torch.dtype):
    kc = bf16(g["k_bits"]).to(dtype)
    vc = bf16(g["v_bits"]).to(dtype)
    q = bf16(g["q_bits"]).to(dtype)
    chunks, flat = [], 0
    for (cached, new), row in zip(g["cached_new"].tolist(), g["tables"].tolist(), strict=True):
        chunks.append(SeqChunk(flat, new, cached, [b for b in row if b >= 0]))
        flat += new
    slots = torch.from_numpy(g["slots"])
    return q, kc, vc, chunks, slots


def test_paged_attention_fixture() -> None:
    g = load("paged_attention.npz")
    for dtype, bar in ((torch.float64, 1e-12), (torch.bfloat16, 1e-2)):
        q, kc, vc, chunks, slots = _attention_case(g, dtype)
        k, v = kc[slots].clone(), vc[slots].clone()  # this step's keys are already in the pool
        meta = build_attention_metadata(chunks, slots, 16)
        out = paged_attention(q, k, v, kc, vc, meta, float(g["scale"]))
        assert rel_l2(out, torch.from_numpy(g["out"])) < bar, dtype


def test_slot_fixture_matches_closed_form() -> None:
    g = load("paged_attention.npz")
    got = []
    for (cached, new), row in zip(g["cached_new"].tolist(), g["tables"].tolist(), strict=True):
        table = torch.tensor([[b for b in row if b >= 0]])
        got.extend(context_slots(table, cached + new, 16)[0, cached:].tolist())
    assert got == g["slots"].tolist()


def test_qwen3_tiny_fixture() -> None:
    mg = golden_module()
    g = load("qwen3_tiny.npz")
    cfg_d = json.loads(str(g["config"]))
    raw = mg.tiny_model_weights(cfg_d, int(g["seed"]))
    assert mg.weights_digest(raw) == str(g["digest"]), "the seeded weight generator changed"
    cfg = om.Config.from_dict(cfg_d)
    w16 = {k: bf16(v) for k, v in raw.items()}
    qw = om.quantize_weights(w16, cfg)
    for key in [k for k in raw if k.endswith("proj.weight")]:  # oracle pack == numpy pack
        q, s, _ = mg.pack_int8(raw[key])
        base = key.removesuffix(".weight")
        assert np.array_equal(qw[f"{base}.qweight"].numpy(), q) and np.array_equal(bits(qw[f"{base}.scale"]), s)
    # float64 with the linears' dequantized values: matches HF's float64 logits tightly
    w64 = {k: v.double() for k, v in w16.items()}
    for key in [k for k in raw if k.endswith("proj.weight")]:
        base = key.removesuffix(".weight")
        w64[key] = dequantize(qw[f"{base}.qweight"], qw[f"{base}.scale"], torch.bfloat16).double()
    tables = om.tables_for(cfg, 256)
    prompts = [mg.prompt_ids(n, s, cfg.vocab_size) for n, s in mg.PROMPTS]
    for dtype, weights in ((torch.float64, w64), (torch.bfloat16, qw)):
        shape = (64, cfg.num_key_value_heads, cfg.head_dim)
        kv = [(torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)) for _ in range(cfg.num_hidden_layers)]
        seqs = [list(p) for p in prompts]
        tabs = [[0, 1], [3, 2]]  # physical blocks out of order for the second sequence
        starts = [0, 0]
        for step in range(mg.DECODE_STEPS + 1):
            sched = [(s, st, len(s) - st, t) for s, st, t in zip(seqs, starts, tabs, strict=True)]
            logits, ids = om.run_step(cfg, weights, kv, om.prepare(sched, 16), 16, tables)
            ref = torch.from_numpy(g["logits"][step])
            if dtype == torch.float64:
                torch.testing.assert_close(logits.double(), ref, atol=1e-6, rtol=1e-5)
                assert ids.tolist() == g["next_ids"][step].tolist()
            else:
                assert rel_l2(logits, ref) < 1e-2, step
                margin = torch.from_numpy(g["top2_margin"][step])
                assert all(int(a) == int(b) or float(m) < 2e-2
                           for a, b, m in zip(ids, g["next_ids"][step], margin, strict=True))
            starts = [len(s) for s in seqs]
            for s, nxt in zip(seqs, g["next_ids"][step].tolist(), strict=True):
                s.append(int(nxt))  # teacher-forced with the float64 model's greedy ids
