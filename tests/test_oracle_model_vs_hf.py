"""Pins the oracle's Qwen3 forward against transformers' Qwen3ForCausalLM in float64.

Mirrors the reference's tests/correctness/test_model_vs_hf.py:17-44 (fresh prefill, a chunk that
attends to cached keys plus single-token decodes, an untied LM head) at atol 1e-6 / rtol 1e-5,
and adds the int8 model (HF weights replaced by their dequantized values) and a model with
Qwen3's real head geometry (head_dim 128, theta 1e6).
"""

from __future__ import annotations

from typing import Any

import torch
from conftest import SMALL_QWEN3, TINY_CONFIG, build_hf_model
from helpers import new_kv_caches, oracle_run_chunk

from oracle import model as om
from oracle.int8 import dequantize


def _oracle(hf: Any) -> tuple[om.Config, dict[str, torch.Tensor], tuple[torch.Tensor, torch.Tensor]]:
    cfg = om.Config.from_dict(hf.config.to_dict())
    weights = om.from_hf_state_dict(hf.state_dict(), cfg, torch.float64)
    tables = om.tables_for(cfg, 512)
    return cfg, weights, tables


def _full(cfg, weights, tables, ids, bs=4):
    kv = new_kv_caches(cfg, -(-len(ids) // bs) * bs, torch.float64)
    return oracle_run_chunk(cfg, weights, kv, ids, 0, bs, tables)


def _hf_logits(hf: Any, ids: list[int]) -> torch.Tensor:
    with torch.no_grad():
        return hf(torch.tensor([ids])).logits[0].double()


def test_prefill_logits_match_hf(tiny_hf: Any) -> None:
    ids = torch.randint(0, 512, (40,), generator=torch.Generator().manual_seed(0)).tolist()
    cfg, w, t = _oracle(tiny_hf)
    torch.testing.assert_close(_full(cfg, w, t, ids).double(), _hf_logits(tiny_hf, ids), atol=1e-6, rtol=1e-5)


def test_chunked_prefill_and_decode_match_hf(tiny_hf: Any) -> None:
    ids = torch.randint(0, 512, (50,), generator=torch.Generator().manual_seed(1)).tolist()
    cfg, w, t = _oracle(tiny_hf)
    kv = new_kv_caches(cfg, 64, torch.float64)
    parts = [
        oracle_run_chunk(cfg, w, kv, ids[:20], 0, 4, t),
        oracle_run_chunk(cfg, w, kv, ids[20:43], 20, 4, t),
        *[oracle_run_chunk(cfg, w, kv, [ids[p]], p, 4, t) for p in range(43, 50)],
    ]
    torch.testing.assert_close(torch.cat(parts).double(), _hf_logits(tiny_hf, ids), atol=1e-6, rtol=1e-5)


def test_untied_lm_head() -> None:
    hf = build_hf_model(tie_word_embeddings=False, seed=3)
    ids = list(range(5, 25))
    cfg, w, t = _oracle(hf)
    assert "lm_head.weight" in w
    torch.testing.assert_close(_full(cfg, w, t, ids).double(), _hf_logits(hf, ids), atol=1e-6, rtol=1e-5)


def _hf_with_int8_weights(hf: Any, cfg: om.Config, qw: dict[str, torch.Tensor]) -> None:
    """Write bf16(q*s)-style dequantized weights back into HF's unfused projections."""
    h, kvh, d, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size
    sd = hf.state_dict()
    for i in range(cfg.num_hidden_layers):
        p = f"layers.{i}"
        deq = {n: dequantize(qw[f"{p}.{n}.qweight"], qw[f"{p}.{n}.scale"], torch.float64) for n in om.QUANTIZED}
        qkv = deq["self_attn.qkv_proj"]
        splits = {"q_proj": qkv[: h * d], "k_proj": qkv[h * d : h * d + kvh * d], "v_proj": qkv[h * d + kvh * d :]}
        for n, wt in splits.items():
            sd[f"model.{p}.self_attn.{n}.weight"].copy_(wt)
        sd[f"model.{p}.self_attn.o_proj.weight"].copy_(deq["self_attn.o_proj"])
        sd[f"model.{p}.mlp.gate_proj.weight"].copy_(deq["mlp.gate_up_proj"][:inter])
        sd[f"model.{p}.mlp.up_proj.weight"].copy_(deq["mlp.gate_up_proj"][inter:])
        sd[f"model.{p}.mlp.down_proj.weight"].copy_(deq["mlp.down_proj"])


def test_int8_model_matches_hf_with_dequantized_weights() -> None:
    hf = build_hf_model(seed=4)
    cfg, w, t = _oracle(hf)
    qw = om.quantize_weights(w, cfg)
    assert "layers.0.self_attn.qkv_proj.weight" not in qw
    assert qw["layers.1.mlp.down_proj.qweight"].dtype == torch.int8
    _hf_with_int8_weights(hf, cfg, qw)
    ids = torch.randint(0, 512, (33,), generator=torch.Generator().manual_seed(4)).tolist()
    kv = new_kv_caches(cfg, 64, torch.float64)
    parts = [
        oracle_run_chunk(cfg, qw, kv, ids[:17], 0, 4, t),
        *[oracle_run_chunk(cfg, qw, kv, [ids[p]], p, 4, t) for p in range(17, 33)],
    ]
    torch.testing.assert_close(torch.cat(parts).double(), _hf_logits(hf, ids), atol=1e-6, rtol=1e-5)


def test_qwen3_head_geometry_matches_hf() -> None:
    """head_dim 128 (RoPE pairs i <-> i+64), theta 1e6, block size 16, decode after prefill."""
    over = {k: v for k, v in SMALL_QWEN3.items() if k not in TINY_CONFIG or SMALL_QWEN3[k] != TINY_CONFIG[k]}
    hf = build_hf_model(seed=5, **over)
    cfg, w, t = _oracle(hf)
    assert cfg.head_dim == 128 and cfg.rope_theta == 1e6
    ids = torch.randint(0, 1024, (37,), generator=torch.Generator().manual_seed(6)).tolist()
    kv = new_kv_caches(cfg, 64, torch.float64)
    parts = [
        oracle_run_chunk(cfg, w, kv, ids[:30], 0, 16, t),
        *[oracle_run_chunk(cfg, w, kv, [ids[p]], p, 16, t) for p in range(30, 37)],
    ]
    torch.testing.assert_close(torch.cat(parts).double(), _hf_logits(hf, ids), atol=1e-6, rtol=1e-5)


def test_greedy_first_index_wins() -> None:
    logits = torch.tensor([[0.0, 3.0, 3.0, 1.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -1.0, -3.0]])
    assert om.greedy(logits).tolist() == [1, 0, 0]
