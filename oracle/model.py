"""Oracle: the Qwen3 forward over a flat batch, logits and greedy sampling (test infrastructure only).

A functional restatement over a flat ``weights`` dict whose keys are the module paths of the
reference model (``layers.{i}.self_attn.qkv_proj.weight`` or ``...qweight`` + ``...scale`` once
quantized, ``embed_tokens.weight``, ``norm.weight``, optional ``lm_head.weight``).

Follows:
  * ``Config``                <- ``Qwen3Config``  model/qwen3.py:18-62
  * ``from_hf_state_dict``    <- the fused row order of model/loader.py:22-28, 41-48
  * ``quantize_weights``      <- ``quantize_int8_``  quant/int8.py:40-60
  * ``attention_block``       <- ``Qwen3Attention.forward``  model/qwen3.py:84-101
  * ``decoder_layer``         <- ``Qwen3DecoderLayer.forward``  model/qwen3.py:112-122
  * ``forward``               <- ``Qwen3ForCausalLM.forward``  model/qwen3.py:140-153
  * ``compute_logits``        <- model/qwen3.py:155-158 (bf16 product, then float32)
  * ``greedy``                <- runner/sampler.py:59 (argmax, first index wins)
  * ``prepare``               <- ``ModelRunner.prepare``  runner/model_runner.py:162-205
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F
from torch import Tensor

from oracle.attention import OracleMeta, SeqChunk, build_attention_metadata, paged_attention
from oracle.int8 import int8_linear, quantize_int8
from oracle.layers import apply_rope, rms_norm, rope_tables

QUANTIZED = ("self_attn.qkv_proj", "self_attn.o_proj", "mlp.gate_up_proj", "mlp.down_proj")


@dataclass(frozen=True)
class Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int
    tie_word_embeddings: bool

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> Config:
        rope = d.get("rope_parameters") or {}
        return cls(
            vocab_size=d["vocab_size"],
            hidden_size=d["hidden_size"],
            intermediate_size=d["intermediate_size"],
            num_hidden_layers=d["num_hidden_layers"],
            num_attention_heads=d["num_attention_heads"],
            num_key_value_heads=d["num_key_value_heads"],
            head_dim=d.get("head_dim") or d["hidden_size"] // d["num_attention_heads"],
            rms_norm_eps=d["rms_norm_eps"],
            rope_theta=float(d.get("rope_theta") or rope.get("rope_theta") or 10000.0),
            max_position_embeddings=d["max_position_embeddings"],
            tie_word_embeddings=bool(d.get("tie_word_embeddings", False)),
        )


def from_hf_state_dict(sd: dict[str, Tensor], cfg: Config, dtype: torch.dtype) -> dict[str, Tensor]:
    """HF checkpoint names -> fused qkv ([q | k | v] rows) and gate_up ([gate | up] rows)."""
    out: dict[str, Tensor] = {}
    for name, t in sd.items():
        if name == "lm_head.weight" and cfg.tie_word_embeddings:
            continue
        out[name.removeprefix("model.")] = t.to(dtype)
    for i in range(cfg.num_hidden_layers):
        p = f"layers.{i}."
        q, k, v = (out.pop(f"{p}self_attn.{n}_proj.weight") for n in "qkv")
        out[f"{p}self_attn.qkv_proj.weight"] = torch.cat([q, k, v], dim=0)
        g, u = (out.pop(f"{p}mlp.{n}_proj.weight") for n in ("gate", "up"))
        out[f"{p}mlp.gate_up_proj.weight"] = torch.cat([g, u], dim=0)
    return out


def quantize_weights(weights: dict[str, Tensor], cfg: Config) -> dict[str, Tensor]:
    """Swap the four decoder-layer linears for (qweight, scale); embedding / LM head stay."""
    out = dict(weights)
    for i in range(cfg.num_hidden_layers):
        for name in QUANTIZED:
            key = f"layers.{i}.{name}"
            q, s = quantize_int8(out.pop(f"{key}.weight"))
            out[f"{key}.qweight"], out[f"{key}.scale"] = q, s
    return out


def linear(weights: dict[str, Tensor], key: str, x: Tensor) -> Tensor:
    if f"{key}.qweight" in weights:
        return int8_linear(x, weights[f"{key}.qweight"], weights[f"{key}.scale"])
    return F.linear(x, weights[f"{key}.weight"])


def attention_block(
    cfg: Config,
    weights: dict[str, Tensor],
    i: int,
    x: Tensor,
    cos: Tensor,
    sin: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    meta: OracleMeta,
) -> Tensor:
    """model/qwen3.py:84-101."""
    p = f"layers.{i}.self_attn"
    t = x.shape[0]
    h, kvh, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    q, k, v = linear(weights, f"{p}.qkv_proj", x).split([h * d, kvh * d, kvh * d], dim=-1)
    q = rms_norm(q.view(t, h, d), weights[f"{p}.q_norm.weight"], cfg.rms_norm_eps)
    k = rms_norm(k.view(t, kvh, d), weights[f"{p}.k_norm.weight"], cfg.rms_norm_eps)
    v = v.view(t, kvh, d)
    q, k = apply_rope(q, k, cos, sin)
    out = paged_attention(q, k, v, k_cache, v_cache, meta, d**-0.5)
    return linear(weights, f"{p}.o_proj", out.reshape(t, h * d))


def decoder_layer(
    cfg: Config,
    weights: dict[str, Tensor],
    i: int,
    x: Tensor,
    cos: Tensor,
    sin: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    meta: OracleMeta,
) -> Tensor:
    """x += attn(norm(x)); x += mlp(norm(x))  (model/qwen3.py:112-122)."""
    p = f"layers.{i}"
    eps = cfg.rms_norm_eps
    h = rms_norm(x, weights[f"{p}.input_layernorm.weight"], eps)
    x = x + attention_block(cfg, weights, i, h, cos, sin, k_cache, v_cache, meta)
    h = rms_norm(x, weights[f"{p}.post_attention_layernorm.weight"], eps)
    gate, up = linear(weights, f"{p}.mlp.gate_up_proj", h).chunk(2, dim=-1)
    return x + linear(weights, f"{p}.mlp.down_proj", F.silu(gate) * up)


def forward(
    cfg: Config,
    weights: dict[str, Tensor],
    input_ids: Tensor,
    positions: Tensor,
    kv_caches: list[tuple[Tensor, Tensor]],
    meta: OracleMeta,
    tables: tuple[Tensor, Tensor],
) -> Tensor:
    """Embed, then every layer, then the final norm (model/qwen3.py:140-153)."""
    x = F.embedding(input_ids, weights["embed_tokens.weight"])
    cos, sin = tables[0][positions], tables[1][positions]
    for i, (kc, vc) in enumerate(kv_caches):
        x = decoder_layer(cfg, weights, i, x, cos, sin, kc, vc, meta)
    return rms_norm(x, weights["norm.weight"], cfg.rms_norm_eps)


def compute_logits(cfg: Config, weights: dict[str, Tensor], hidden: Tensor) -> Tensor:
    """LM head in the model dtype, then float32 (model/qwen3.py:155-158)."""
    w = weights["embed_tokens.weight"] if cfg.tie_word_embeddings else weights["lm_head.weight"]
    return F.linear(hidden, w).float()


def greedy(logits: Tensor) -> Tensor:
    """runner/sampler.py:59 -- ``argmax`` returns the first index among equal maxima."""
    return logits.argmax(dim=-1)


def tables_for(cfg: Config, max_positions: int) -> tuple[Tensor, Tensor]:
    return rope_tables(cfg.head_dim, max_positions, cfg.rope_theta)


@dataclass
class StepInputs:
    input_ids: Tensor
    positions: Tensor
    slot_mapping: Tensor
    chunks: list[SeqChunk]
    logits_rows: Tensor


def prepare(
    seqs: list[tuple[list[int], int, int, list[int]]], block_size: int
) -> StepInputs:
    """Flatten scheduled sequences (model_runner.py:179-205, without speculation).

    Each entry is (token_ids, num_computed, num_new, block_table). A row is sampled when the
    chunk reaches the end of the sequence's tokens.
    """
    ids: list[int] = []
    pos: list[int] = []
    slots: list[int] = []
    chunks: list[SeqChunk] = []
    rows: list[int] = []
    for tokens, start, n, table in seqs:
        flat = len(ids)
        ids.extend(tokens[start : start + n])
        pos.extend(range(start, start + n))
        slots.extend(table[p // block_size] * block_size + p % block_size for p in range(start, start + n))
        chunks.append(SeqChunk(flat, n, start, table))
        if start + n == len(tokens):
            rows.append(flat + n - 1)
    return StepInputs(
        torch.tensor(ids, dtype=torch.long),
        torch.tensor(pos, dtype=torch.long),
        torch.tensor(slots, dtype=torch.long),
        chunks,
        torch.tensor(rows, dtype=torch.long),
    )


def run_step(
    cfg: Config,
    weights: dict[str, Tensor],
    kv_caches: list[tuple[Tensor, Tensor]],
    step: StepInputs,
    block_size: int,
    tables: tuple[Tensor, Tensor],
) -> tuple[Tensor, Tensor]:
    """One runner step (model_runner.py:207-227, greedy): returns (logits [R, V], ids [R])."""
    meta = build_attention_metadata(step.chunks, step.slot_mapping, block_size)
    with torch.inference_mode():
        hidden = forward(cfg, weights, step.input_ids, step.positions, kv_caches, meta, tables)
        logits = compute_logits(cfg, weights, hidden[step.logits_rows])
    return logits, greedy(logits)
