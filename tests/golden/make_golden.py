"""Writes the golden fixtures of this directory. Run from the repository root:

    python tests/golden/make_golden.py

The expected values come from computations independent of ``oracle/`` and of the HIP library:

* ``int8_pack.npz``   -- int8 weight packing (the reference's quant/int8.py:27-32) restated in
  numpy: IEEE float32 ``amax / 127``, float32 division, ``np.rint`` (half to even), clamp, and
  the bf16 scale and the dequantized ``bf16(q * s)`` rounded to nearest even in integer
  arithmetic. Crafted rows: exact half-way ties, an all-zero row, values below the 1e-8 clamp, a
  negative maximum, values near the bf16 maximum.
* ``int8_linear.npz`` -- ``x @ bf16(q * s)^T`` in float64 (quant/int8.py:35-37), ragged M = 5.
* ``paged_attention.npz`` -- float64 brute-force softmax attention through block tables
  (attention/backends.py:145-197 semantics): four decode rows with contexts 1, 16, 17 and 33
  (one key; exactly one block; one past a block; three blocks) and one three-token chunk after
  14 cached keys (a speculative-verify shape crossing a block boundary), GQA 4 query heads over
  2 KV heads, permuted physical blocks; the expected slot of every new token
  (``table[p // 16] * 16 + p % 16``, model_runner.py:189).
* ``qwen3_tiny.npz``  -- a 2-layer Qwen3 (head_dim 128, 2 query / 1 KV heads, hidden 128,
  vocabulary 512) whose weights come from ``tiny_model_weights`` below; the decoder linears are
  packed by the numpy restatement and ``transformers.Qwen3ForCausalLM`` runs in float64 on the
  dequantized values: logits of the last row of two sequences after their prompts and after each
  of three greedy decode steps, the greedy ids, and a sha256 of the generated weights.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BLOCK = 16

TINY_QWEN3 = {
    "vocab_size": 512,
    "hidden_size": 128,
    "intermediate_size": 256,
    "num_hidden_layers": 2,
    "num_attention_heads": 2,
    "num_key_value_heads": 1,
    "head_dim": 128,
    "rms_norm_eps": 1e-6,
    "rope_theta": 1_000_000.0,
    "max_position_embeddings": 2048,
    "tie_word_embeddings": True,
}
TINY_SEED = 20
PROMPTS = ((23, 101), (9, 202))  # (length, seed) of each sequence's prompt
DECODE_STEPS = 3
LINEARS = ("self_attn.qkv_proj", "self_attn.o_proj", "mlp.gate_up_proj", "mlp.down_proj")


# ---- bf16 and the int8 pack, in numpy --------------------------------------------------------------


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_int8(w_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """bf16 weight bits [out, in] -> (q int8, scale bf16 bits, dequantized bf16 bits)."""
    w = bf16_value(w_bits)
    amax = np.abs(w).max(axis=1)
    s32 = np.maximum(amax, np.float32(1e-8)).astype(np.float32) / np.float32(127.0)
    q = np.clip(np.rint(w / s32[:, None]), -127, 127).astype(np.int8)
    scale = bf16_bits(s32)
    deq = bf16_bits(q.astype(np.float32) * bf16_value(scale)[:, None])  # exact product, then RNE
    return q, scale, deq


# ---- the tiny model's weights -----------------------------------------------------------------------


def tiny_weight_shapes(cfg: dict) -> dict[str, tuple[int, ...]]:
    """Parameter name -> shape with the fused qkv / gate_up rows (q|k|v, gate|up)."""
    h, d = cfg["hidden_size"], cfg["head_dim"]
    q, kv, inter = cfg["num_attention_heads"] * d, cfg["num_key_value_heads"] * d, cfg["intermediate_size"]
    shapes: dict[str, tuple[int, ...]] = {"embed_tokens.weight": (cfg["vocab_size"], h)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"layers.{i}."
        shapes[p + "input_layernorm.weight"] = (h,)
        shapes[p + "self_attn.qkv_proj.weight"] = (q + 2 * kv, h)
        shapes[p + "self_attn.o_proj.weight"] = (h, q)
        shapes[p + "self_attn.q_norm.weight"] = (d,)
        shapes[p + "self_attn.k_norm.weight"] = (d,)
        shapes[p + "post_attention_layernorm.weight"] = (h,)
        shapes[p + "mlp.gate_up_proj.weight"] = (2 * inter, h)
        shapes[p + "mlp.down_proj.weight"] = (h, inter)
    shapes["norm.weight"] = (h,)
    return shapes


def tiny_model_weights(cfg: dict = TINY_QWEN3, seed: int = TINY_SEED) -> dict[str, np.ndarray]:
    """bf16 bit patterns: linears and the embedding N(0, 0.02), norm weights 1 + 0.1 N(0, 1)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in tiny_weight_shapes(cfg).items():
        z = rng.standard_normal(shape, dtype=np.float32)
        val = (np.float32(1.0) + np.float32(0.1) * z) if name.endswith("norm.weight") else np.float32(0.02) * z
        out[name] = bf16_bits(val)
    return out


def weights_digest(weights: dict[str, np.ndarray]) -> str:
    h = hashlib.sha256()
    for name in sorted(weights):
        h.update(name.encode())
        h.update(np.ascontiguousarray(weights[name]).tobytes())
    return h.hexdigest()


def prompt_ids(length: int, seed: int, vocab: int) -> list[int]:
    return np.random.default_rng(seed).integers(0, vocab, size=length).tolist()


# ---- fixtures -----------------------------------------------------------------------------------------


def make_pack() -> None:
    rng = np.random.default_rng(1)
    k = 64
    rows = [0.02 * rng.standard_normal(k)]
    ties = np.array([127.5 - 0.5] + [(j + 0.5) * (1 if j % 2 else -1) for j in range(k - 1)]) / 128.0
    rows.append(ties)  # max 127/128 -> s = 1/128 exactly, so w / s = j + 0.5 exactly
    rows.append(np.zeros(k))
    rows.append(np.full(k, 1e-12) * rng.choice([-1.0, 1.0], size=k))  # below the clamp: q = 0
    near = rng.uniform(-5e-9, 5e-9, size=k)
    near[7] = 5e-9
    rows.append(near)  # amax < 1e-8: the clamp sets the scale
    neg = 0.25 * rng.standard_normal(k)
    neg[11] = -1.5
    rows.append(neg)  # the row maximum is negative
    big = rng.uniform(-1.0, 1.0, size=k) * 3.0e38
    big[3] = 3.3e38
    rows.append(big)  # near the bf16 maximum
    rows.append(rng.standard_normal(k) * 100.0)
    w_bits = bf16_bits(np.array(rows, dtype=np.float32))
    q, scale, deq = pack_int8(w_bits)
    assert np.abs(q).max() <= 127 and (q[2] == 0).all() and (q[3] == 0).all()
    # the tie row: w / s = +-(j + 0.5) rounds to the even neighbour
    t = np.array([(j + 0.5) * (1 if j % 2 else -1) for j in range(k - 1)])
    assert (q[1, 1:] == np.rint(t)).all() and q[1, 0] == 127
    np.savez_compressed(HERE / "int8_pack.npz", w_bits=w_bits, q=q, scale_bits=scale, deq_bits=deq)


def make_linear() -> None:
    rng = np.random.default_rng(2)
    w_bits = bf16_bits(0.02 * rng.standard_normal((24, 64), dtype=np.float32))
    x_bits = bf16_bits(rng.standard_normal((5, 64), dtype=np.float32))
    q, scale, deq = pack_int8(w_bits)
    y = bf16_value(x_bits).astype(np.float64) @ bf16_value(deq).astype(np.float64).T
    np.savez_compressed(HERE / "int8_linear.npz", w_bits=w_bits, x_bits=x_bits, q=q, scale_bits=scale, y=y)


def make_attention() -> None:
    rng = np.random.default_rng(3)
    heads, kv_heads, dim, num_blocks = 4, 2, 128, 9
    group = heads // kv_heads
    k_bits = bf16_bits(rng.standard_normal((num_blocks * BLOCK, kv_heads, dim), dtype=np.float32))
    v_bits = bf16_bits(rng.standard_normal((num_blocks * BLOCK, kv_heads, dim), dtype=np.float32))
    # (num_cached, num_new, block table); rows are laid out in this order in the flat batch
    seqs = [(0, 1, [5]), (15, 1, [2]), (16, 1, [7, 0]), (32, 1, [3, 6, 1]), (14, 3, [4, 8])]
    rows = sum(n for _, n, _ in seqs)
    q_bits = bf16_bits(rng.standard_normal((rows, heads, dim), dtype=np.float32))
    scale = dim**-0.5
    kf, vf, qf = (bf16_value(b).astype(np.float64) for b in (k_bits, v_bits, q_bits))
    out = np.zeros((rows, heads, dim))
    slots = np.zeros(rows, dtype=np.int64)
    r = 0
    for cached, new, table in seqs:
        for j in range(new):
            pos = cached + j
            slots[r] = table[pos // BLOCK] * BLOCK + pos % BLOCK
            keys = [table[p // BLOCK] * BLOCK + p % BLOCK for p in range(pos + 1)]  # causal: keys 0..pos
            for h in range(heads):
                kk, vv = kf[keys, h // group], vf[keys, h // group]
                s = kk @ qf[r, h] * scale
                p = np.exp(s - s.max())
                out[r, h] = (p / p.sum()) @ vv
            r += 1
    tables = np.full((len(seqs), 3), -1, dtype=np.int32)
    for i, (_, _, t) in enumerate(seqs):
        tables[i, : len(t)] = t
    info = np.array([[c, n] for c, n, _ in seqs], dtype=np.int32)
    np.savez_compressed(HERE / "paged_attention.npz", k_bits=k_bits, v_bits=v_bits, q_bits=q_bits,
                        tables=tables, cached_new=info, slots=slots, out=out, scale=np.float64(scale),
                        heads=np.int32(heads), kv_heads=np.int32(kv_heads))


def make_qwen3_tiny() -> None:
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = TINY_QWEN3
    weights = tiny_model_weights()
    h, kvh, d, inter = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["intermediate_size"]
    hf = Qwen3ForCausalLM(Qwen3Config(**cfg)).to(torch.float64).eval()
    sd = hf.state_dict()

    def put(name: str, arr: np.ndarray) -> None:
        sd[name].copy_(torch.from_numpy(arr.astype(np.float64)))

    put("model.embed_tokens.weight", bf16_value(weights["embed_tokens.weight"]))
    put("model.norm.weight", bf16_value(weights["norm.weight"]))
    for i in range(cfg["num_hidden_layers"]):
        p = f"layers.{i}."
        for n in ("input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm"):
            put(f"model.{p}{n}.weight", bf16_value(weights[f"{p}{n}.weight"]))
        deq = {n: bf16_value(pack_int8(weights[f"{p}{n}.weight"])[2]) for n in LINEARS}
        qkv = deq["self_attn.qkv_proj"]
        put(f"model.{p}self_attn.q_proj.weight", qkv[: h * d])
        put(f"model.{p}self_attn.k_proj.weight", qkv[h * d : h * d + kvh * d])
        put(f"model.{p}self_attn.v_proj.weight", qkv[h * d + kvh * d :])
        put(f"model.{p}self_attn.o_proj.weight", deq["self_attn.o_proj"])
        put(f"model.{p}mlp.gate_proj.weight", deq["mlp.gate_up_proj"][:inter])
        put(f"model.{p}mlp.up_proj.weight", deq["mlp.gate_up_proj"][inter:])
        put(f"model.{p}mlp.down_proj.weight", deq["mlp.down_proj"])
    assert hf.lm_head.weight.data_ptr() == hf.model.embed_tokens.weight.data_ptr()  # tied
    seqs = [prompt_ids(n, s, cfg["vocab_size"]) for n, s in PROMPTS]
    logits = np.zeros((DECODE_STEPS + 1, len(seqs), cfg["vocab_size"]))
    ids = np.zeros((DECODE_STEPS + 1, len(seqs)), dtype=np.int64)
    with torch.no_grad():
        for step in range(DECODE_STEPS + 1):
            for i, s in enumerate(seqs):
                logits[step, i] = hf(torch.tensor([s])).logits[0, -1].numpy()
                ids[step, i] = int(np.argmax(logits[step, i]))
            for i, s in enumerate(seqs):
                s.append(int(ids[step, i]))
    top2 = np.sort(logits, axis=-1)[..., -2:]
    np.savez_compressed(HERE / "qwen3_tiny.npz", config=np.array(json.dumps(cfg)), seed=np.int64(TINY_SEED),
                        digest=np.array(weights_digest(weights)), logits=logits, next_ids=ids,
                        top2_margin=top2[..., 1] - top2[..., 0])


if __name__ == "__main__":
    make_pack()
    make_linear()
    make_attention()
    make_qwen3_tiny()
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")
