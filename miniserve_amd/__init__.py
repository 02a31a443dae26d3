"""miniserve_amd -- MiniServe's per-step hot path (int8 weight-only linears, paged attention over
16-token blocks with GQA, and the norms / RoPE / SwiGLU around them) as hand-written HIP kernels
for MI355X (gfx950), behind the reference's own Python module signatures.

Module map (reference paths in parentheses):
  quant/int8.py            Int8Linear, quantize_int8_            (src/miniserve/quant/int8.py)
  attention/backends.py    SeqChunk, AttentionMetadata,
                           build_attention_metadata, paged_attention (src/miniserve/attention/backends.py)
  model/layers.py          RMSNorm, RotaryEmbedding, SwiGLU       (src/miniserve/model/layers.py)
  model/qwen3.py           Qwen3Config, Qwen3ForCausalLM          (src/miniserve/model/qwen3.py)
  runner/model_runner.py   KV pool, flat batch, greedy step        (src/miniserve/runner/model_runner.py)
  runner/sampler.py        greedy sample                           (src/miniserve/runner/sampler.py)
  utils.py                 to_device                               (src/miniserve/utils.py)
  kernels.py / _native.py  tensor wrappers over the C ABI of include/miniserve_amd.h
  build.py                 hipcc build of libminiserve_amd.so
"""

__version__ = "0.1.0"
