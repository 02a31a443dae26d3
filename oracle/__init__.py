"""CPU oracle for the int8 decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with stock PyTorch ops, what the reference MiniServe computes on
its per-step hot path (int8 weight-only linears, RMSNorm / RoPE / SwiGLU, paged attention over
16-token blocks with GQA, the Qwen3 forward over a flat batch and greedy sampling). Every function
cites the reference file:line it follows (paths relative to the reference's repository root).

Who may use it: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``, and only as the checker (or the timed CPU baseline), never as the thing measured or
shipped. ``miniserve_amd`` (the product) never imports it; the product fails loudly when its HIP
library is missing instead of falling back here.

How it is pinned (what a plausible mistake would trip):

* ``int8.quantize_int8``  -- an independent numpy restatement (IEEE float32 division, ``np.rint``
  half-to-even) bit for bit, the closed-form invariants (|q| <= 127, max|q| = 127 on nonzero rows,
  |w - q*s| <= s/2), the all-zero-row special case, and crafted exact half-way ties.
* ``int8.int8_linear`` -- float64 brute force on the dequantized weights, and the bf16 rounding
  of ``q*s`` checked bit-wise against a numpy round-to-nearest-even.
* ``layers`` / ``model`` -- ``transformers.Qwen3ForCausalLM`` (a library restatement of the same
  model) in float64 at atol 1e-6 through fresh prefill, cached-prefix prefill and decode, with
  tied and untied heads, and with int8 weights substituted as their dequantized values.
* ``attention`` -- float64 brute-force dense softmax attention per sequence through the block
  table, invariance under permuted physical block placement, and batched == alone.
* ``model.greedy`` -- ``np.argmax`` (first index wins ties).
* all of the above -- the golden fixtures of ``tests/golden/`` (numpy, float64 brute force and
  transformers' float64 Qwen3; ``tests/test_golden.py``).

Nothing here is "parity unpinned".
"""
