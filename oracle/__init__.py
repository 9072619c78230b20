"""CPU oracle for the Strata per-token hot path (TEST INFRASTRUCTURE ONLY).

This package restates, in NumPy (and plain C under ``oracle/c``), the
reference's algorithms for the quantized linear layer, RoPE, the KV-cache
append contract, chunked grouped-query attention, the Llama decoder block and
the greedy loop.  Every function cites the reference file:line it follows
(paths relative to the reference repository root, ``src/ollm/...``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline.  The product path (``lokahi_amd``) never imports it and
has no CPU fallback.

Parity status per function (what pins it, beyond the restatement itself):

* ``bf16``: round-to-nearest-even f32->bf16, pinned against torch's own
  ``.to(torch.bfloat16)`` conversion on random and special values.
* ``q4.pack/unpack``: pinned by brute force on tiny cases and the closed-form
  nibble rule (element k of row n is nibble k%8 of word k/8, LSB first).
* ``q4.quantized_matmul``: pinned against torch float64 matmul of the
  dequantized matrix, the all-zero-code closed form, one-hot inputs and
  linearity.  Exact MLX accumulation order: parity unpinned (MLX absent).
* ``q4.quantize``: a fixture generator only (matmul parity is defined on the
  packed triple); MLX's exact scale/bias selection: parity unpinned.
* ``rope``: pinned by the complex-number form of the rotation, identity at
  position 0, per-pair norm preservation and relative-position invariance.
* ``kvcache``: pinned by the reference tests' arange known answers
  (tests/test_mlx_kvcache.py:23-68).
* ``attention``: pinned against torch float64 scaled-dot-product attention,
  chunk-size independence and the causal "future values" invariant
  (tests/test_mlx_attention.py:113-130).
* ``llama`` / ``generation``: pinned by cached-decode == full-forward
  (tests/test_mlx_generation.py:140-156) and the recording-model greedy
  contract (tests/test_mlx_generation.py:282-323).
"""
