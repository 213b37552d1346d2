"""CPU restatement of gLLM's attention hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the thing measured or shipped.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product (``gllm_amd``) never imports it and
has no CPU fallback.

Each function cites the reference file:line it restates (paths relative to the
TheEpicDolphin/gllm checkout).  The restatement follows the reference's op
order in torch on the CPU (fp32 / model dtype), and ``oracle.bruteforce``
holds independent fp64 loop versions used to pin it.

Pinning status (what each function is checked against, in
``tests/test_oracle.py``):

* ``metadata.build_metadata`` — brute-force per-element enumeration of the
  slot / bias formulas, slot-uniqueness and block-0 invariants, and the
  mask-equivalence theorem (bias == 0  <=>  p <= c_i + r on real rows).
* ``rope.rope_cache`` — fp64 closed form, exact identity at position 0.
* ``rope.apply_rope`` — exact identity at position 0, known-angle rotations,
  pair-norm preservation, inverse rotation, an fp64 closed form, and bit for
  bit a numpy brute force that rounds to bf16 (round-to-nearest-even, from
  the bit pattern) after every op, on inputs where one rounding of the exact
  result differs; in fp32, separate roundings with no fused multiply-add.
* ``attention.reference_attention`` — fp64 brute-force textbook softmax, one
  visible key => that V row, Q = 0 => mean of visible V, GQA head mapping
  h -> h // G, NaN on fully masked rows.
* ``attention.attention_layer_forward`` — write-then-gather round trip on a
  sentinel pool, and equality with ``paged_attention`` on real rows.
* ``attention.paged_attention`` — fp64 brute force, LSE split-merge identity.
* ``engine.rms_norm`` / ``engine.mlp`` — properties fixed by the maths:
  unit RMS, scale invariance, the one-hot closed form; ``x * silu(x)`` at
  known values of silu with identity weights, linearity in ``down``.
* ``engine`` (the layer loop) — the paged engine against a cache-free full
  recompute; greedy sampling is argmax.

The reference ships no golden vectors or fixtures for this path, so no
function here is checked against reference-produced numbers; none is left
"parity unpinned".
"""
