"""CPU oracle for the Gated DeltaNet path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithms that the HIP
kernels replace.  It exists to check the GPU path, never to serve it:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker.  The product
path (``engine.kernels``) never imports this package and fails loudly when
its HIP library is missing.

Modules
-------
gdn   recurrence, chunk-64 algorithm, l2norm, varlen and spec-verify helpers
conv  causal depthwise conv1d (prefill fn and single-step update)
proj  the decode step's input projections + conv update

Pinning (how each function is known to be right, independent of itself)
------------------------------------------------------------------------
* ``gdn.recurrent_gated_delta_rule``: golden vectors written by the installed
  transformers 5.15.0 ``torch_recurrent_gated_delta_rule`` (the function the
  reference imports at engine/runtime/cuda_graphs.py:126-135), plus closed
  forms: beta=0 pure decay, single-token rank-1 write, delta-rule
  write-then-read, linearity in v at zero initial state.
* ``gdn.chunk_gated_delta_rule``: golden vectors from transformers 5.15.0
  ``torch_chunk_gated_delta_rule`` (the reference's ``_torch_fallback``,
  engine/kernels/delta_rule.py:286-349, is a line-for-line copy of it);
  equality with the recurrence in fp64 for T in {1,63,64,65,127,256};
  the forward-substitution inverse against ``numpy.linalg.solve``; state
  passing (split T and thread S) and zero-padding invariance.
* ``gdn.l2norm``: closed form ||n(x)|| = sqrt(s/(s+eps)).
* ``conv.causal_conv1d_fn`` / ``causal_conv1d_update``: golden vectors from
  transformers 5.15.0 ``causal_conv1d_fn`` / ``causal_conv1d_update`` and
  ``numpy.convolve`` per channel; update == last column of fn.
* varlen and spec-verify helpers: defined by composition of the pinned
  functions above (per-sequence loop; snapshot[t] == state after t+1 tokens).
* ``proj.round_bf16``: torch's own fp32 -> bf16 conversion.
  ``proj.in_proj_decode``: HF's module on the CPU (its four nn.Linear in
  bf16 and its causal_conv1d_update) and brute-force sums on tiny shapes.
"""
