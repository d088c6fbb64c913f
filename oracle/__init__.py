"""CPU oracle for the Gated DeltaNet path: test infrastructure, not product code.

This package restates, in plain torch on the CPU, the math of the reference
(yuyifanbupt/myvllm) kernels for:

* the fused recurrent decode step   (``ops/gated_delta_rule/fused_recurrent_gdn.py``),
* the chunked gated-delta-rule prefill (``ops/gated_delta_rule/gated_delta_rule.py``
  and the six stages it calls),
* the varlen causal conv1d prefill and the decode conv update (``ops/causal_conv1d.py``),
* the glue of the GDN layer (``layers/linear_attention.py``, ``layers/norm.py``),
* the full-attention ops beside it (``ops/full_attention.py``; ``attention.py``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
The product path (``myvllm_amd``) never imports it and has no CPU fallback.

Parity pinning (every function is pinned; none is "parity unpinned"):

* ``gdn.recurrent_gated_delta_rule_ref`` -- closed forms (single token from a
  zero state, beta=1/g=0 exact write, beta=0 pure decay, g -> -inf reset) and
  the GVA head map, in ``tests/test_oracle.py``.
* ``gdn.chunk_gated_delta_rule_ref`` -- equals the token recurrence in fp64
  for chunk 16/32/64, varlen == per-sequence, split prefill == one prefill,
  slot permutation, and its triangular inverse equals
  ``torch.linalg.solve_triangular``.
* ``conv.causal_conv1d_fn_ref`` / ``conv.causal_conv1d_update_ref`` -- equal a
  brute-force scalar loop and ``torch.nn.functional.conv1d``; update == 1-token
  prefill; new state == last W-1 rows.
* ``layer`` glue -- closed forms of sigmoid/softplus/L2/RMS norms.
* ``attention`` -- scalar loops with GQA, closed forms and permuted pages
  (its module docstring).

The reference itself has no tests, golden vectors or CPU path, and its Triton
kernels cannot run without a GPU; it is read, never imported or run.
"""
