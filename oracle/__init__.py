"""CPU oracle for the DeBERTa disentangled-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, and only as the checker (or the timed CPU
baseline), never as a fallback for the HIP path.

Contents (each function cites the reference file:line it restates):

* ``positions``  - log-bucket function, compact slot plan, dense gather map
  (``_reference.py:115-158``, ``position.py:89-156``).  Pinned by closed forms
  (S(L) table, bucket(256) = 192, bucket(511) = 255, odd symmetry, identity
  inside the mid band), float32-vs-float64 agreement, brute force, the
  reference's own test (``tests/test_position.py:13-16``) and the Hugging Face
  ``make_log_bucket_position`` vectors in ``tests/golden``.
* ``attention``  - float64 numpy restatements of the unfused "original"
  equation (``_reference.py:252-422``) and of the fused kernel contract
  (``kernel.py:196-345``), plus a pure-Python brute force for tiny shapes.
  Pinned by the Hugging Face (transformers 5.15.0) ``DisentangledSelfAttention``
  vectors in ``tests/golden``, by textbook SDPA when the relative terms are off,
  and by the padded-row / L = 1 closed forms.
* ``optimized``  - torch CPU restatement of the prepared "optimized" forward
  (``_torch.py:316-387``), the timed CPU baseline.  Pinned against the float64
  original equation.
"""
