"""CPU oracle for the Block-RVQ / route-codebook linear forward.

TEST INFRASTRUCTURE ONLY.  Two restatements of the reference's arithmetic live
here, and only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import them, as the checker (never as the thing that
is measured or shipped):

* ``rvq_oracle.c`` (loaded through ``oracle.c_oracle``): a plain-C restatement
  with its own IEEE-754 round-to-nearest-even conversions; the bit-exact
  reference for dequantised weights.
* ``oracle.ref_ops``: the reference's torch op sequence for the default
  ``per_group`` strategy, executed by torch on the CPU; the CPU baseline, and
  the independent check that the C restatement rounds the way torch does.

Pinning (what checks each function, see ``tests/test_oracle.py``):

* ``or_f32_to_f16`` / ``or_f32_to_bf16`` / ``or_f16_to_f32``: against numpy's
  and torch's casts over random and special bit patterns.
* ``or_reconstruct_weight``: against ``ref_ops.reconstruct_weight`` (torch),
  closed forms (S = 1 constant codebook, zero stages, all-zero ids), the
  one-hot contraction identity, and a float64 error bound.
* ``or_reconstruct_weight_fast``: against ``ref_ops.reconstruct_weight_fast``
  and the active-stage fixtures in ``tests/golden``.
* ``or_linear_f64``: against numpy float64 matmul.
* ``or_triton_rvq_matmul``: against a float64 closed form (S = 1, unit scale)
  and ``ref_ops.triton_rvq_matmul``.
* ``or_id_route_weight``: against ``ref_ops.id_route_weight``.
"""
