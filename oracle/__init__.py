"""CPU oracle for the SMat chunkwise schedule -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to produce expected values or to time the CPU baseline.
Nothing under ``smat_attention_amd/`` imports it; the product's GPU path runs
hand-written HIP kernels and raises when they are missing.

Modules
-------
mask_ref   the incidence and the dense mask rebuilt from their definitions
           with plain loops (small cases), independent of the product's
           vectorised ``smat_attention_amd.mask``.
schedule   a restatement of the reference's torch path for every stage of the
           schedule (src/smat/attention.py torch branches), the fp64 dense
           oracle, the decoder, and the backward through torch autograd.

How each function is pinned (see the tests named):
  mask_ref.incidence_rows      golden C_indices (sha256 from the reference's
                               own build_mask), closed forms q, B, N0, deg,
                               theory CSV nnz of the materialised mask
                               -- tests/test_mask.py
  mask_ref.dense_mask          G == R C S^T, block layout, theory_structure.csv
                               nnz / density -- tests/test_mask.py
  schedule.smat_attention      fp64 dense masked kernel attention < 1e-10,
                               pooled == direct == subtractive, decode ==
                               prefill, chunk-width invariance, d=1 == plain
                               causal linear attention, exact non-influence
                               -- tests/test_oracle.py
  schedule.walsh_incidence /   dense Walsh / zeta matrices -- tests/test_oracle.py
  schedule.zeta_transform
  schedule backward (autograd) central finite differences in fp64
                               -- tests/test_oracle.py
"""
