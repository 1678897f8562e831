"""CPU oracle of the LeanKV decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU (numpy / torch-CPU), the reference
algorithms that the HIP kernels of ``leankv_amd`` replace, each function citing
the reference file:line it follows.  It is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and the product package never imports, calls or
falls back to it.

Pins (what makes each restatement trustworthy beyond retyping the formula):
  teal.sparse_gemv / gateup_swiglu -- fp64 brute force + closed-form checks
      (all-pass mask == dense matvec, all-drop == 0, linearity in x).
  teal.threshold_for_sparsity      -- torch.kthvalue (library routine) + exact
      zero-count property when magnitudes are distinct.
  turboquant.rotation_matrix       -- Q orthogonal and Q^T G upper triangular
      with positive diagonal (unique QR), G = seeded torch.randn.
  turboquant.pack/unpack           -- brute-force bit loops on tiny inputs,
      round trip, byte layout of the reference's shifts.
  turboquant.quantize              -- searchsorted == per-coordinate boundary
      count (brute force); fp64 rotation for tie analysis.
  codebook values                  -- golden fixtures written by the
      reference's own solver (tests/golden/make_golden.py), plus the
      Lloyd-Max optimality conditions.
  attention                        -- fp64 softmax closed form; dequantize +
      attention equals the rotated-domain factorisation.
No function of this package is "parity unpinned".
"""
