"""HIP sparse GEMV kernels for TEAL (replaces the reference's Triton kernels)."""
