"""TEAL: training-free activation sparsity (magnitude thresholding) on HIP kernels."""
