"""TurboQuant KV-cache quantization (MSE variant) on HIP kernels."""
