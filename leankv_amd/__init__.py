"""leankv_amd -- MI355X (gfx950) native decode hot path of LeanKV.

Module map (mirrors the reference's public API):
  leankv_amd.teal.sparse_fns          SparsifyFn, threshold selection
  leankv_amd.teal.kernels.sparse_gemv sparse_gemv / prepare_weight_for_sparse_gemv
  leankv_amd.teal.patching            apply_teal / remove_teal (HIP kernel patch)
  leankv_amd.turboquant.codebook      Lloyd-Max codebook
  leankv_amd.turboquant.rotation      random rotation
  leankv_amd.turboquant.quantizer     TurboQuantMSE (HIP quantize / dequantize)
  leankv_amd.turboquant.cache         TurboQuantCache (static packed storage)
  leankv_amd.turboquant.attention     fused decode attention for HF models
  leankv_amd.combined                 optimize_model / load_model
  leankv_amd.engine                   graph-captured static decode engine
  leankv_amd.kernels                  torch wrappers of the C ABI (include/leankv_amd.h)
"""

__version__ = "0.1.0"
