/*
 * leankv_amd — C ABI of the MI355X (gfx950) decode hot path of LeanKV.
 *
 * All entry points take plain device pointers, sizes and a hipStream_t passed
 * as `void*` (NULL = the legacy default stream).  They enqueue work and return
 * immediately; nothing synchronises the host.  Return value: LKV_OK (0) or a
 * negative LKV_ERR_* code; lkv_last_error() then holds a message (per thread).
 *
 * fp16 data is passed as `const void*` / `void*` holding IEEE binary16 values.
 * Every entry point validates shapes, alignment and workspace size on the host
 * before it launches anything; a rejected call launches nothing.
 *
 * Workspaces: the split-K entry points need a caller-provided device workspace
 * of at least the size returned by the matching *_workspace_bytes() query.  It
 * needs no initialisation: every call writes the partial sums it later reads.
 * Calls that share a workspace must not overlap (use one workspace per
 * concurrently running stream).
 */
#ifndef LEANKV_AMD_H
#define LEANKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LKV_OK 0
#define LKV_ERR_INVALID (-1)     /* bad argument: shape, alignment, size      */
#define LKV_ERR_HIP (-2)         /* HIP runtime error at launch               */
#define LKV_ERR_UNSUPPORTED (-3) /* valid in the reference, not built here    */

#define LKV_DTYPE_F32 0
#define LKV_DTYPE_F16 1

/* Library version (major*10000 + minor*100 + patch) and last error text. */
int lkv_version(void);
const char* lkv_last_error(void);

/* ------------------------------------------------------------------------ */
/* TEAL sparse GEMV                                                          */
/* ------------------------------------------------------------------------ */

/*
 * y[n] = sum_{z : |x[z]| > threshold} W[n, z] * x[z]      (fp32 accumulate)
 *
 * Replaces leankv/teal/kernels/sparse_gemv.py:143-181 `sparse_gemv(x, weight,
 * threshold, sparsity_bin)` and its Triton kernel (:61-87).  `w_colmajor` is
 * the weight W[N, Z] in the column-major layout that
 * prepare_weight_for_sparse_gemv (sparse_gemv.py:229-234) produces, i.e. the
 * row-major array A[Z][N] with A[z][n] = W[n][z]; row z holds N contiguous
 * fp16 values.  x is fp16 [Z], y is fp16 [N].  The comparison is made in
 * fp32 (|x| widened, threshold as given), strictly greater, as the Triton
 * kernel does (sparse_gemv.py:82).  Rows of A whose activation fails the test
 * are never read.  Requires N % 8 == 0 and 16-byte aligned x, A, y.
 * Deterministic: the split-K partials are reduced in a fixed order.
 */
size_t lkv_sparse_gemv_workspace_bytes(int64_t N, int64_t Z);
int lkv_sparse_gemv(const void* x, const void* w_colmajor, float threshold,
                    int64_t N, int64_t Z, void* y,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * lkv_sparse_gemv without a workspace argument and without any allocation:
 * the same kernels and the same result bit for bit, with the split-K partial
 * sums in a library-owned device array of lkv_sparse_gemv_noalloc_max_bytes()
 * bytes (8 MiB; each GPU the library runs on holds its own copy until the
 * process ends).  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Runs on the current device.
 * Shapes whose partials exceed the array (lkv_sparse_gemv_workspace_bytes(N, Z)
 * above the maximum) are rejected with LKV_ERR_INVALID.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * host threads) race and must be serialised by the caller.
 */
size_t lkv_sparse_gemv_noalloc_max_bytes(void);
int lkv_sparse_gemv_noalloc(const void* x, const void* w_colmajor, float threshold,
                            int64_t N, int64_t Z, void* y, void* stream);

/*
 * Fused TEAL gate/up projection with the SwiGLU epilogue of a Mistral MLP:
 *   g = sparse_gemv(x, Wg, t_gate), u = sparse_gemv(x, Wu, t_up)
 *   h = fp16( fp16(silu(fp16(g))) * fp16(u) )
 * x is read once.  The rounding steps reproduce the eager fp16 torch
 * sequence `act_fn(gate_proj(x)) * up_proj(x)` of
 * transformers/models/mistral/modeling_mistral.py:46-47 when gate_proj and
 * up_proj are TEAL-patched (leankv/teal/patching.py:152-183).
 * Wg, Wu: column-major [N, Z] as above (A[Z][N] rows); x fp16 [Z]; h fp16 [N].
 * No single reference function: it fuses two reference sparse_gemv calls.
 */
size_t lkv_sparse_gateup_workspace_bytes(int64_t N, int64_t Z);
int lkv_sparse_gateup_swiglu(const void* x, const void* wg_colmajor,
                             const void* wu_colmajor, float t_gate, float t_up,
                             int64_t N, int64_t Z, void* h,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Up to 3 TEAL sparse GEMVs that share one input x, in one launch that reads
 * x once: y[s] = sparse_gemv(x, w[s], thresholds[s]) for s < n.  This is the
 * q/k/v step of an attention layer (leankv/teal/patching.py:169-177 patches
 * q_proj, k_proj and v_proj, PROJ_NAMES :31, which the reference runs as
 * three sparse_gemv calls on the same x).  w[s] is column-major [N[s], Z] as
 * for lkv_sparse_gemv (N[s] % 8 == 0), y[s] fp16 [N[s]]; w, thresholds, N and
 * y are host arrays of n entries.  The chunking is the fused decode step's
 * q|k|v launch, so y[s] equals that step's projection bit for bit.
 */
size_t lkv_sparse_gemv_multi_workspace_bytes(int n, const int64_t* N, int64_t Z);
int lkv_sparse_gemv_multi(const void* x, int n, const void* const* w, const float* thresholds,
                          const int64_t* N, int64_t Z, void* const* y, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * The split-K pass of lkv_sparse_gemv / lkv_sparse_gateup_swiglu alone: the
 * fp32 partial sums, without the reduction over row chunks, for callers that
 * fuse that reduction into their own consumer (the decode step does this
 * internally).  Layout: [mat][slab][chunk][256] with slab = n / 256 and
 * lkv_sparse_gemv_chunks(N, Z) chunks; mat 1 (up) only when w_up != NULL.
 * Summing a column's chunks in chunk order from 0 and rounding to fp16 gives
 * lkv_sparse_gemv's output bit for bit.
 */
int lkv_sparse_gemv_chunks(int64_t N, int64_t Z);
int lkv_sparse_gemv_partials(const void* x, const void* w_gate, const void* w_up, float t_gate, float t_up,
                             int64_t N, int64_t Z, float* partials, size_t partials_bytes, void* stream);

/*
 * batched_sparse_gemm (leankv/teal/kernels/sparse_gemv.py:184-226, kernel
 * :92-138): B > 1 decode rows, each with its own TEAL mask, one weight.
 *   y[b][n] = fp16( sum over z with |x[b][z]| > threshold of A[z][n] * x[b][z] )
 * x: fp16 [B][Z] (rows contiguous); w: the column-major weight of
 * lkv_sparse_gemv (row z of A[Z][N] holds the N weights of input z), N a
 * multiple of 8; y: fp16 [B][N].  A weight row is read once for all batch rows
 * that keep its activation (fp32 accumulate, chunk-ordered sums: equal to B
 * lkv_sparse_gemv calls up to fp32 summation order, which follows the union
 * of the batch's masks, so a row's last bits can depend on the other rows).
 */
size_t lkv_sparse_gemm_batched_workspace_bytes(int64_t B, int64_t N, int64_t Z);
int lkv_sparse_gemm_batched(const void* x, const void* w, float threshold, int64_t B, int64_t N, int64_t Z,
                            void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Up to 3 batched_sparse_gemm products of one x [B][Z] in one launch (a block
 * reads its share of x once), each product's arithmetic that of its own
 * lkv_sparse_gemm_batched call (same chunking and summation order), with an
 * epilogue in the chunk reduce:
 *   LKV_EPI_NONE      y[s] = lkv_sparse_gemm_batched(x, w[s], thresholds[s]), s < n
 *   LKV_EPI_SWIGLU    n == 2, N[0] == N[1]: y[0] = fp16(fp16(silu(fp16 g)) * fp16 u)
 *                     for g, u the two products: HF MistralMLP's
 *                     act_fn(gate_proj(x)) * up_proj(x) (modeling_mistral.py:46-47)
 *   LKV_EPI_RESIDUAL  n == 1: y[0] = fp16(residual + fp16(product)), the decoder
 *                     layer's fp16 residual add (modeling_mistral.py:233, 239);
 *                     y[0] may be residual (in place), residual fp16 [B][N[0]]
 *   LKV_EPI_ROPE      n == 2 or 3 (q, k[, v]), N[0] and N[1] multiples of 128:
 *                     y[0], y[1] = HF's apply_rotary_pos_emb (modeling_mistral.py:
 *                     51-81, fp16 arithmetic as lkv_rope_f16) of the fp16 products'
 *                     heads of 128 dims at the position whose 128 fp16 factors
 *                     cos_row / sin_row hold; y[2] = the third product as it is
 * The q/k/v projections of an attention layer (leankv/teal/patching.py:169-180
 * runs them as three dense calls at B > 1) and the gate/up pair are the
 * products that share an input (and RoPE follows q and k).  w, thresholds and N are host arrays of n
 * entries, y of n (1 for LKV_EPI_SWIGLU); weights column-major as for
 * lkv_sparse_gemm_batched, outputs fp16 [B][N[s]].  Products whose
 * chunk sizes differ run as launches of their own.
 */
#define LKV_EPI_NONE 0
#define LKV_EPI_SWIGLU 1
#define LKV_EPI_RESIDUAL 2
#define LKV_EPI_ROPE 3
size_t lkv_sparse_gemm_batched_multi_workspace_bytes(int64_t B, int n, const int64_t* N, int64_t Z);
int lkv_sparse_gemm_batched_multi(const void* x, int64_t B, int n, const void* const* w, const float* thresholds,
                                  const int64_t* N, int64_t Z, int epilogue, const void* residual,
                                  const void* cos_row, const void* sin_row, void* const* y, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * The q, k and v products of lkv_sparse_gemm_batched_multi with LKV_EPI_ROPE
 * (w, thresholds, N and y host arrays of 3 entries), and, with k_hot / v_hot
 * non-null, the ring half of lkv_tq_cache_append (cache.py:84-141: the new
 * token enters the hot window): k (rotated) and v also go to ring slot
 * *pos % hot_cap of rows (batch b, kv head h) = b * N[1] / 128 + h of
 * k_hot / v_hot (fp16 [B * N[1] / 128][hot_cap][128]); a negative *pos
 * writes no ring slot.  With
 * lkv_tq_cache_evict run before it, the cache afterwards equals
 * lkv_tq_cache_append's on the same k and v.  No single reference
 * counterpart: the q/k/v calls of a decode layer at B > 1
 * (leankv/teal/patching.py:169-180), RoPE (modeling_mistral.py:51-81) and
 * TurboQuantCache.update's ring write.
 */
int lkv_sparse_gemm_batched_qkv_rope(const void* x, int64_t B, const void* const* w, const float* thresholds,
                                     const int64_t* N, int64_t Z, const void* cos_row, const void* sin_row,
                                     void* const* y, void* k_hot, void* v_hot, const int32_t* pos, int64_t hot_cap,
                                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * One batched_sparse_gemm product followed by the decoder layer's fp16
 * residual add and the next RMSNorm (no single reference counterpart: the
 * patched o_proj / down_proj call at B > 1, leankv/teal/patching.py:169-180,
 * then modeling_mistral.py:233 / 239 and the following MistralRMSNorm,
 * :190-197):
 *   x_out[b] = fp16(residual[b] + fp16(product[b]))   (x_out may be residual)
 *   y_out[b] = RMSNorm(x_out[b]) * norm_w             (lkv_rmsnorm's arithmetic)
 * x_out equals lkv_sparse_gemm_batched_multi's LKV_EPI_RESIDUAL output and
 * y_out lkv_rmsnorm of it, bit for bit; one launch does both after the
 * product, one block per batch row.  N % 8 == 0, N <= 8192; residual, x_out,
 * norm_w and y_out 16-byte aligned; workspace as for lkv_sparse_gemm_batched.
 */
int lkv_sparse_gemm_batched_residual_rmsnorm(const void* x, const void* w, float threshold, int64_t B, int64_t N,
                                             int64_t Z, const void* residual, const void* norm_w, float eps,
                                             void* x_out, void* y_out, void* workspace, size_t workspace_bytes,
                                             void* stream);

/* ------------------------------------------------------------------------ */
/* TurboQuant (MSE variant), head_dim 128                                    */
/* ------------------------------------------------------------------------ */

/* Bytes of one packed code row for `bits` (1..4) at dim 128: 16, 32, 64, 64. */
int lkv_tq_packed_row_bytes(int bits);

/*
 * TurboQuantMSE.quantize (leankv/turboquant/quantizer.py:119-129):
 *   n = ||x||;  u = x / (n + 1e-10);  y = float(u) @ Pi^T;
 *   idx = #{b in bounds : b < y}   (torch.searchsorted, right=False);
 *   packed = _pack_indices(idx, bits)   (quantizer.py:38-62)
 * x: [M, 128], dtype LKV_DTYPE_F32 or LKV_DTYPE_F16 (the norm, the division
 * and its rounding follow x's dtype, as in torch).  Pi: fp32 [128, 128]
 * row-major.  bounds: fp32 decision boundaries, 2^bits - 1 of them
 * (boundaries[1:-1], quantizer.py:115-117).  packed: uint8 [M, row_bytes].
 * norms: [M] of x's dtype.  The rotation runs on fp32 MFMA.
 */
int lkv_tq_quantize(const void* x, int x_dtype, int64_t M, const float* Pi,
                    const float* bounds, int bits, uint8_t* packed, void* norms,
                    void* stream);

/*
 * The searchsorted + pack half of quantize on an already rotated fp32 y
 * [M, 128] (quantizer.py:126-127).  Exact on every element.
 */
int lkv_tq_quantize_rotated(const float* y, int64_t M, const float* bounds,
                            int bits, uint8_t* packed, void* stream);

/*
 * TurboQuantMSE.dequantize (quantizer.py:131-137):
 *   x_hat = (centroids[unpack(packed)] @ Pi) * norm
 * packed uint8 [M, row_bytes]; norms [M] of norm_dtype; centroids fp32
 * [2^bits]; out [M, 128] of out_dtype (LKV_DTYPE_F16 reproduces the cache's
 * `.to(float16)` of cache.py:176-181).  fp32 MFMA.
 */
int lkv_tq_dequantize(const uint8_t* packed, const void* norms, int norm_dtype,
                      int64_t M, const float* Pi, const float* centroids, int bits,
                      void* out, int out_dtype, void* stream);

/*
 * rotate_forward / rotate_backward (leankv/turboquant/rotation.py:45-52):
 *   transpose == 0:  y = x @ Pi^T        transpose == 1:  y = x @ Pi
 * x [M, 128] (F32 or F16), y fp32 [M, 128].  fp32 MFMA.
 */
int lkv_tq_rotate(const void* x, int x_dtype, int64_t M, const float* Pi,
                  int transpose, float* y, void* stream);

/*
 * TurboQuantProd.quantize (leankv/turboquant/quantizer.py:206-222), one launch:
 *   codes, norms = TurboQuantMSE(mse_bits).quantize(x)       (as lkv_tq_quantize)
 *   x_hat = (centroids[codes] @ Pi) * norm;  r = x - x_hat      (fp32)
 *   rnorms = ||r||;  signs: bit i of byte j = [(r @ S^T)[8j + i] > 0]
 *                                              (_pack_qjl_signs, :181-194)
 * x [M, 128] (F32 or F16); Pi and S fp32 [128, 128] row-major (S is
 * generate_qjl_matrix(128, seed + 1000), rotation.py:32-42); bounds fp32
 * [2^mse_bits - 1]; centroids fp32 [2^mse_bits]; codes uint8 [M, row_bytes
 * of mse_bits]; norms [M] of x's dtype; signs uint8 [M, 16]; rnorms fp32 [M].
 * mse_bits = TurboQuantProd bits - 1, 1..4.  Codes equal lkv_tq_quantize's
 * and the signs equal those of lkv_tq_rotate(x - lkv_tq_dequantize(...), S),
 * bit for bit.  fp32 MFMA.
 */
int lkv_tq_prod_quantize(const void* x, int x_dtype, int64_t M, const float* Pi,
                         const float* bounds, const float* centroids, const float* S,
                         int mse_bits, uint8_t* codes, void* norms, uint8_t* signs,
                         float* rnorms, void* stream);

/*
 * TurboQuantProd.dequantize (quantizer.py:224-237), one launch:
 *   out = (centroids[codes] @ Pi) * norm + (s @ S) * (qjl_scale * rnorm)
 * with s = +1 / -1 from the sign bits (_unpack_qjl_signs, :196-204) and
 * qjl_scale = sqrt(pi / 2) / 128 for the reference's estimator.  Shapes as
 * lkv_tq_prod_quantize; norms of norm_dtype; out [M, 128] of out_dtype.
 */
int lkv_tq_prod_dequantize(const uint8_t* codes, const void* norms, int norm_dtype,
                           const uint8_t* signs, const float* rnorms, int64_t M,
                           const float* Pi, const float* centroids, const float* S,
                           int mse_bits, float qjl_scale, void* out, int out_dtype,
                           void* stream);

/*
 * Decode-step cache append of TurboQuantCache.update for one layer
 * (leankv/turboquant/cache.py:84-159) on a static ring layout.
 * Current length before the append is *pos (device int32, read by the
 * kernel, never written).  The hot window keeps the last `hot_cap` tokens in
 * fp16 ring slots (token p lives in slot p % hot_cap); when pos >= hot_cap
 * the token that leaves the window (p = pos - hot_cap) is quantized from its
 * fp16 slot, widened to fp32 as cache.py:141-142 does, into cold row p;
 * then the new token is written into slot pos % hot_cap.
 *   k_new, v_new: fp16 [R, 128]       (R = batch * kv_heads)
 *   k_hot, v_hot: fp16 [R, hot_cap, 128]
 *   k_codes, v_codes: uint8 [R, cap, row_bytes];  k_norms, v_norms: fp32 [R, cap]
 *   PiK, PiV: fp32 [128,128]; bounds fp32 [2^bits - 1]
 * Rows beyond `cap` are never written: a call with pos - hot_cap >= cap
 * skips the quantize (the host must size cap for the whole sequence); a
 * negative *pos writes nothing.
 */
int lkv_tq_cache_append(const void* k_new, const void* v_new, void* k_hot, void* v_hot,
                        uint8_t* k_codes, float* k_norms, uint8_t* v_codes, float* v_norms,
                        const float* PiK, const float* PiV, const float* bounds, int bits,
                        const int32_t* pos, int64_t R, int64_t hot_cap, int64_t cap,
                        void* stream);

/*
 * Decode attention (q_len 1) over a TurboQuant cache, reading packed codes
 * directly.  Equals SDPA over cat(dequantize(cold).fp16, hot) as built by
 * TurboQuantCache._get_full_cache (cache.py:169-189) and consumed by
 * transformers/integrations/sdpa_attention.py:79-105 (GQA, no mask), but never
 * materialises the dequantized K/V:
 *   s_t = scale * n_t * ((q @ PiK^T) . c[idx_t])     for cold tokens
 *   o   = (sum_t p_t n_t c[idx_t]) @ PiV + sum_hot p_t v_t
 * q: fp16 [B, Hq, 128]; codes uint8 [B, Hkv, cap, row_bytes] in the packing of
 * lkv_tq_quantize (row_bytes = lkv_tq_packed_row_bytes(bits): 64 for 3 and 4
 * bits, 32 for 2, 16 for 1); norms fp32 [B, Hkv, cap]; hot fp16
 * [B, Hkv, hot_cap, 128] ring as in lkv_tq_cache_append, hot_cap 1..256.  The current length L = *seq_len (device
 * int32, includes every token already appended); cold tokens are
 * [0, max(0, L - hot_cap)), hot tokens the rest.  max_len (host) bounds L and
 * sizes the launch; L > max_len is clamped to max_len.  out: fp16 [B, Hq, 128].
 * Hq must be a multiple of Hkv with Hq / Hkv <= 16.
 */
size_t lkv_tq_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len);
int lkv_tq_decode_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                       const uint8_t* v_codes, const float* v_norms,
                       const void* k_hot, const void* v_hot,
                       const float* PiK, const float* PiV, const float* centroids, int bits,
                       const int32_t* seq_len, int64_t max_len,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t hot_cap,
                       float scale, void* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Causal prefill attention (S >= 1 new queries) over a TurboQuant cache,
 * reading packed codes directly.  Equals HF SDPA with the causal mask over
 * cat(dequantize(cold).fp16, hot) as TurboQuantCache.update returns it for an
 * update of several tokens (cache.py:119-125, 169-189;
 * transformers/integrations/sdpa_attention.py:79-105), without materialising
 * the dequantized K/V.  The cache holds kv_len tokens (every new token already
 * appended): cold tokens [0, max(0, kv_len - hot_cap)) as codes, the rest in
 * the hot ring (token t in slot t % hot_cap).  The S queries are the newest S
 * tokens: query i sits at position kv_len - S + i and sees keys
 * 0 .. kv_len - S + i.
 *   s_t = scale * n_t * ((q @ PiK^T) . c[idx_t])       cold keys
 *   s_t = scale * (q @ PiK^T) . fp16(k_t @ PiK^T)       hot keys
 *   o   = (sum_t p_t n_t c[idx_t] + sum_hot p_t fp16(v_t @ PiV^T)) @ PiV
 * q: fp16 [B, Hq, S, 128] (post-RoPE); codes uint8 [B, Hkv, cap, row_bytes]
 * (row_bytes as for lkv_tq_decode_attn, bits 1..4); norms fp32 [B, Hkv, cap];
 * hot fp16 [B, Hkv, hot_cap, 128];
 * out fp16 [B, Hq, S, 128].  Hq / Hkv must be 1, 2, 4, 8 or 16.  The workspace
 * holds the two hot rings rotated into the key / value domains.
 */
size_t lkv_tq_prefill_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hot_cap);
int lkv_tq_prefill_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                        const uint8_t* v_codes, const float* v_norms,
                        const void* k_hot, const void* v_hot,
                        const float* PiK, const float* PiV, const float* centroids, int bits,
                        int64_t kv_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                        int64_t cap, int64_t hot_cap, float scale, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Batch decode attention over a paged fp16 KV pool (one layer), the kernel
 * PagedKVCache.decode_attention runs (leankv/turboquant/paged_cache.py:194-257,
 * there FlashInfer BatchDecodeWithPagedKVCacheWrapper, NHD layout, no
 * positional encoding).  kv_data: fp16 [max_pages][2 (K, V)][page_size][Hkv][128];
 * sequence b owns pages kv_indices[kv_indptr[b] .. kv_indptr[b + 1]) (int32,
 * device) and its last page holds kv_last_page_len[b] tokens (1 .. page_size).
 * q fp16 [B, Hq, 128] -> out fp16 [B, Hq, 128] = softmax(q K^T * scale) V,
 * query head h reading kv head h / (Hq / Hkv), Hq / Hkv <= 16.  max_len (host)
 * bounds every sequence length and sizes the launch.  Page ids outside
 * [0, max_pages) are clamped; kv_indptr must index inside kv_indices.
 */
size_t lkv_paged_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len);
int lkv_paged_decode_attn(const void* q, const void* kv_data, const int32_t* kv_indptr,
                          const int32_t* kv_indices, const int32_t* kv_last_page_len,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t page_size, int64_t max_pages,
                          int64_t max_len, float scale, void* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Decode attention over a PAGED packed (TurboQuant) cache, one layer.  No
 * counterpart in the reference, whose paged cache (paged_cache.py:32-362) is
 * fp16: this is lkv_tq_decode_attn with the cold store in pages, for ragged
 * batches that grow and free pages independently.  Same math as
 * lkv_tq_decode_attn (cache.py:169-189 semantics + sdpa_attention.py:79-105).
 *   k_codes, v_codes: uint8 [max_pages, Hkv, page_size, row_bytes] (row_bytes
 *   = lkv_tq_packed_row_bytes(bits), bits 1..4)
 *   k_norms, v_norms: fp32  [max_pages, Hkv, page_size]
 *   sequence b's cold token t (t < seq_lens[b] - hot_cap) lies in page
 *   kv_indices[kv_indptr[b] + t / page_size], slot t % page_size (FlashInfer's
 *   CSR page table, int32 device arrays);
 *   k_hot, v_hot: fp16 [B, Hkv, hot_cap, 128] rings (token t in slot t % hot_cap,
 *   hot_cap 1..256);
 *   seq_lens: int32 [B] on the device, each <= max_len.
 * page_size 16, 32, 64 or 128; the code pool below 2^32 bytes.  Page ids are
 * clamped to the pool and tokens past a sequence's pages are not read.
 */
size_t lkv_tq_paged_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len,
                                                int64_t page_size);
int lkv_tq_paged_decode_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                             const uint8_t* v_codes, const float* v_norms, const void* k_hot,
                             const void* v_hot, const float* PiK, const float* PiV,
                             const float* centroids, int bits, const int32_t* kv_indptr,
                             const int32_t* kv_indices, const int32_t* seq_lens, int64_t B,
                             int64_t Hq, int64_t Hkv, int64_t page_size, int64_t max_pages,
                             int64_t max_len, int64_t hot_cap, float scale, void* out,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused B=1 decode step                                                     */
/* ------------------------------------------------------------------------ */

/*
 * One greedy decode step of a Mistral/Llama-shaped decoder (head_dim 128) with
 * TEAL sparse projections and a TurboQuant cache, as a fixed sequence of
 * launches on device-resident state, so that it can be captured into a HIP
 * graph and replayed per token.  No single reference function corresponds:
 * the step runs, per layer, what the reference executes through HF
 * MistralDecoderLayer (transformers/models/mistral/modeling_mistral.py) with
 * every projection patched by _patch_linear_with_triton
 * (leankv/teal/patching.py:152-183), keys/values going through
 * TurboQuantCache.update (leankv/turboquant/cache.py:84-189) and attention
 * over its output; then the final RMSNorm, the dense lm_head and argmax of
 * scripts/benchmark.py's greedy loop.  Per step, before the layers,
 * lkv_decode_evict quantizes the token leaving every layer's hot window
 * (lkv_tq_cache_append arithmetic).  Per layer (8 launches):
 *   1. q/k/v GEMV, RMSNorm(x) computed in the prologue;
 *   2-3. packed-KV attention split + combine (lkv_tq_decode_attn kernels);
 *      the split kernel's prologue reduces the q/k/v partials, applies RoPE,
 *      rotates q (the arithmetic of lkv_tq_decode_attn's own rotation) and
 *      writes the new token's key and value to the hot ring;
 *   4. o_proj GEMV;  5. x += o (fp16 residual);
 *   6. gate/up GEMV, RMSNorm(x) in the prologue;
 *   7. down GEMV, SwiGLU of the gate/up partials in the prologue;
 *   8. x += down.
 * Rounding follows the fp16 HF modules: projections, RMSNorm output, RoPE
 * products and sums, SwiGLU and residual adds are rounded to fp16 where HF
 * stores fp16 tensors.  A threshold of 0 keeps every nonzero input (dense).
 *
 * Weights are fp16 in the column-major layout of lkv_sparse_gemv (row z holds
 * the N weights of input z), including lm_head ([hidden][vocab]).
 * Device state: tok (int64, the token fed next) and pos (int64, its
 * position); lkv_decode_head writes the argmax into tok and increments pos.
 * Positions at or beyond max_len are clamped (results are then meaningless);
 * the caller bounds the number of steps.
 */
typedef struct lkv_decode_dims {
  int64_t hidden;        /* model width, multiple of 256 */
  int64_t ffn;           /* MLP width, multiple of 256 */
  int64_t vocab;         /* multiple of 8 */
  int64_t n_heads;       /* query heads */
  int64_t n_kv_heads;    /* n_heads / n_kv_heads <= 8 */
  int64_t max_len;       /* RoPE table rows; tokens the cache holds */
  int64_t cap;           /* cold rows per (layer, kv head) */
  int64_t hot_cap;       /* fp16 window, 1..256 */
  int32_t bits;          /* 1..4 (the packings of quantizer.py:38-62) */
  float eps;             /* RMSNorm epsilon */
  float scale;           /* attention scale */
  const float* bounds;   /* 2^bits - 1 decision boundaries (fp32) */
  const float* centroids;/* 2^bits centroids (fp32) */
  const void* rope_cos;  /* fp16 [max_len][128] */
  const void* rope_sin;  /* fp16 [max_len][128] */
} lkv_decode_dims;

typedef struct lkv_decode_layer {
  const void* input_norm;  /* fp16 [hidden] */
  const void* post_norm;   /* fp16 [hidden] */
  const void* wq;          /* [hidden][n_heads * 128] */
  const void* wk;          /* [hidden][n_kv_heads * 128] */
  const void* wv;
  const void* wo;          /* [n_heads * 128][hidden] */
  const void* wg;          /* [hidden][ffn] */
  const void* wu;
  const void* wd;          /* [ffn][hidden] */
  float tq, tk, tv, to, tg, tu, td;  /* TEAL thresholds */
  void* k_codes;           /* uint8 [n_kv_heads, cap, 64] */
  void* k_norms;           /* fp32 [n_kv_heads, cap] */
  void* v_codes;
  void* v_norms;
  void* k_hot;             /* fp16 [n_kv_heads, hot_cap, 128] ring */
  void* v_hot;
  const float* PiK;        /* fp32 [128, 128] */
  const float* PiV;
} lkv_decode_layer;

/*
 * The eviction half of lkv_tq_cache_append for every layer of a decode step
 * in one launch (cache.py:84-141: once the window holds hot_cap tokens, the
 * oldest is quantized into the cold store): at position *pos (device int32,
 * the position of the token this step feeds) the token pos - hot_cap leaves
 * ring slot pos % hot_cap of each of the R rows (batch x kv head) of each
 * layer and its codes and norms go to cold slot pos - hot_cap (nothing when
 * pos < hot_cap or pos - hot_cap >= cap).  The codes and norms equal
 * lkv_tq_cache_append's.  Run it before the step writes its new token into
 * the ring (lkv_sparse_gemm_batched_qkv_rope does, as the append's second
 * half).  Buffers as for lkv_tq_cache_append, codes 16-byte aligned; layers
 * is a host array of n_layers entries.
 */
typedef struct lkv_cache_layer {
  void* k_codes;       /* uint8 [R, cap, row bytes] */
  void* k_norms;       /* fp32 [R, cap] */
  void* v_codes;
  void* v_norms;
  const void* k_hot;   /* fp16 [R, hot_cap, 128] ring */
  const void* v_hot;
  const float* PiK;    /* fp32 [128, 128] */
  const float* PiV;
} lkv_cache_layer;
int lkv_tq_cache_evict(const lkv_cache_layer* layers, int64_t n_layers, int64_t R, int64_t hot_cap, int64_t cap,
                       const float* bounds, int bits, const int32_t* pos, void* stream);

/*
 * y = RMSNorm(x) * w for M rows of Z fp16 values (x 16-byte aligned, Z % 8 == 0):
 * HF MistralRMSNorm (modeling_mistral.py:190-197) with the summation order of
 * the RMSNorm fused into lkv_decode_layer_step's GEMV prologues, so a caller
 * gets bit-identical normalised activations (and therefore identical TEAL
 * masks) outside the fused step.
 */
int lkv_rmsnorm(const void* x, const void* w, float eps, int64_t M, int64_t Z, void* y, void* stream);

/*
 * RoPE of B decode rows in place, one launch for the query and the key:
 * q fp16 [B][Hq][128], k fp16 [B][Hkv][128] (contiguous), cos_row / sin_row
 * the 128 fp16 factors of the tokens' position.  HF apply_rotary_pos_emb on
 * fp16 tensors (transformers/models/mistral/modeling_mistral.py:51-81,
 * x * cos + rotate_half(x) * sin, each product and the sum rounded to fp16)
 * bit for bit, the arithmetic of the fused step's split prologue.
 * B * (Hq + Hkv) < 2^24.
 */
int lkv_rope_f16(void* q, void* k, const void* cos_row, const void* sin_row, int64_t B, int64_t Hq, int64_t Hkv,
                 void* stream);

/* Workspace shared by the four calls below (no initialisation needed).
 * A step is: lkv_decode_begin, lkv_decode_evict, lkv_decode_layer_step per
 * layer, lkv_decode_head, all on one stream. */
size_t lkv_decode_workspace_bytes(const lkv_decode_dims* dims);
/* Where the step leaves its intermediate results in the workspace (byte
 * offsets from its start), for callers that read a layer's projections after
 * lkv_decode_layer_step: the split-K partial sums of every GEMV, fp32
 * [slab][chunk][256] per matrix (slab = output column / 256; summing a
 * column's chunks in chunk order from 0 and rounding to fp16 gives the
 * projection, as for lkv_sparse_gemv_partials), the RoPE'd query and the
 * attention output (fp16 [n_heads * 128]).  They hold the last call's values
 * until the next call overwrites them.  No reference counterpart: it exposes
 * what the reference's per-projection calls (leankv/teal/patching.py:169-180)
 * return one by one. */
typedef struct lkv_decode_layout {
  size_t part_q, part_k, part_v; /* q|k|v GEMV, one region per segment */
  size_t part_o;                 /* o_proj */
  size_t part_gate, part_up;     /* gate|up */
  size_t part_down;              /* down */
  size_t part_lm;                /* lm_head (lkv_decode_head) */
  size_t q_rope;                 /* fp16 query after RoPE */
  size_t attn_out;               /* fp16 attention output (o_proj input) */
  size_t total;                  /* = lkv_decode_workspace_bytes */
  int32_t chunks_qkv, chunks_o, chunks_gateup, chunks_down, chunks_lm;
} lkv_decode_layout;
int lkv_decode_workspace_layout(const lkv_decode_dims* dims, lkv_decode_layout* layout);
/* x = embed[tok] (embed fp16 [vocab][hidden] row-major); latches pos. */
int lkv_decode_begin(const lkv_decode_dims* dims, const void* embed, const int64_t* tok, const int64_t* pos,
                     void* x, void* workspace, size_t workspace_bytes, void* stream);
/* The token leaving every layer's hot window at the latched position
 * (cache.py:84-141 `_flush_to_cold`: once the window exceeds hot_cap its
 * oldest token is quantized to the cold store): for each of the n_layers
 * layers (host array; only the cache fields and PiK / PiV are read), token
 * pos - hot_cap is read from ring slot pos % hot_cap, quantized with the
 * layer's rotation and written to cold slot pos - hot_cap, with the codes of
 * lkv_tq_cache_append.  Must run after lkv_decode_begin and before the
 * step's first lkv_decode_layer_step (which overwrites that ring slot). */
int lkv_decode_evict(const lkv_decode_dims* dims, const lkv_decode_layer* layers, int64_t n_layers,
                     void* workspace, size_t workspace_bytes, void* stream);
/* One decoder layer on the fp16 residual stream x [hidden], in place; the
 * step's new key / value enter the hot ring (eviction is lkv_decode_evict's). */
int lkv_decode_layer_step(const lkv_decode_dims* dims, const lkv_decode_layer* layer, void* x,
                          void* workspace, size_t workspace_bytes, void* stream);
/* The same decoder layer with a plain fp16 KV cache instead of the TurboQuant
 * one: the dense-fp16 decode that the reference's baseline runs
 * (scripts/raw_baseline.py:33-62: HF decode with an fp16 DynamicCache), on
 * this library's kernels (with every TEAL threshold 0 the projections are
 * dense).  The step's key and value are RoPE'd as in lkv_decode_layer_step and
 * written to kv_pool, fp16 [ceil(max_len / 16)][2 (K, V)][16][n_kv_heads][128]
 * (token t in page t / 16, slot t % 16, the layout of lkv_paged_decode_attn),
 * and the layer attends to tokens 0 .. pos as lkv_paged_decode_attn does over
 * identity pages (with at most 4 query heads per kv head the split kernel sums
 * the projection partials and writes the new token itself).  The cache fields of
 * `layer` are not read; lkv_decode_evict is not needed. */
int lkv_decode_layer_step_f16kv(const lkv_decode_dims* dims, const lkv_decode_layer* layer, void* kv_pool, void* x,
                                void* workspace, size_t workspace_bytes, void* stream);
/* logits = lm_head(RMSNorm(x) * final_norm) (fp16 [vocab]); tok = argmax
 * (lowest index among equal maxima); pos += 1. */
/* tok_history (optional, int64 [history_len] on the device): the step at
 * position p also writes its token to tok_history[p] (p < history_len), so a
 * replayed decode loop keeps every token without a copy per step. */
int lkv_decode_head(const lkv_decode_dims* dims, const void* final_norm, const void* lm_head, const void* x,
                    void* logits, int64_t* tok, int64_t* pos, int64_t* tok_history, int64_t history_len,
                    void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LEANKV_AMD_H */
