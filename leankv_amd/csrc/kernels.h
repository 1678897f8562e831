// Internal interfaces shared by the kernel translation units: the sparse GEMV
// launcher with its input prologues, the split-K partial-sum layout, and the
// packed-KV attention launcher.  Not part of the C ABI.
#pragma once

#include "common.h"

namespace lkv {

// ------------------------------------------------------------------ GEMV
// A GEMV launch covers column slabs of kGemvBN outputs x row chunks of BZ
// inputs.  Each (slab, chunk) block writes kGemvBN fp32 partial sums; the sum
// over chunks, in chunk order, happens in a consumer.  Partials of one matrix
// are laid out [slab][chunk][kGemvBN].
constexpr int kGemvThreads = 256;
constexpr int kGemvBN = 256;
constexpr int kMaxSeg = 3;

enum GemvIn {
  kInRaw = 0,      // x fp16 as given
  kInRmsNorm = 1,  // x = RMSNorm(x_resid) * norm_w, computed per block
  kInSwiglu = 2,   // x = SwiGLU(gate, up), gate/up summed from partials
};

struct GemvArgs {
  const uint16_t* x;       // kInRaw / kInRmsNorm: fp16 [Z], 16-byte aligned
  const uint16_t* norm_w;  // kInRmsNorm: fp16 [Z]
  float eps;
  const float* in_part;    // kInSwiglu: [2][in_nslab][in_nchunk][kGemvBN] (gate, then up)
  int in_nslab, in_nchunk;
  // Segments: weight matrices that share x, each [Z][N[s]] column-major fp16
  // (row z = the N[s] weights of input z).  Global column slab g belongs to
  // segment s when slab0[s] <= g < slab0[s + 1].
  int nseg;
  const uint16_t* A[kMaxSeg];
  const uint16_t* A_up;    // dual mode: the up matrix, same shape as A[0]
  uint32_t a_bytes[kMaxSeg];
  int N[kMaxSeg];
  float t[kMaxSeg];
  float t_up;
  int slab0[kMaxSeg + 1];
  int slab0_seg[kMaxSeg];  // slab0[0 .. kMaxSeg) as set by gemv_launch (selected without dynamic indexing)
  int Z, nchunk;
  float* part;             // partials of segment s at part + part_off[s]
  size_t part_off[kMaxSeg];
  size_t part_up_off;      // dual mode: the up matrix's partials
  uint16_t* y;             // non-null only when nchunk == 1 and nseg == 1: write fp16 (SwiGLU if dual)
  int chunk_major;         // set by gemv_launch (block order)
};

int gemv_pick_bz(int64_t slabs, int64_t Z, int quarter_blocks = 3);
int gemv_launch(const GemvArgs& G, int bz, bool dual, int mode, int nslab_total, hipStream_t st);

inline int64_t gemv_slabs(int64_t N) { return (N + kGemvBN - 1) / kGemvBN; }
inline int64_t gemv_chunks(int64_t Z, int bz) { return Z > 0 ? (Z + bz - 1) / bz : 1; }
inline size_t gemv_part_floats(int64_t N, int64_t nchunk) {
  return static_cast<size_t>(gemv_slabs(N)) * nchunk * kGemvBN;
}

// Column n of a [slab][chunk][kGemvBN] partial array summed over chunks in
// chunk order, starting from 0.  Loads are issued 16 at a time.
__device__ __forceinline__ float column_sum(const float* __restrict__ P, int n, int nchunk) {
  constexpr int kBatch = 32;
  const float* p = P + static_cast<size_t>(n / kGemvBN) * nchunk * kGemvBN + (n % kGemvBN);
  float s = 0.f;
  for (int k0 = 0; k0 < nchunk; k0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) v[i] = (k0 + i < nchunk) ? p[static_cast<size_t>(k0 + i) * kGemvBN] : 0.f;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) s += v[i];
  }
  return s;
}

// Columns n0 and n1 of a [slab][chunk][kGemvBN] GEMV partial array, each
// summed over the chunks in chunk order from 0 (column_sum's order), with the
// loads of both columns in flight together.
__device__ __forceinline__ void column_sum2(const float* __restrict__ P, int n0, int n1, int nchunk, float& s0,
                                            float& s1) {
  constexpr int kB = 16;
  const float* p0 = P + static_cast<size_t>(n0 / kGemvBN) * nchunk * kGemvBN + (n0 % kGemvBN);
  const float* p1 = P + static_cast<size_t>(n1 / kGemvBN) * nchunk * kGemvBN + (n1 % kGemvBN);
  s0 = 0.f;
  s1 = 0.f;
  for (int k0 = 0; k0 < nchunk; k0 += kB) {
    float a[kB], c[kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const size_t o = static_cast<size_t>(min(k0 + i, nchunk - 1)) * kGemvBN;
      a[i] = p0[o];
      c[i] = p1[o];
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      s0 += k0 + i < nchunk ? a[i] : 0.f;
      s1 += k0 + i < nchunk ? c[i] : 0.f;
    }
  }
}

// RoPE of the dim pair (d, d + 64) of an fp16 row, x * cos + rotate_half(x) *
// sin with fp16 products and sum (apply_rotary_pos_emb on fp16 tensors,
// modeling_mistral.py); x0, x1 are the fp32 projection sums, rounded to fp16
// first as the fp16 projection output is.  Each product is rounded to fp16
// before the sum: contraction is off here, since the compiler otherwise turns
// the fp16 product and the fp32 add into one fma and skips that rounding.
__device__ __forceinline__ void rope_pair_v(float x0, float x1, uint16_t cos0, uint16_t cos1, uint16_t sin0,
                                            uint16_t sin1, float& o0, float& o1) {
#pragma clang fp contract(off)
  const float a = h2f(f2h(x0)), c = h2f(f2h(x1));
  const float c0 = h2f(cos0), c1 = h2f(cos1);
  const float s0 = h2f(sin0), s1 = h2f(sin1);
  o0 = h2f(f2h(h2f(f2h(a * c0)) + h2f(f2h(-c * s0))));
  o1 = h2f(f2h(h2f(f2h(c * c1)) + h2f(f2h(a * s1))));
}
__device__ __forceinline__ void rope_pair(float x0, float x1, const uint16_t* __restrict__ cos_row,
                                          const uint16_t* __restrict__ sin_row, int d, float& o0, float& o1) {
  rope_pair_v(x0, x1, cos_row[d], cos_row[d + 64], sin_row[d], sin_row[d + 64], o0, o1);
}

// 1 / sqrt(mean(x^2) + eps) over fp16 x[0..Z) in fp32, computed by a whole
// block (every thread gets the result).  Fixed summation order, the same for
// any block size: thread t < 256 accumulates x[8t .. 8t+7], x[8t + 2048 ..],
// ... with fmaf, then a wave butterfly, then the 4 wave sums in order
// (threads >= 256 of a larger block take no part).  Requires Z % 8 == 0 and
// 16-byte aligned x.  Every RMSNorm of this library goes through it, so all
// of them round identically.
__device__ __forceinline__ float rms_rstd(const uint16_t* __restrict__ x, int Z, float eps, float* s_wsum) {
  const int tid = threadIdx.x;
  constexpr int kStride = kGemvThreads * 8;
  constexpr int kBatch = 4;  // vectors up to kBatch * kStride: every load issued before the first is used
  float ss = 0.f;
  if (tid < kGemvThreads) {
    if (Z <= kBatch * kStride) {
      uint4 u[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) u[k] = *reinterpret_cast<const uint4*>(x + min(tid * 8 + k * kStride, Z - 8));
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const bool ok = tid * 8 + k * kStride < Z;
        const uint32_t w[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = h2f(static_cast<uint16_t>(w[i] & 0xffffu));
          const float b = h2f(static_cast<uint16_t>(w[i] >> 16));
          ss = ok ? fmaf(a, a, ss) : ss;
          ss = ok ? fmaf(b, b, ss) : ss;
        }
      }
    } else {
      for (int z = tid * 8; z < Z; z += kStride) {
        const uint4 u = *reinterpret_cast<const uint4*>(x + z);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = h2f(static_cast<uint16_t>(w[i] & 0xffffu));
          const float b = h2f(static_cast<uint16_t>(w[i] >> 16));
          ss = fmaf(a, a, ss);
          ss = fmaf(b, b, ss);
        }
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & (kWave - 1)) == 0 && tid < kGemvThreads) s_wsum[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kGemvThreads / kWave; ++w) tot += s_wsum[w];
  return rsqrtf(tot / static_cast<float>(Z) + eps);
}

// HF MistralRMSNorm output element (modeling_mistral.py:190-197): x * rstd in
// fp32 cast to fp16, times the fp16 weight, product rounded to fp16.  The
// fp32 product goes through an empty asm so that it exists as an fp32 value:
// the compiler otherwise selects one fp16-output fma for product and cast
// (v_fma_mixlo_f16: one rounding of the exact product instead of two) in some
// kernels and not in others, depending on how it vectorises the element loop,
// and two kernels' norms of one row then differ in rare elements.
__device__ __forceinline__ float rms_apply(uint16_t x, uint16_t w, float rstd) {
  float t = h2f(x) * rstd;
  __asm__ volatile("" : "+v"(t));
  return h2f(f2h(h2f(w) * h2f(f2h(t))));
}

// SwiGLU with the rounding of the eager fp16 torch sequence of
// transformers/models/mistral/modeling_mistral.py:46-47 on fp16 projection
// outputs: silu(fp16 g) -> fp16, times fp16 u -> fp16.
__device__ __forceinline__ uint16_t swiglu_f16(float g, float u) {
  const float g16 = h2f(f2h(g));
  const float u16 = h2f(f2h(u));
  const float s16 = h2f(f2h(g16 / (1.0f + expf(-g16))));
  return f2h(s16 * u16);
}

// ------------------------------------------------------------- attention
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// q_rot = q @ PiK^T for the query heads (at most 16) of one kv head: the one
// arithmetic of the attention's rotated query, shared by the split kernel
// and the decode step so both give identical bits.  PiK is split into
// hi = fp16(x) (toward zero) and lo = fp16((x - hi) * 2^11) (toward zero),
// q is fp16, so both products run on v_mfma_f32_16x16x32_f16 with exact
// fp32 products: q_rot = acc_hi + acc_lo * 2^-11, error ~2^-20 relative.
// The tile is transposed (rows = output dims, columns = heads).  Wave w
// covers input dims 32w .. 32w+31 (lane group g' holding 32w + 8g' .. +7)
// for 8 output tiles; tile c row r is output dim 32(r/4) + 4c + r%4, so lane
// (h = lane%16, g = lane/16) ends with dims 32g .. 32g+31 of head h.  The 4
// wave partials are summed through LDS in the fixed order ((w0+w1)+w2)+w3.
// Called by all 4 waves of a 256-thread block (one __syncthreads inside).
//   qb   this lane's q[h][32w + 8g .. +7] as fp16 pairs (zero for unused h)
//   part LDS scratch, 4 x 16 rows of `ld` floats (ld >= 128, ld % 4 == 0)
//   out  out[i] = q_rot[h][32g + 4i .. 4i+3]
// The PiK operand of rotate_query_hilo, loadable ahead of the query (the
// decode step issues it before summing the query's partials).
__device__ __forceinline__ void load_pik_operand(const float* __restrict__ PiK, int wave, int lane,
                                                 float4 (&pa)[8][2]) {
  const int h = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int row = 32 * (h >> 2) + 4 * c + (h & 3);  // lane % 16 is the A row here
    const float4* src = reinterpret_cast<const float4*>(PiK + row * 128 + 32 * wave + 8 * g);
    pa[c][0] = src[0];
    pa[c][1] = src[1];
  }
}

__device__ __forceinline__ void rotate_query_hilo_loaded(const float4 (&pa)[8][2], const u32x4& qb, int wave,
                                                         int lane, float* part, int ld, float4 (&out)[8]) {
  const int h = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float x[8] = {pa[c][0].x, pa[c][0].y, pa[c][0].z, pa[c][0].w,
                        pa[c][1].x, pa[c][1].y, pa[c][1].z, pa[c][1].w};
    u32x4 hi, lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const auto hp = __builtin_amdgcn_cvt_pkrtz(x[2 * j], x[2 * j + 1]);
      const float r0 = (x[2 * j] - static_cast<float>(hp[0])) * 2048.f;
      const float r1 = (x[2 * j + 1] - static_cast<float>(hp[1])) * 2048.f;
      hi[j] = __builtin_bit_cast(uint32_t, hp);
      lo[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
    }
    const f32x4 ah = mfma16x16x32(hi, qb, f32x4{0.f, 0.f, 0.f, 0.f});
    const f32x4 al = mfma16x16x32(lo, qb, f32x4{0.f, 0.f, 0.f, 0.f});
    *reinterpret_cast<float4*>(part + (wave * 16 + h) * ld + 32 * g + 4 * c) =
        make_float4(fmaf(al[0], 1.f / 2048.f, ah[0]), fmaf(al[1], 1.f / 2048.f, ah[1]),
                    fmaf(al[2], 1.f / 2048.f, ah[2]), fmaf(al[3], 1.f / 2048.f, ah[3]));
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float4 p[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) p[w] = *reinterpret_cast<const float4*>(part + (w * 16 + h) * ld + 32 * g + 4 * i);
    out[i] = make_float4(((p[0].x + p[1].x) + p[2].x) + p[3].x, ((p[0].y + p[1].y) + p[2].y) + p[3].y,
                         ((p[0].z + p[1].z) + p[2].z) + p[3].z, ((p[0].w + p[1].w) + p[2].w) + p[3].w);
  }
}

__device__ __forceinline__ void rotate_query_hilo(const float* __restrict__ PiK, const u32x4& qb, int wave,
                                                  int lane, float* part, int ld, float4 (&out)[8]) {
  float4 pa[8][2];
  load_pik_operand(PiK, wave, lane, pa);
  rotate_query_hilo_loaded(pa, qb, wave, lane, part, ld, out);
}

// y = x @ Pi^T (transpose 0) or x @ Pi (transpose 1) for M rows of 128, fp32
// MFMA (the lkv_tq_rotate kernel); x and y fp32 or fp16.
int rotate_rows(const void* x, bool x_f16, int64_t M, const float* Pi, int transpose, void* y, bool y_f16,
                hipStream_t st);

struct AttnPlan {
  int nsplit, split_tokens;
  size_t qrot_off, part_off, total;
};
// max_split_tokens > 0 caps the tokens of one split (the paged layout stages a
// split's page ids in LDS); the split count then grows past the target.
AttnPlan attn_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t hot_cap,
                   int64_t max_split_tokens = 0);

struct AttnCall {
  const float* qrot;        // [B, Hq, 128] fp32 = q @ PiK^T (when PiK is null)
  const uint16_t* q;        // [B, Hq, 128] fp16 (the fp16 hot window uses the unrotated query)
  const uint8_t* k_codes;   // [B, Hkv, cap, 64]
  const float* k_norms;     // [B, Hkv, cap]
  const uint8_t* v_codes;
  const float* v_norms;
  const uint16_t* k_hot;    // [B, Hkv, hot_cap, 128] ring, token t in slot t % hot_cap
  const uint16_t* v_hot;
  const float* PiV;         // [128, 128]
  const float* PiK;         // non-null: rotate q in the split kernel (qrot unused); null: qrot given
  const float* centroids;   // [2^bits]
  const int32_t* seq_len;   // device scalar: tokens in the cache (after this step's append)
  float* partials;          // split records (workspace)
  uint16_t* out;            // [B, Hq, 128] fp16
  float scale;
  int64_t max_len, B, Hq, Hkv, cap, hot_cap;
  int bits;
  // Decode step (B = 1), set when pq is non-null: the query, key and value
  // of the new token arrive as q|k|v GEMV partials ([slab][chunk][kGemvBN]).
  // The split kernel sums them, applies RoPE at position *pos, rotates the
  // query with PiK (q_rot and q are then unused as inputs); its last split
  // block writes the RoPE'd query to q16 (read by the combine as q) and the
  // new key / value into ring slot *pos % hot_cap.
  const float* pq;
  const float* pk;
  const float* pv;
  int nchunk;
  const uint16_t* rope_cos;  // [max_len, 128] fp16
  const uint16_t* rope_sin;
  const int32_t* pos;
  uint16_t* q16;
  uint16_t* k_ring;
  uint16_t* v_ring;
  // Paged cold store, set when indptr is non-null: k/v codes and norms are
  // pools of [max_pages][Hkv][1 << page_shift] rows, sequence b owns pages
  // indices[indptr[b] .. indptr[b + 1]) and seq_len holds B lengths.
  const int32_t* indptr;
  const int32_t* indices;
  int page_shift;
  int64_t max_pages;
};
// Launch the split and combine kernels.
int attn_launch(const AttnCall& c, const AttnPlan& pl, hipStream_t st);

// Attention of the dense fp16-KV decode step (B = 1, at most 4 query heads
// per kv head) over the page pool kv [page][K, V][page_size][Hkv][128] fp16,
// token t in page t / page_size (identity pages).  The query, key and value
// of the new token arrive as q|k|v GEMV partials ([slab][chunk][kGemvBN]);
// the split kernel sums them, applies RoPE at position *pos (query and key
// rounded to fp16), writes the new key and value into the pool and attends
// over tokens 0 .. *pos; then the combine writes out [Hq, 128] fp16.
struct F16kvStepAttn {
  const float* pq;
  const float* pk;
  const float* pv;
  int nchunk;
  const uint16_t* rope_cos;  // [max_len, 128] fp16
  const uint16_t* rope_sin;
  const int32_t* pos;
  uint16_t* kv;
  int64_t Hq, Hkv, page_size, max_pages, max_len;
  float scale;
  uint16_t* out;
  void* records;  // lkv_paged_decode_attn_workspace_bytes(1, Hq, Hkv, max_len) bytes
  size_t record_bytes;
};
int f16kv_step_attn(const F16kvStepAttn& a, hipStream_t st);

}  // namespace lkv
