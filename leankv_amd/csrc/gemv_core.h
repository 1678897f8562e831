// The body of one TEAL sparse GEMV work item (one column slab of kGemvBN
// outputs x one chunk of BZ input rows): every GEMV launch of the library
// (standalone entry points and the decode step's prologue variants) runs it,
// so all compute the same partial sums bit for bit.
//
// Semantics: leankv/teal/kernels/sparse_gemv.py:61-87 -- the item sums
// A[z, n] * x[z] over the rows z of its chunk whose |x[z]| > threshold
// (strict, fp32 compare), fp32 accumulate.  A is the column-major weight of
// prepare_weight_for_sparse_gemv (:229-234): row z is N contiguous fp16.
//
//   1. compaction: |x| > t over the chunk's BZ inputs (in registers) into
//      an LDS list of surviving rows, wave ballot + mbcnt prefix + a
//      cross-wave prefix; padded to whole streaming batches with (last row, 0);
//   2. streaming: 32 lanes cover one 512-byte row segment with 16-byte buffer
//      loads (out-of-range columns read 0); SLOTS row slots each keep U rows
//      in flight per lane;
//   3. the row slots are reduced through LDS into kGemvBN fp32 column sums,
//      returned to threads 0 .. kGemvBN-1.
#pragma once

#include "kernels.h"

namespace lkv {

typedef uint32_t gemv_u32x4 __attribute__((ext_vector_type(4)));

template <int NT, int BZ, bool DUAL, int U>
struct GemvLds {
  static constexpr int kLpr = kGemvBN / 8;   // lanes per row segment
  static constexpr int kSlots = NT / kLpr;   // rows processed side by side
  static constexpr int kNl = DUAL ? 2 : 1;
  static constexpr int kPad = U * kSlots;    // list granularity
  int idx[kNl][BZ + kPad];
  float xv[kNl][BZ + kPad];
  int cnt[kNl][NT / kWave];
  int last[kNl][NT / kWave];
  float wsum[NT / kWave];
  alignas(16) float red[kNl * kSlots * kGemvBN];
};

__device__ __forceinline__ void gemv_fma8(float (&acc)[8], const gemv_u32x4& w, float xv) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] = fmaf(h2f(static_cast<uint16_t>(w[i] & 0xffffu)), xv, acc[2 * i]);
    acc[2 * i + 1] = fmaf(h2f(static_cast<uint16_t>(w[i] >> 16)), xv, acc[2 * i + 1]);
  }
}

// Buffer descriptor over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemv_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Stream the padded survivor list: total is a multiple of U * SLOTS.  CP is
// the buffer-load cache policy (2 = nt: streamed once, no L2 retention).
template <int SLOTS, int U, int CP>
__device__ __forceinline__ void gemv_stream_rows(__amdgpu_buffer_rsrc_t A, uint32_t row_bytes, uint32_t col_bytes,
                                                 const int* __restrict__ idx, const float* __restrict__ xv, int total,
                                                 int slot, float (&acc)[8]) {
  for (int s = slot; s < total; s += U * SLOTS) {
    int r[U];
    float xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      r[u] = idx[s + u * SLOTS];
      xs[u] = xv[s + u * SLOTS];
    }
    gemv_u32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      w[u] = __builtin_amdgcn_raw_buffer_load_b128(A, static_cast<uint32_t>(r[u]) * row_bytes + col_bytes, 0, CP);
#pragma unroll
    for (int u = 0; u < U; ++u) gemv_fma8(acc, w[u], xs[u]);
  }
}

// Steps 1-3 for the chunk of inputs z0 .. z0 + BZ (thread t holds inputs
// z0 + E t + j in v[j], E = BZ / NT, 0 past Z) and the output columns n0 ..
// n0 + kGemvBN of an N-column matrix A0 (and A1 in dual mode, thresholds
// t0 / t1).  sums[l] is the column sum of matrix l for column n0 + threadIdx.x
// (threads < kGemvBN).  The LDS is still being read when it returns: a caller
// that reuses it needs a barrier first.
template <int NT, int BZ, bool DUAL, int U, int CP>
__device__ __forceinline__ void gemv_core(GemvLds<NT, BZ, DUAL, U>& sm, const float (&v)[BZ / NT], const uint16_t* A0,
                                          const uint16_t* A1, uint32_t a_bytes, int N, float t0, float t1, int z0,
                                          int Z, int n0, float (&sums)[DUAL ? 2 : 1]) {
  using L = GemvLds<NT, BZ, DUAL, U>;
  constexpr int NL = L::kNl, PAD = L::kPad, LPR = L::kLpr, SLOTS = L::kSlots, BN = kGemvBN;
  static_assert(BZ % NT == 0, "BZ must be a multiple of the block size");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  // ---- 1. compaction of surviving activation rows, one round: thread t
  // tests inputs E t .. E t + E - 1 (E = BZ / NT), so the list comes out in
  // ascending row order; lane offsets from one ballot per input, wave offsets
  // from one cross-wave prefix through LDS.  The last surviving row (the
  // padding value) is found from the per-wave counts without reading the list.
  constexpr int E = BZ / NT;
  int total[NL];
  {
    int pre[NL], cnt[NL], lastz[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      pre[l] = 0;
      cnt[l] = 0;
      lastz[l] = -1;
      int wtot = 0;
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const int z = z0 + E * tid + j;
        const float t = (l == 0) ? t0 : t1;
        const bool p = z < Z && fabsf(v[j]) > t;
        const uint64_t m = wave_ballot(p);
        pre[l] += lane_prefix(m);
        wtot += __popcll(m);
        cnt[l] += p ? 1 : 0;
        lastz[l] = p ? z : lastz[l];
      }
      // the wave's last surviving row sits in its highest lane with a survivor
      const uint64_t any = wave_ballot(cnt[l] > 0);
      if (lane == 0) sm.cnt[l][wave] = wtot;
      if (any != 0 && lane == 63 - __builtin_clzll(any)) sm.last[l][wave] = lastz[l];
    }
    __syncthreads();
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      int off = pre[l], tot = 0, last = 0;
#pragma unroll
      for (int w = 0; w < NT / kWave; ++w) {
        const int cw = sm.cnt[l][w];
        off += (w < wave) ? cw : 0;
        tot += cw;
        last = cw > 0 ? sm.last[l][w] : last;
      }
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const int z = z0 + E * tid + j;
        const float t = (l == 0) ? t0 : t1;
        if (z < Z && fabsf(v[j]) > t) {
          sm.idx[l][off] = z;
          sm.xv[l][off] = v[j];
          ++off;
        }
      }
      // pad each list to a multiple of PAD with (last row, 0): padded loads hit the line just fetched
      const int padded = (tot + PAD - 1) / PAD * PAD;
      if (tot > 0 && tid < padded - tot) {
        sm.idx[l][tot + tid] = last;
        sm.xv[l][tot + tid] = 0.f;
      }
      total[l] = padded;
    }
  }
  __syncthreads();

  // ---- 2. stream surviving weight rows
  const int c = tid % LPR;
  const int slot = tid / LPR;
  const int col = n0 + c * 8;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * 2u;
  // Columns past N would alias the next row: push them past the descriptor end.
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : a_bytes;
  float acc[NL][8];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[l][j] = 0.f;
  gemv_stream_rows<SLOTS, U, CP>(gemv_rsrc(A0, a_bytes), row_bytes, col_bytes, sm.idx[0], sm.xv[0], total[0], slot,
                                 acc[0]);
  if (DUAL)
    gemv_stream_rows<SLOTS, U, CP>(gemv_rsrc(A1, a_bytes), row_bytes, col_bytes, sm.idx[NL - 1], sm.xv[NL - 1],
                                   total[NL - 1], slot, acc[NL - 1]);

  // ---- 3. cross-slot reduction through LDS, every matrix at once
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float4* dst = reinterpret_cast<float4*>(sm.red + (l * SLOTS + slot) * BN + c * 8);
    dst[0] = make_float4(acc[l][0], acc[l][1], acc[l][2], acc[l][3]);
    dst[1] = make_float4(acc[l][4], acc[l][5], acc[l][6], acc[l][7]);
  }
  __syncthreads();
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float s = 0.f;
    if (tid < BN) {
#pragma unroll
      for (int sl = 0; sl < SLOTS; ++sl) s += sm.red[(l * SLOTS + sl) * BN + tid];
    }
    sums[l] = s;
  }
}

// Dense variant, for launches whose thresholds are all 0: every row of the
// chunk takes part (for finite weights the same sums as the compacted list,
// since a row whose input is exactly 0 adds 0), so there is no compaction and
// slot k walks rows k, k + SLOTS, ... of the chunk, the order the list has when
// nothing is dropped.  The weight loads do not depend on x: the caller issues
// the first kDensePf batches (gemv_dense_first) before using its input
// prologue's loads, so the memory round trips overlap.  Rows past Z read 0 through the descriptor and
// have input 0.
__device__ __forceinline__ uint32_t gemv_dense_off(int z, int Z, uint32_t row_bytes, uint32_t col_bytes,
                                                   uint32_t a_bytes) {
  return z < Z ? static_cast<uint32_t>(z) * row_bytes + col_bytes : a_bytes;  // past Z: past the descriptor end
}

// Batches the dense variant issues ahead of its input prologue (1 -> 2: config-5
// dense step 326.05 -> 326.39 tok/s on one box).
constexpr int kDensePf = 2;

template <int NT, int U, int CP>
__device__ __forceinline__ void gemv_dense_first(const uint16_t* A0, uint32_t a_bytes, int N, int z0, int Z, int n0,
                                                 gemv_u32x4 (&w)[U * kDensePf]) {
  constexpr int LPR = kGemvBN / 8, SLOTS = NT / LPR;
  const int tid = threadIdx.x;
  const int col = n0 + (tid % LPR) * 8;
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : a_bytes;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * 2u;
  const __amdgpu_buffer_rsrc_t A = gemv_rsrc(A0, a_bytes);
#pragma unroll
  for (int u = 0; u < U * kDensePf; ++u)
    w[u] = __builtin_amdgcn_raw_buffer_load_b128(
        A, gemv_dense_off(z0 + tid / LPR + u * SLOTS, Z, row_bytes, col_bytes, a_bytes), 0, CP);
}

template <int NT, int BZ, bool DUAL, int U, int CP>
__device__ __forceinline__ void gemv_core_dense(GemvLds<NT, BZ, DUAL, U>& sm, const float (&v)[BZ / NT],
                                                const gemv_u32x4 (&w0)[U * kDensePf], const uint16_t* A0, const uint16_t* A1,
                                                uint32_t a_bytes, int N, int z0, int Z, int n0,
                                                float (&sums)[DUAL ? 2 : 1]) {
  using L = GemvLds<NT, BZ, DUAL, U>;
  constexpr int NL = L::kNl, LPR = L::kLpr, SLOTS = L::kSlots, BN = kGemvBN, E = BZ / NT;
  static_assert(BZ % (U * SLOTS) == 0 && BZ >= kDensePf * U * SLOTS, "whole streaming batches per chunk");
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < E; ++j) sm.xv[0][E * tid + j] = v[j];
  __syncthreads();

  const int c = tid % LPR;
  const int slot = tid / LPR;
  const int col = n0 + c * 8;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * 2u;
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : a_bytes;
  const float* xs = sm.xv[0];
  float acc[NL][8];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[l][j] = 0.f;
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const __amdgpu_buffer_rsrc_t A = gemv_rsrc(l == 0 ? A0 : A1, a_bytes);
    int s = slot;
    if (l == 0) {  // the preloaded first batches
#pragma unroll
      for (int u = 0; u < U * kDensePf; ++u) gemv_fma8(acc[0], w0[u], xs[s + u * SLOTS]);
      s += U * kDensePf * SLOTS;
    }
    for (; s < BZ; s += U * SLOTS) {
      gemv_u32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(
            A, gemv_dense_off(z0 + s + u * SLOTS, Z, row_bytes, col_bytes, a_bytes), 0, CP);
#pragma unroll
      for (int u = 0; u < U; ++u) gemv_fma8(acc[l], w[u], xs[s + u * SLOTS]);
    }
  }

  // the cross-slot reduction of gemv_core
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float4* dst = reinterpret_cast<float4*>(sm.red + (l * SLOTS + slot) * BN + c * 8);
    dst[0] = make_float4(acc[l][0], acc[l][1], acc[l][2], acc[l][3]);
    dst[1] = make_float4(acc[l][4], acc[l][5], acc[l][6], acc[l][7]);
  }
  __syncthreads();
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float s = 0.f;
    if (tid < BN) {
#pragma unroll
      for (int sl = 0; sl < SLOTS; ++sl) s += sm.red[(l * SLOTS + sl) * BN + tid];
    }
    sums[l] = s;
  }
}

}  // namespace lkv
