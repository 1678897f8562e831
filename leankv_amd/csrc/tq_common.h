// TurboQuant device helpers shared by the quantize / rotate kernels and the
// decode-step kernels: the 16-vector MFMA rotation tile, the normalisation and
// bucketing arithmetic of leankv/turboquant/quantizer.py:119-129, and the
// packed-row stores.  All kernels that quantize go through these, so a vector
// gets bit-identical codes whichever kernel quantizes it.
//
// Rotation tile (fp32 MFMA, v_mfma_f32_16x16x4_f32), 4 waves per block:
//   * every wave holds the whole 16x128 tile as its A operand (lane l: vector
//     l%16, the 32 contiguous coordinates 32*(l/16) .. +31, so the k order of
//     the contraction is permuted; B uses the same permutation);
//   * wave w produces output dims {8n + 2w, 8n + 2w + 1 : n = 0..15} from
//     two 16-column MFMA tiles whose B operands (64 fp32 of Pi per lane) stay
//     in registers.  Those two dims are exactly the two nibbles of byte
//     4n + w of a packed 4-bit row.
#pragma once

#include "common.h"

namespace lkv {
namespace tq {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kRows = 16;


// Packing width in bits of one code (reference rounds 3 up to 4 bits).
__host__ __device__ constexpr int pack_bits(int bits) { return bits == 1 ? 1 : (bits == 2 ? 2 : 4); }
__host__ __device__ constexpr int row_bytes_for(int bits) { return kD * pack_bits(bits) / 8; }

// B operand for the two MFMA column tiles of this wave.
//   transpose == false: y = x @ Pi^T  -> B[k][j] = Pi[j][k]
//   transpose == true : y = x @ Pi    -> B[k][j] = Pi[k][j]
__device__ __forceinline__ void load_pi_operand(const float* __restrict__ Pi, bool transpose,
                                                int wave, int lane, float (&b)[2][32]) {
  const int n = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = 8 * n + 2 * wave + t;
    if (!transpose) {
      const float4* src = reinterpret_cast<const float4*>(Pi + j * kD + 32 * q);
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float4 f = src[v];
        b[t][4 * v] = f.x;
        b[t][4 * v + 1] = f.y;
        b[t][4 * v + 2] = f.z;
        b[t][4 * v + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) b[t][s] = Pi[(32 * q + s) * kD + j];
    }
  }
}

// acc[t][i] = sum_k a_row[k] * B[k][col] for row 4*(lane/16)+i, col = dim 8*(lane%16)+2*wave+t.
__device__ __forceinline__ void rotate_tile(const float (&a)[32], const float (&b)[2][32],
                                            f32x4 (&acc)[2]) {
  acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
  acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 32; ++s) {
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[0][s], acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[1][s], acc[1], 0, 0, 0);
  }
}

__device__ __forceinline__ void load_row_f32(const float* __restrict__ p, float (&a)[32]) {
  const float4* src = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const float4 f = src[v];
    a[4 * v] = f.x;
    a[4 * v + 1] = f.y;
    a[4 * v + 2] = f.z;
    a[4 * v + 3] = f.w;
  }
}

__device__ __forceinline__ void load_row_f16(const uint16_t* __restrict__ p, float (&a)[32]) {
  const uint4* src = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint4 u = src[v];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[8 * v + 2 * i] = h2f(static_cast<uint16_t>(w[i] & 0xffffu));
      a[8 * v + 2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

// norm = ||row|| (fp32 accumulate, the 4 lanes sharing a row combine), then
// u = x / (norm + 1e-10) with the rounding of x's dtype.  Returns the norm
// as stored by the reference (fp32, or fp32 value of the fp16 norm).
template <bool F16>
__device__ __forceinline__ float normalize_row(float (&a)[32]) {
#pragma clang fp contract(off)
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < 32; ++s) ss = fmaf(a[s], a[s], ss);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float nrm = sqrtf(ss);
  if (!F16) {
    const float d = nrm + 1e-10f;
#pragma unroll
    for (int s = 0; s < 32; ++s) a[s] = a[s] / d;
    return nrm;
  } else {
    const float n16 = h2f(f2h(nrm));
    const float d = h2f(f2h(n16 + 1e-10f));
    // a / d correctly rounded from one division per row: r = 1 / d (IEEE), then
    // per element q0 = a r and one FMA correction (Markstein); e == 0 means q0
    // is exact (and keeps the sign of a zero quotient).  Every fp16 a and
    // positive fp16 d gives the IEEE quotient bit for bit (tests/fp16_div_check.c
    // checks all 2.0e9 pairs); d is 0 only for an all-zero row, NaN either way.
    const float r = 1.f / d;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      const float q0 = a[s] * r;
      const float e = fmaf(-q0, d, a[s]);
      a[s] = h2f(f2h(e == 0.f ? q0 : fmaf(e, r, q0)));
    }
    return n16;
  }
}

// normalize_row<false> applied only where `apply` holds (every lane takes part
// in the shuffles; rows without `apply` are left unchanged).  Same arithmetic,
// so an fp32 row quantized here gets the codes the quantize kernels give it.
__device__ __forceinline__ float normalize_row_f32_if(float (&a)[32], bool apply) {
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < 32; ++s) ss = fmaf(a[s], a[s], ss);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float nrm = sqrtf(ss);
  if (apply) {
    const float d = nrm + 1e-10f;
#pragma unroll
    for (int s = 0; s < 32; ++s) a[s] = a[s] / d;
  }
  return nrm;
}

template <int BITS>
__device__ __forceinline__ int bucket(float y, const float* bd) {
  constexpr int NB = (1 << BITS) - 1;
  int c = 0;
#pragma unroll
  for (int i = 0; i < NB; ++i) c += (bd[i] < y) ? 1 : 0;
  return c;
}

// Write this wave's codes of the tile into s_codes[16][128].
template <int BITS>
__device__ __forceinline__ void codes_to_lds(const f32x4 (&acc)[2], const float* bd, int wave,
                                             int lane, uint8_t* s_codes) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * (lane >> 4) + i;
      const int dim = 8 * (lane & 15) + 2 * wave + t;
      s_codes[row * kD + dim] = static_cast<uint8_t>(bucket<BITS>(acc[t][i], bd));
    }
}

// Pack s_codes rows into dwords and store rows [row0, row0+16) (valid < M).
// Row r goes to dst + row_offset(r) bytes.
template <int BITS, typename RowOff>
__device__ __forceinline__ void pack_store(const uint8_t* s_codes, uint8_t* __restrict__ dst,
                                           int64_t row0, int64_t M, RowOff row_off) {
  constexpr int PB = pack_bits(BITS);
  constexpr int RB = row_bytes_for(BITS);
  constexpr int DPW = 32 / PB;  // dims per packed dword
  constexpr int WPR = RB / 4;   // dwords per row
  for (int i = threadIdx.x; i < kRows * WPR; i += kThreads) {
    const int r = i / WPR, w = i % WPR;
    if (row0 + r >= M) continue;
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < DPW; ++e) v |= static_cast<uint32_t>(s_codes[r * kD + w * DPW + e]) << (PB * e);
    *reinterpret_cast<uint32_t*>(dst + row_off(row0 + r) + 4 * w) = v;
  }
}


}  // namespace tq
}  // namespace lkv
