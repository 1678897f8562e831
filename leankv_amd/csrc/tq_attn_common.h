// Device helpers shared by the packed-KV attention kernels (decode split /
// combine in tq_attn.hip, prefill in tq_prefill.hip): fp16 packing, exp2,
// 3-bit code decode with v_perm_b32 table lookups, and reductions over the
// four lane groups of a wave.
#pragma once

#include "kernels.h"

namespace lkv {
namespace {

__device__ __forceinline__ uint32_t pack2h(float lo, float hi) {
  return static_cast<uint32_t>(f2h(lo)) | (static_cast<uint32_t>(f2h(hi)) << 16);
}

// 2^x on the hardware exp (v_exp_f32); arguments here are <= 0 and results
// below 2^-126 flush to 0, which only drops contributions < 1e-38 of the max.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 3-bit codes decoded on the VALU: one code dword = 8 nibbles (dims 0..7)
// becomes 4 dwords of fp16 pairs in the dim order [0,2 | 4,6 | 1,3 | 5,7].
// tab[0..1] hold the low bytes of the 8 fp16 centroids, tab[2..3] the high
// bytes; v_perm_b32 picks 4 of those 8 bytes per instruction (selector bytes
// 0..7 address {S0: bytes 4-7, S1: bytes 0-3}), so a lookup is 4 nibbles per
// instruction with no LDS traffic.  The query operand uses the same dim
// order, so each MFMA sees the same fp16 products as with natural order.
__device__ __forceinline__ void decode8(uint32_t w, const uint32_t (&tab)[4], uint32_t (&d)[4]) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // codes of dims 0, 2, 4, 6 (one per byte)
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // dims 1, 3, 5, 7
  const uint32_t llo = __builtin_amdgcn_perm(tab[1], tab[0], lo), hlo = __builtin_amdgcn_perm(tab[3], tab[2], lo);
  const uint32_t lhi = __builtin_amdgcn_perm(tab[1], tab[0], hi), hhi = __builtin_amdgcn_perm(tab[3], tab[2], hi);
  d[0] = __builtin_amdgcn_perm(hlo, llo, 0x05010400u);  // dims 0, 2
  d[1] = __builtin_amdgcn_perm(hlo, llo, 0x07030602u);  // dims 4, 6
  d[2] = __builtin_amdgcn_perm(hhi, lhi, 0x05010400u);  // dims 1, 3
  d[3] = __builtin_amdgcn_perm(hhi, lhi, 0x07030602u);  // dims 5, 7
}
// Position p of a decoded group holds dim kPermDim[p].
__device__ constexpr int kPermDim[8] = {0, 2, 4, 6, 1, 3, 5, 7};

// PERM: decode8 (3-bit codes).  Otherwise a 256-entry LDS table maps one
// code byte to the fp16 pair (c[lo nibble], c[hi nibble]) in natural order.
template <bool PERM>
__device__ __forceinline__ void decode_dw(uint32_t w, const uint32_t (&tab)[4], const uint32_t* s_lut,
                                          uint32_t (&d)[4]) {
  if constexpr (PERM) {
    decode8(w, tab, d);
  } else {
    d[0] = s_lut[w & 0xffu];
    d[1] = s_lut[(w >> 8) & 0xffu];
    d[2] = s_lut[(w >> 16) & 0xffu];
    d[3] = s_lut[w >> 24];
  }
}
// Pairs 2*half and 2*half + 1 of decode_dw (the value pass decodes in two
// halves to halve the live registers).
template <bool PERM>
__device__ __forceinline__ void decode_half(uint32_t w, int half, const uint32_t (&tab)[4], const uint32_t* s_lut,
                                            uint32_t (&d)[2]) {
  if constexpr (PERM) {
    const uint32_t c = (half ? (w >> 4) : w) & 0x0F0F0F0Fu;
    const uint32_t lo = __builtin_amdgcn_perm(tab[1], tab[0], c), hi = __builtin_amdgcn_perm(tab[3], tab[2], c);
    d[0] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    d[1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  } else {
    d[0] = s_lut[(w >> (16 * half)) & 0xffu];
    d[1] = s_lut[(w >> (16 * half + 8)) & 0xffu];
  }
}

__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Online-softmax offset headroom, log2 units.  When a block's score exceeds
// the running offset m, m moves to that score plus the headroom, so the
// following blocks, whose scores mostly stay below it, skip the rescale of
// the accumulators.  Any offset at or above every score seen gives the same
// softmax (sums and accumulators are relative to it); every weight stays
// exp2(s - m) <= 1, so p * n_v cannot overflow its fp16 operand, and weights
// shrink by at most 2^-headroom, far above the fp16 denormal floor for any
// weight that matters.  0 gives the plain running maximum.
#ifndef LKV_SOFTMAX_HEADROOM
#define LKV_SOFTMAX_HEADROOM 4.0f
#endif
constexpr float kHeadroom = LKV_SOFTMAX_HEADROOM;

// Max / sum over the four lanes l, l^16, l^32, l^48 (the lane groups that
// hold the other tokens of the same head), result in all four.
__device__ __forceinline__ float xgroup_max(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xgroup_sum(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace
}  // namespace lkv
