// TurboQuant (MSE variant) rotate / quantize / pack / dequantize at head_dim 128.
//
// Semantics: leankv/turboquant/quantizer.py:38-137 (pack, unpack, quantize,
// dequantize) and leankv/turboquant/rotation.py:45-52 (x @ Pi^T, y @ Pi).
//
// The 128x128 rotation is a dense fp32 contraction and runs on fp32 MFMA
// through the 16-vector tile of tq_common.h.  Blocks are persistent over the
// 16-vector tiles so the Pi operand is read from L2 once per block, not once
// per tile.  Codes go through LDS so that packed rows leave in coalesced
// dword stores.
#include "tq_common.h"

namespace lkv {
namespace {

using namespace tq;

enum Mode { kQuant = 0, kRotate = 1, kDequant = 2, kAppend = 3 };

// ---------------------------------------------------------------- quantize
// Nibble layouts (3- and 4-bit codes): one wave owns a whole 16-vector tile
// and computes all 8 output column tiles, so each vector is loaded and
// normalised once (the 4-wave kernel below repeats both in every wave).
// Column tile c holds output dims 8n + c (n = lane % 16): exactly nibble c
// of packed dword n, so a lane packs the dwords of its 4 rows in registers
// and stores them directly.  Each output's MFMA chain -- the same 32 k-steps
// with the same operands in the same order as rotate_tile -- is unchanged,
// so the codes equal every other quantizing kernel's bit for bit.  The B
// operands of the 8 tiles are staged once per block in LDS in MFMA operand
// order: s_b[c][kq][lane] = Pi[8n + c][32q + 4kq .. +3] for lane = 16q + n
// (rows padded by one float4 so the staging writes do not collide in banks).
// #(b < y) over the 2^BITS - 1 sorted decision boundaries by binary search
// (BITS compares instead of 2^BITS - 1): the same count as bucket<BITS>.
// Every boundary index is a compile-time constant (selects, no indexing).
template <int BITS>
__device__ __forceinline__ int bucket_bsearch(float y, const float (&bd)[(1 << BITS) - 1]) {
  static_assert(BITS == 3 || BITS == 4, "nibble layouts");
  if constexpr (BITS == 3) {
    const bool h2 = bd[3] < y;
    const bool h1 = (h2 ? bd[5] : bd[1]) < y;
    const float t0 = h2 ? (h1 ? bd[6] : bd[4]) : (h1 ? bd[2] : bd[0]);
    return (h2 ? 4 : 0) + (h1 ? 2 : 0) + (t0 < y ? 1 : 0);
  } else {
    const bool h3 = bd[7] < y;
    const bool h2 = (h3 ? bd[11] : bd[3]) < y;
    const float t1 = h3 ? (h2 ? bd[13] : bd[9]) : (h2 ? bd[5] : bd[1]);
    const bool h1 = t1 < y;
    const float t0 = h3 ? (h2 ? (h1 ? bd[14] : bd[12]) : (h1 ? bd[10] : bd[8]))
                        : (h2 ? (h1 ? bd[6] : bd[4]) : (h1 ? bd[2] : bd[0]));
    return (h3 ? 8 : 0) + (h2 ? 4 : 0) + (h1 ? 2 : 0) + (t0 < y ? 1 : 0);
  }
}

// The 4-bit search of bucket_bsearch on a boundary table in LDS: the same
// comparisons, the next boundary addressed by the bucket so far (kept in
// registers, the selects between boundaries compile to an indexed load from a
// private, memory-backed copy of the table).
__device__ __forceinline__ int bucket_bsearch4_lds(float y, const float* s_bd) {
  int k = s_bd[7] < y ? 8 : 0;
  k += s_bd[k + 3] < y ? 4 : 0;
  k += s_bd[k + 1] < y ? 2 : 0;
  return k + (s_bd[k] < y ? 1 : 0);
}

template <int BITS, bool F16>
__global__ __launch_bounds__(kThreads, 2) void quantize_wave_kernel(const void* __restrict__ xin, int64_t M,
                                                                    const float* __restrict__ Pi,
                                                                    const float* __restrict__ bounds,
                                                                    uint8_t* __restrict__ packed,
                                                                    void* __restrict__ norms) {
  static_assert(pack_bits(BITS) == 4 && row_bytes_for(BITS) == 64, "nibble layouts only");
  __shared__ float4 s_b[8][8][65];  // 64 KB + one float4 of padding per row: the staging writes of 8
                                     // consecutive threads (8 k-quarters) fall in different banks
  __shared__ float s_bd[16];        // 4-bit boundaries
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int64_t ntiles = (M + kRows - 1) / kRows;
  int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  // The first tile's vectors load while the rotation matrix is staged.
  float a[32];
  auto load_a = [&](int64_t tl) {
    const int64_t r = tl * kRows + n;
    const int64_t rl = r < M ? r : M - 1;  // rows past M read row M - 1 and are zeroed after
    if (F16)
      load_row_f16(static_cast<const uint16_t*>(xin) + rl * kD + 32 * g, a);
    else
      load_row_f32(static_cast<const float*>(xin) + rl * kD + 32 * g, a);
  };
  if (tile < ntiles) load_a(tile);
  // Pi, coalesced: thread tid holds float4 f = 256 i + tid (row f / 32, columns
  // 4 (f % 32) ..), written to its operand slot.
  float4 pr[kD * kD / 4 / kThreads];
#pragma unroll
  for (int i = 0; i < kD * kD / 4 / kThreads; ++i) pr[i] = reinterpret_cast<const float4*>(Pi)[i * kThreads + threadIdx.x];
  float bd[(1 << BITS) - 1];
#pragma unroll
  for (int i = 0; i < (1 << BITS) - 1; ++i) bd[i] = BITS == 3 ? bounds[i] : 0.f;
  if (BITS == 4 && threadIdx.x < (1 << BITS) - 1) s_bd[threadIdx.x] = bounds[threadIdx.x];
#pragma unroll
  for (int i = 0; i < kD * kD / 4 / kThreads; ++i) {
    const int f = i * kThreads + threadIdx.x;
    const int j = f >> 5, c4 = f & 31;  // Pi row j = 8n' + c, columns 32q' + 4kq ..
    s_b[j & 7][c4 & 7][16 * (c4 >> 3) + (j >> 3)] = pr[i];
  }
  __syncthreads();
  for (; tile < ntiles; tile += static_cast<int64_t>(gridDim.x) * 4) {
    const int64_t row0 = tile * kRows;
    const int64_t r = row0 + n;
#pragma unroll
    for (int k = 0; k < 32; ++k) a[k] = r < M ? a[k] : 0.f;
    const float nrm = normalize_row<F16>(a);
    if (g == 0 && r < M) {
      if (F16)
        static_cast<uint16_t*>(norms)[r] = f2h(nrm);
      else
        static_cast<float*>(norms)[r] = nrm;
    }
    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kq = 0; kq < 8; ++kq) {
      float4 bv[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) bv[c] = s_b[c][kq][lane];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const float av = a[4 * kq + cc];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float b = cc == 0 ? bv[c].x : cc == 1 ? bv[c].y : cc == 2 ? bv[c].z : bv[c].w;
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b, acc[c], 0, 0, 0);
        }
      }
      // keeps the next k-quarter's LDS reads after these MFMAs (the compiler
      // otherwise hoists all 256 operand values and spills)
      __builtin_amdgcn_sched_barrier(0);
    }
    const int64_t next = tile + static_cast<int64_t>(gridDim.x) * 4;
    if (next < ntiles) load_a(next);  // in flight during the bucketing and stores
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + 4 * g + i;
      uint32_t v = 0;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int code = BITS == 3 ? bucket_bsearch<BITS>(acc[c][i], bd) : bucket_bsearch4_lds(acc[c][i], s_bd);
        v |= static_cast<uint32_t>(code) << (4 * c);
      }
      if (row < M) *reinterpret_cast<uint32_t*>(packed + row * 64 + 4 * n) = v;
    }
  }
}

template <int BITS, bool F16>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const void* __restrict__ xin, int64_t M,
                                                            const float* __restrict__ Pi,
                                                            const float* __restrict__ bounds,
                                                            uint8_t* __restrict__ packed,
                                                            void* __restrict__ norms) {
  __shared__ uint8_t s_codes[kRows * kD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float bd[(1 << BITS) - 1];
#pragma unroll
  for (int i = 0; i < (1 << BITS) - 1; ++i) bd[i] = bounds[i];
  float b[2][32];
  load_pi_operand(Pi, false, wave, lane, b);
  const int64_t ntiles = (M + kRows - 1) / kRows;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kRows;
    const int64_t r = row0 + (lane & 15);
    float a[32];
    if (r < M) {
      if (F16)
        load_row_f16(static_cast<const uint16_t*>(xin) + r * kD + 32 * (lane >> 4), a);
      else
        load_row_f32(static_cast<const float*>(xin) + r * kD + 32 * (lane >> 4), a);
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) a[s] = 0.f;
    }
    const float nrm = normalize_row<F16>(a);
    if (wave == 0 && lane < 16 && r < M) {
      if (F16)
        static_cast<uint16_t*>(norms)[r] = f2h(nrm);
      else
        static_cast<float*>(norms)[r] = nrm;
    }
    f32x4 acc[2];
    rotate_tile(a, b, acc);
    codes_to_lds<BITS>(acc, bd, wave, lane, s_codes);
    __syncthreads();
    pack_store<BITS>(s_codes, packed, row0, M,
                     [](int64_t rr) { return rr * static_cast<int64_t>(row_bytes_for(BITS)); });
    __syncthreads();
  }
}

// -------------------------------------------------------- quantize_rotated
template <int BITS>
__global__ __launch_bounds__(kThreads) void quantize_rotated_kernel(const float* __restrict__ y, int64_t M,
                                                                    const float* __restrict__ bounds,
                                                                    uint8_t* __restrict__ packed) {
  constexpr int PB = pack_bits(BITS);
  constexpr int DPW = 32 / PB;
  constexpr int WPR = row_bytes_for(BITS) / 4;
  float bd[(1 << BITS) - 1];
#pragma unroll
  for (int i = 0; i < (1 << BITS) - 1; ++i) bd[i] = bounds[i];
  const int64_t total = M * WPR;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t r = i / WPR;
    const int w = static_cast<int>(i % WPR);
    const float* src = y + r * kD + w * DPW;
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < DPW; ++e) v |= static_cast<uint32_t>(bucket<BITS>(src[e], bd)) << (PB * e);
    reinterpret_cast<uint32_t*>(packed)[i] = v;
  }
}

// ----------------------------------------------------- rotate / dequantize
// mode kRotate : y(f32)  = x @ Pi^T (transpose=0) or x @ Pi (transpose=1)
// mode kDequant: out     = (centroids[unpack(codes)] @ Pi) * norm
template <int MODE, int BITS, bool IN_F16, bool OUT_F16>
__global__ __launch_bounds__(kThreads) void rotate_kernel(const void* __restrict__ xin,
                                                          const void* __restrict__ norms_in, int64_t M,
                                                          const float* __restrict__ Pi, int transpose,
                                                          const float* __restrict__ centroids,
                                                          void* __restrict__ out) {
  __shared__ __align__(16) float s_out[kRows * kD];
  __shared__ float s_tab[16];
  __shared__ float s_norm[kRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (MODE == kDequant && threadIdx.x < 16) {
    constexpr int NC = 1 << BITS;
    s_tab[threadIdx.x] = centroids[threadIdx.x < NC ? threadIdx.x : NC - 1];
  }
  __syncthreads();
  float b[2][32];
  load_pi_operand(Pi, MODE == kDequant ? true : transpose != 0, wave, lane, b);
  const int64_t ntiles = (M + kRows - 1) / kRows;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kRows;
    const int64_t r = row0 + (lane & 15);
    const int q = lane >> 4;
    float a[32];
    if (r < M) {
      if (MODE == kRotate) {
        if (IN_F16)
          load_row_f16(static_cast<const uint16_t*>(xin) + r * kD + 32 * q, a);
        else
          load_row_f32(static_cast<const float*>(xin) + r * kD + 32 * q, a);
      } else {
        constexpr int PB = pack_bits(BITS);
        constexpr int RB = row_bytes_for(BITS);
        // The 32 codes of dims 32q..32q+31 occupy 32*PB/8 = 4*PB bytes.
        const uint8_t* src = static_cast<const uint8_t*>(xin) + r * RB + q * 4 * PB;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < PB; ++i) w[i] = reinterpret_cast<const uint32_t*>(src)[i];
#pragma unroll
        for (int s = 0; s < 32; ++s) {
          const int bit = s * PB;
          const uint32_t code = (w[bit >> 5] >> (bit & 31)) & ((1u << PB) - 1u);
          a[s] = s_tab[code];
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) a[s] = 0.f;
    }
    if (MODE == kDequant && threadIdx.x < kRows) {
      const int64_t rr = row0 + threadIdx.x;
      float nv = 0.f;
      if (rr < M) nv = IN_F16 ? h2f(static_cast<const uint16_t*>(norms_in)[rr])
                              : static_cast<const float*>(norms_in)[rr];
      s_norm[threadIdx.x] = nv;
    }
    f32x4 acc[2];
    rotate_tile(a, b, acc);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * (lane >> 4) + i;
        const int dim = 8 * (lane & 15) + 2 * wave + t;
        s_out[row * kD + dim] = acc[t][i];
      }
    __syncthreads();
    // 16 rows x 128 = 2048 values; each thread stores 8 consecutive ones.
    {
      const int row = threadIdx.x >> 4;
      const int c0 = (threadIdx.x & 15) * 8;
      const int64_t rg = row0 + row;
      if (rg < M) {
        float v[8];
        const float sc = (MODE == kDequant) ? s_norm[row] : 1.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = s_out[row * kD + c0 + e] * sc;
        if (OUT_F16) {
          uint4 o;
          o.x = f2h(v[0]) | (static_cast<uint32_t>(f2h(v[1])) << 16);
          o.y = f2h(v[2]) | (static_cast<uint32_t>(f2h(v[3])) << 16);
          o.z = f2h(v[4]) | (static_cast<uint32_t>(f2h(v[5])) << 16);
          o.w = f2h(v[6]) | (static_cast<uint32_t>(f2h(v[7])) << 16);
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + rg * kD + c0) = o;
        } else {
          float4* dst = reinterpret_cast<float4*>(static_cast<float*>(out) + rg * kD + c0);
          dst[0] = make_float4(v[0], v[1], v[2], v[3]);
          dst[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
      }
    }
    __syncthreads();
  }
}

// --------------------------------------------------------------- cache append
// blockIdx.y: 0 = keys, 1 = values.  One tile of 16 (batch, kv-head) rows.
template <int BITS>
__global__ __launch_bounds__(kThreads) void append_kernel(
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new, uint16_t* __restrict__ k_hot,
    uint16_t* __restrict__ v_hot, uint8_t* __restrict__ k_codes, float* __restrict__ k_norms,
    uint8_t* __restrict__ v_codes, float* __restrict__ v_norms, const float* __restrict__ PiK,
    const float* __restrict__ PiV, const float* __restrict__ bounds, const int32_t* __restrict__ pos_p,
    int64_t R, int64_t hot_cap, int64_t cap) {
  constexpr int RB = row_bytes_for(BITS);
  __shared__ uint8_t s_codes[kRows * kD];
  const bool is_v = blockIdx.y == 1;
  const uint16_t* xnew = is_v ? v_new : k_new;
  uint16_t* hot = is_v ? v_hot : k_hot;
  uint8_t* codes = is_v ? v_codes : k_codes;
  float* norms = is_v ? v_norms : k_norms;
  const float* Pi = is_v ? PiV : PiK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t pos = static_cast<int64_t>(*pos_p);
  if (pos < 0) return;  // uniform: a negative position has no ring slot
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int64_t slot = pos % hot_cap;
  const int64_t cold = pos - hot_cap;  // token leaving the hot window
  if (pos >= hot_cap && cold < cap) {
    float bd[(1 << BITS) - 1];
#pragma unroll
    for (int i = 0; i < (1 << BITS) - 1; ++i) bd[i] = bounds[i];
    float b[2][32];
    load_pi_operand(Pi, false, wave, lane, b);
    const int64_t r = row0 + (lane & 15);
    float a[32];
    if (r < R) {
      load_row_f16(hot + (r * hot_cap + slot) * kD + 32 * (lane >> 4), a);
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) a[s] = 0.f;
    }
    // cache.py:141 quantizes flush_k.float(): fp32 semantics on fp16 data.
    const float nrm = normalize_row<false>(a);
    if (wave == 0 && lane < 16 && r < R) norms[r * cap + cold] = nrm;
    f32x4 acc[2];
    rotate_tile(a, b, acc);
    codes_to_lds<BITS>(acc, bd, wave, lane, s_codes);
    __syncthreads();  // every wave has consumed the old hot slot
    pack_store<BITS>(s_codes, codes, row0, R,
                     [=](int64_t rr) { return (rr * cap + cold) * static_cast<int64_t>(RB); });
  }
  __syncthreads();
  // New token into its ring slot: 16 rows x 256 B, 16 bytes per thread.
  {
    const int row = threadIdx.x >> 4;
    const int c0 = (threadIdx.x & 15) * 8;
    const int64_t rg = row0 + row;
    if (rg < R)
      *reinterpret_cast<uint4*>(hot + (rg * hot_cap + slot) * kD + c0) =
          *reinterpret_cast<const uint4*>(xnew + rg * kD + c0);
  }
}

int grid_for(int64_t M) {
  const int64_t ntiles = (M + kRows - 1) / kRows;
  const int64_t g = 2 * static_cast<int64_t>(device_cu_count());
  return static_cast<int>(ntiles < g ? (ntiles > 0 ? ntiles : 1) : g);
}

int check_bits(int bits, const char* what) {
  LKV_REQUIRE(bits >= 1 && bits <= 4, "%s: bits=%d unsupported (1..4 are bit-packed)", what, bits);
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" int lkv_tq_packed_row_bytes(int bits) {
  if (bits < 1 || bits > 4) return -1;
  return row_bytes_for(bits);
}

#define LKV_BITS_SWITCH(bits, ...)        \
  switch (bits) {                         \
    case 1: { constexpr int B_ = 1; __VA_ARGS__; break; } \
    case 2: { constexpr int B_ = 2; __VA_ARGS__; break; } \
    case 3: { constexpr int B_ = 3; __VA_ARGS__; break; } \
    default: { constexpr int B_ = 4; __VA_ARGS__; break; } \
  }

extern "C" int lkv_tq_quantize(const void* x, int x_dtype, int64_t M, const float* Pi,
                               const float* bounds, int bits, uint8_t* packed, void* norms,
                               void* stream) {
  if (int e = check_bits(bits, "tq_quantize")) return e;
  LKV_REQUIRE(M >= 0, "tq_quantize: negative M");
  LKV_REQUIRE(x_dtype == LKV_DTYPE_F32 || x_dtype == LKV_DTYPE_F16, "tq_quantize: x dtype must be f32/f16");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(x && Pi && bounds && packed && norms, "tq_quantize: null pointer");
  LKV_REQUIRE(aligned16(x) && aligned16(Pi) && aligned4(packed),
              "tq_quantize: x and Pi must be 16-byte aligned, packed 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (bits >= 3) {  // nibble layouts: one wave per 16-vector tile
    const int64_t ntiles = (M + kRows - 1) / kRows;
    const int64_t cap = 2 * static_cast<int64_t>(device_cu_count());  // 64 KB of LDS: 2 blocks per CU
    const int gw = static_cast<int>(std::min<int64_t>((ntiles + 3) / 4, cap));
    if (x_dtype == LKV_DTYPE_F16) {
      if (bits == 3)
        hipLaunchKernelGGL((quantize_wave_kernel<3, true>), dim3(gw), dim3(kThreads), 0, st, x, M, Pi, bounds, packed, norms);
      else
        hipLaunchKernelGGL((quantize_wave_kernel<4, true>), dim3(gw), dim3(kThreads), 0, st, x, M, Pi, bounds, packed, norms);
    } else {
      if (bits == 3)
        hipLaunchKernelGGL((quantize_wave_kernel<3, false>), dim3(gw), dim3(kThreads), 0, st, x, M, Pi, bounds, packed, norms);
      else
        hipLaunchKernelGGL((quantize_wave_kernel<4, false>), dim3(gw), dim3(kThreads), 0, st, x, M, Pi, bounds, packed, norms);
    }
    LKV_LAUNCH_CHECK("tq_quantize");
    return LKV_OK;
  }
  const int g = grid_for(M);
  if (x_dtype == LKV_DTYPE_F16) {
    LKV_BITS_SWITCH(bits, hipLaunchKernelGGL((quantize_kernel<B_, true>), dim3(g), dim3(kThreads), 0, st,
                                             x, M, Pi, bounds, packed, norms))
  } else {
    LKV_BITS_SWITCH(bits, hipLaunchKernelGGL((quantize_kernel<B_, false>), dim3(g), dim3(kThreads), 0, st,
                                             x, M, Pi, bounds, packed, norms))
  }
  LKV_LAUNCH_CHECK("tq_quantize");
  return LKV_OK;
}

extern "C" int lkv_tq_quantize_rotated(const float* y, int64_t M, const float* bounds, int bits,
                                       uint8_t* packed, void* stream) {
  if (int e = check_bits(bits, "tq_quantize_rotated")) return e;
  LKV_REQUIRE(M >= 0, "tq_quantize_rotated: negative M");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(y && bounds && packed, "tq_quantize_rotated: null pointer");
  LKV_REQUIRE(aligned4(packed), "tq_quantize_rotated: packed must be 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t words = M * (row_bytes_for(bits) / 4);
  int64_t g = (words + kThreads - 1) / kThreads;
  if (g > 8 * device_cu_count()) g = 8 * device_cu_count();
  LKV_BITS_SWITCH(bits, hipLaunchKernelGGL((quantize_rotated_kernel<B_>), dim3(static_cast<unsigned>(g)),
                                           dim3(kThreads), 0, st, y, M, bounds, packed))
  LKV_LAUNCH_CHECK("tq_quantize_rotated");
  return LKV_OK;
}

namespace lkv {
int rotate_rows(const void* x, bool x_f16, int64_t M, const float* Pi, int transpose, void* y, bool y_f16,
                hipStream_t st) {
  if (M == 0) return LKV_OK;
  const int g = grid_for(M);
#define LKV_ROT(IF, OF)                                                                                         \
  hipLaunchKernelGGL((rotate_kernel<kRotate, 4, IF, OF>), dim3(g), dim3(kThreads), 0, st, x, nullptr, M, Pi, \
                     transpose, nullptr, y)
  if (x_f16) {
    if (y_f16) { LKV_ROT(true, true); } else { LKV_ROT(true, false); }
  } else {
    if (y_f16) { LKV_ROT(false, true); } else { LKV_ROT(false, false); }
  }
#undef LKV_ROT
  LKV_LAUNCH_CHECK("tq_rotate");
  return LKV_OK;
}
}  // namespace lkv

extern "C" int lkv_tq_rotate(const void* x, int x_dtype, int64_t M, const float* Pi, int transpose,
                             float* y, void* stream) {
  LKV_REQUIRE(M >= 0, "tq_rotate: negative M");
  LKV_REQUIRE(x_dtype == LKV_DTYPE_F32 || x_dtype == LKV_DTYPE_F16, "tq_rotate: x dtype must be f32/f16");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(x && Pi && y, "tq_rotate: null pointer");
  LKV_REQUIRE(aligned16(x) && aligned16(Pi) && aligned16(y), "tq_rotate: pointers must be 16-byte aligned");
  return rotate_rows(x, x_dtype == LKV_DTYPE_F16, M, Pi, transpose, y, false, static_cast<hipStream_t>(stream));
}

extern "C" int lkv_tq_dequantize(const uint8_t* packed, const void* norms, int norm_dtype, int64_t M,
                                 const float* Pi, const float* centroids, int bits, void* out,
                                 int out_dtype, void* stream) {
  if (int e = check_bits(bits, "tq_dequantize")) return e;
  LKV_REQUIRE(M >= 0, "tq_dequantize: negative M");
  LKV_REQUIRE(norm_dtype == LKV_DTYPE_F32 || norm_dtype == LKV_DTYPE_F16, "tq_dequantize: bad norm dtype");
  LKV_REQUIRE(out_dtype == LKV_DTYPE_F32 || out_dtype == LKV_DTYPE_F16, "tq_dequantize: bad out dtype");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(packed && norms && Pi && centroids && out, "tq_dequantize: null pointer");
  LKV_REQUIRE(aligned4(packed) && aligned16(out) && aligned16(Pi),
              "tq_dequantize: packed 4-byte, out and Pi 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int g = grid_for(M);
#define LKV_DQ(NF16, OF16)                                                                          \
  LKV_BITS_SWITCH(bits, hipLaunchKernelGGL((rotate_kernel<kDequant, B_, NF16, OF16>), dim3(g),    \
                                           dim3(kThreads), 0, st, packed, norms, M, Pi, 1, centroids, out))
  if (norm_dtype == LKV_DTYPE_F16) {
    if (out_dtype == LKV_DTYPE_F16) { LKV_DQ(true, true) } else { LKV_DQ(true, false) }
  } else {
    if (out_dtype == LKV_DTYPE_F16) { LKV_DQ(false, true) } else { LKV_DQ(false, false) }
  }
#undef LKV_DQ
  LKV_LAUNCH_CHECK("tq_dequantize");
  return LKV_OK;
}

extern "C" int lkv_tq_cache_append(const void* k_new, const void* v_new, void* k_hot, void* v_hot,
                                   uint8_t* k_codes, float* k_norms, uint8_t* v_codes, float* v_norms,
                                   const float* PiK, const float* PiV, const float* bounds, int bits,
                                   const int32_t* pos, int64_t R, int64_t hot_cap, int64_t cap,
                                   void* stream) {
  if (int e = check_bits(bits, "tq_cache_append")) return e;
  LKV_REQUIRE(R >= 0 && hot_cap >= 1 && cap >= 0, "tq_cache_append: bad sizes R=%lld hot_cap=%lld cap=%lld",
              (long long)R, (long long)hot_cap, (long long)cap);
  if (R == 0) return LKV_OK;
  LKV_REQUIRE(k_new && v_new && k_hot && v_hot && k_codes && k_norms && v_codes && v_norms && PiK && PiV &&
                  bounds && pos,
              "tq_cache_append: null pointer");
  LKV_REQUIRE(aligned16(k_new) && aligned16(v_new) && aligned16(k_hot) && aligned16(v_hot) &&
                  aligned16(PiK) && aligned16(PiV) && aligned4(k_codes) && aligned4(v_codes),
              "tq_cache_append: fp16 rows and Pi must be 16-byte aligned, codes 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>((R + kRows - 1) / kRows), 2);
  LKV_BITS_SWITCH(bits, hipLaunchKernelGGL((append_kernel<B_>), grid, dim3(kThreads), 0, st,
                                           static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new),
                                           static_cast<uint16_t*>(k_hot), static_cast<uint16_t*>(v_hot), k_codes,
                                           k_norms, v_codes, v_norms, PiK, PiV, bounds, pos, R, hot_cap, cap))
  LKV_LAUNCH_CHECK("tq_cache_append");
  return LKV_OK;
}
