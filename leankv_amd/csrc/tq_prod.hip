// TurboQuantProd: MSE codes at mse_bits plus a 1-bit QJL sketch of the residual,
// quantize and dequantize at head_dim 128.
//
// Semantics: leankv/turboquant/quantizer.py:144-237 with rotation.py:32-52.
//   quantize:   codes, norm = TurboQuantMSE(mse_bits).quantize(x)
//               x_hat = (centroid[codes] @ Pi) * norm;  r = x - x_hat  (fp32)
//               rnorm = ||r||;  signs: bit i of byte j = [(r @ S^T)[8j + i] > 0]
//   dequantize: (centroid[codes] @ Pi) * norm + (s @ S) * (qjl_scale * rnorm),  s = +1 / -1
//
// Every 128x128 product is the fp32 MFMA chain of rotate_tile (same 32
// k-steps, same operands, same order), so the codes equal lkv_tq_quantize's,
// x_hat equals lkv_tq_dequantize's fp32 output and r @ S^T equals
// lkv_tq_rotate(r, S)'s bit for bit: the fused kernel gives the signs the
// separate kernels would.  Three 16x128x128 products per 16-vector tile make
// the quantize kernel fp32-MFMA bound (98 KFLOP per vector against ~300 B).
// Pi's forward and backward operands stay in registers (two rotate_tile B
// operands); S is staged once per block in LDS in MFMA operand order,
// s_s[w][t][kq][lane] = S[8n + 2w + t][32q + 4kq .. +3] for lane = 16q + n, one
// conflict-free 16-byte read per k-quarter.
#include "tq_common.h"

namespace lkv {
namespace {

using namespace tq;

template <int MB, bool F16>
__global__ __launch_bounds__(kThreads, 2) void prod_quantize_kernel(
    const void* __restrict__ xin, int64_t M, const float* __restrict__ Pi, const float* __restrict__ bounds,
    const float* __restrict__ centroids, const float* __restrict__ S, uint8_t* __restrict__ codes,
    void* __restrict__ norms, uint8_t* __restrict__ signs, float* __restrict__ rnorms) {
#pragma clang fp contract(off)
  constexpr int NC = 1 << MB;
  __shared__ float4 s_s[4][2][8][65];                // S operand, 64 KB + a float4 of padding per row
  __shared__ __align__(16) float s_xh[kRows][kD + 4];  // x_hat of the tile
  __shared__ __align__(16) uint8_t s_codes[kRows * kD];
  __shared__ uint8_t s_bits[4][kRows][16];           // sign bits per wave (2 of every byte)
  __shared__ float s_tab[16];
  __shared__ float s_norm[kRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, q = lane >> 4;
  if (threadIdx.x < 16) s_tab[threadIdx.x] = centroids[threadIdx.x < NC ? threadIdx.x : NC - 1];
#pragma unroll 4
  for (int i = 0; i < kD * kD / 4 / kThreads; ++i) {
    const int f = i * kThreads + threadIdx.x;  // float4 f: S row f / 32, columns 4 (f % 32) ..
    const int j = f >> 5, c4 = f & 31;
    s_s[(j & 7) >> 1][j & 1][c4 & 7][16 * (c4 >> 3) + (j >> 3)] = reinterpret_cast<const float4*>(S)[f];
  }
  float bd[NC - 1];
#pragma unroll
  for (int i = 0; i < NC - 1; ++i) bd[i] = bounds[i];
  float bf[2][32], bb[2][32];
  load_pi_operand(Pi, false, wave, lane, bf);  // x @ Pi^T
  load_pi_operand(Pi, true, wave, lane, bb);   // y @ Pi
  __syncthreads();
  const int64_t ntiles = (M + kRows - 1) / kRows;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kRows;
    const int64_t r = row0 + n;
    float xo[32];
    if (r < M) {
      if (F16)
        load_row_f16(static_cast<const uint16_t*>(xin) + r * kD + 32 * q, xo);
      else
        load_row_f32(static_cast<const float*>(xin) + r * kD + 32 * q, xo);
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) xo[s] = 0.f;
    }
    float a[32];
#pragma unroll
    for (int s = 0; s < 32; ++s) a[s] = xo[s];
    const float nrm = normalize_row<F16>(a);
    if (wave == 0 && lane < 16) {
      s_norm[n] = nrm;
      if (r < M) {
        if (F16)
          static_cast<uint16_t*>(norms)[r] = f2h(nrm);
        else
          static_cast<float*>(norms)[r] = nrm;
      }
    }
    f32x4 acc[2];
    rotate_tile(a, bf, acc);
    codes_to_lds<MB>(acc, bd, wave, lane, s_codes);
    __syncthreads();  // codes and norms of the tile
    pack_store<MB>(s_codes, codes, row0, M,
                   [](int64_t rr) { return rr * static_cast<int64_t>(row_bytes_for(MB)); });
    // x_hat = (centroid[codes] @ Pi) * norm, A operand: vector n, dims 32q ..
    {
      const uint4* cp = reinterpret_cast<const uint4*>(s_codes + n * kD + 32 * q);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 u = cp[h];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) a[16 * h + e] = s_tab[(w[e >> 2] >> (8 * (e & 3))) & 0xffu];
      }
    }
    rotate_tile(a, bb, acc);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_xh[4 * q + i][8 * n + 2 * wave + t] = acc[t][i] * s_norm[4 * q + i];
    __syncthreads();  // x_hat of the tile
    // residual in A layout and its norm
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float4 h = *reinterpret_cast<const float4*>(&s_xh[n][32 * q + 4 * v]);
      a[4 * v] = xo[4 * v] - h.x;
      a[4 * v + 1] = xo[4 * v + 1] - h.y;
      a[4 * v + 2] = xo[4 * v + 2] - h.z;
      a[4 * v + 3] = xo[4 * v + 3] - h.w;
    }
#pragma unroll
    for (int s = 0; s < 32; ++s) ss = fmaf(a[s], a[s], ss);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (wave == 0 && lane < 16 && r < M) rnorms[r] = sqrtf(ss);
    // r @ S^T, B operand from LDS in rotate_tile's k order
    acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kq = 0; kq < 8; ++kq) {
      const float4 b0 = s_s[wave][0][kq][lane];
      const float4 b1 = s_s[wave][1][kq][lane];
      const float x0[4] = {b0.x, b0.y, b0.z, b0.w};
      const float x1[4] = {b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * kq + cc], x0[cc], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * kq + cc], x1[cc], acc[1], 0, 0, 0);
      }
    }
    // dim 8n + 2w + t is bit 2w + t of sign byte n
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s_bits[wave][4 * q + i][n] =
          static_cast<uint8_t>(((acc[0][i] > 0.f ? 1u : 0u) | (acc[1][i] > 0.f ? 2u : 0u)) << (2 * wave));
    __syncthreads();  // sign bits of the tile
    if (threadIdx.x < kRows * 4) {
      const int row = threadIdx.x >> 2, dw = threadIdx.x & 3;
      uint32_t v = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int b = 4 * dw + e;
        v |= static_cast<uint32_t>(s_bits[0][row][b] | s_bits[1][row][b] | s_bits[2][row][b] | s_bits[3][row][b])
             << (8 * e);
      }
      if (row0 + row < M) *reinterpret_cast<uint32_t*>(signs + (row0 + row) * 16 + 4 * dw) = v;
    }
    // No barrier here: the next tile writes s_norm, s_codes, s_xh and s_bits
    // only after barriers that every reader of this tile's values has passed.
  }
}

template <int MB, bool NF16, bool OF16>
__global__ __launch_bounds__(kThreads, 2) void prod_dequantize_kernel(
    const uint8_t* __restrict__ codes, const void* __restrict__ norms_in, const uint8_t* __restrict__ signs,
    const float* __restrict__ rnorms, int64_t M, const float* __restrict__ Pi, const float* __restrict__ centroids,
    const float* __restrict__ S, float qjl_scale, void* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr int NC = 1 << MB;
  constexpr int PB = pack_bits(MB);
  constexpr int RB = row_bytes_for(MB);
  __shared__ __align__(16) float s_out[kRows * kD];
  __shared__ float s_tab[16];
  __shared__ float s_norm[kRows];
  __shared__ float s_scale[kRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, q = lane >> 4;
  if (threadIdx.x < 16) s_tab[threadIdx.x] = centroids[threadIdx.x < NC ? threadIdx.x : NC - 1];
  float bp[2][32], bs[2][32];
  load_pi_operand(Pi, true, wave, lane, bp);  // y @ Pi
  load_pi_operand(S, true, wave, lane, bs);   // s @ S
  const int64_t ntiles = (M + kRows - 1) / kRows;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kRows;
    const int64_t r = row0 + n;
    if (threadIdx.x < kRows) {
      const int64_t rr = row0 + threadIdx.x;
      float nv = 0.f, sc = 0.f;
      if (rr < M) {
        nv = NF16 ? h2f(static_cast<const uint16_t*>(norms_in)[rr]) : static_cast<const float*>(norms_in)[rr];
        sc = qjl_scale * rnorms[rr];
      }
      s_norm[threadIdx.x] = nv;
      s_scale[threadIdx.x] = sc;
    }
    __syncthreads();  // centroid table, norms and scales of the tile
    float a[32], sg[32];
    if (r < M) {
      // the 32 codes of dims 32q .. 32q + 31 occupy 4 * PB bytes
      const uint32_t* src = reinterpret_cast<const uint32_t*>(codes + r * RB + q * 4 * PB);
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < PB; ++i) w[i] = src[i];
#pragma unroll
      for (int s = 0; s < 32; ++s) {
        const int bit = s * PB;
        a[s] = s_tab[(w[bit >> 5] >> (bit & 31)) & ((1u << PB) - 1u)];
      }
      const uint32_t sb = *reinterpret_cast<const uint32_t*>(signs + r * 16 + 4 * q);
#pragma unroll
      for (int s = 0; s < 32; ++s) sg[s] = ((sb >> s) & 1u) ? 1.f : -1.f;
    } else {
#pragma unroll
      for (int s = 0; s < 32; ++s) a[s] = sg[s] = 0.f;
    }
    f32x4 am[2], aq[2];
    rotate_tile(a, bp, am);
    rotate_tile(sg, bs, aq);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * q + i;
        const float x_mse = am[t][i] * s_norm[row];
        const float x_qjl = aq[t][i] * s_scale[row];
        s_out[row * kD + 8 * n + 2 * wave + t] = x_mse + x_qjl;
      }
    __syncthreads();  // the tile's output rows
    {
      const int row = threadIdx.x >> 4;
      const int c0 = (threadIdx.x & 15) * 8;
      const int64_t rg = row0 + row;
      if (rg < M) {
        const float* v = s_out + row * kD + c0;
        if (OF16) {
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
    __syncthreads();  // s_out, s_norm and s_scale are rewritten by the next tile
  }
}

int prod_grid(int64_t M) {
  const int64_t ntiles = (M + kRows - 1) / kRows;
  const int64_t g = 2 * static_cast<int64_t>(device_cu_count());
  return static_cast<int>(ntiles < g ? (ntiles > 0 ? ntiles : 1) : g);
}

}  // namespace
}  // namespace lkv

using namespace lkv;

#define LKV_MB_SWITCH(mb, ...)                              \
  switch (mb) {                                             \
    case 1: { constexpr int MB_ = 1; __VA_ARGS__; break; } \
    case 2: { constexpr int MB_ = 2; __VA_ARGS__; break; } \
    case 3: { constexpr int MB_ = 3; __VA_ARGS__; break; } \
    default: { constexpr int MB_ = 4; __VA_ARGS__; break; } \
  }

extern "C" int lkv_tq_prod_quantize(const void* x, int x_dtype, int64_t M, const float* Pi, const float* bounds,
                                    const float* centroids, const float* S, int mse_bits, uint8_t* codes,
                                    void* norms, uint8_t* signs, float* rnorms, void* stream) {
  LKV_REQUIRE(mse_bits >= 1 && mse_bits <= 4, "tq_prod_quantize: mse_bits=%d unsupported (1..4)", mse_bits);
  LKV_REQUIRE(M >= 0, "tq_prod_quantize: negative M");
  LKV_REQUIRE(x_dtype == LKV_DTYPE_F32 || x_dtype == LKV_DTYPE_F16, "tq_prod_quantize: x dtype must be f32/f16");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(x && Pi && bounds && centroids && S && codes && norms && signs && rnorms,
              "tq_prod_quantize: null pointer");
  LKV_REQUIRE(aligned16(x) && aligned16(Pi) && aligned16(S) && aligned4(codes) && aligned4(signs),
              "tq_prod_quantize: x, Pi and S must be 16-byte aligned, codes and signs 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int g = prod_grid(M);
  if (x_dtype == LKV_DTYPE_F16) {
    LKV_MB_SWITCH(mse_bits, hipLaunchKernelGGL((prod_quantize_kernel<MB_, true>), dim3(g), dim3(kThreads), 0, st,
                                               x, M, Pi, bounds, centroids, S, codes, norms, signs, rnorms))
  } else {
    LKV_MB_SWITCH(mse_bits, hipLaunchKernelGGL((prod_quantize_kernel<MB_, false>), dim3(g), dim3(kThreads), 0, st,
                                               x, M, Pi, bounds, centroids, S, codes, norms, signs, rnorms))
  }
  LKV_LAUNCH_CHECK("tq_prod_quantize");
  return LKV_OK;
}

extern "C" int lkv_tq_prod_dequantize(const uint8_t* codes, const void* norms, int norm_dtype, const uint8_t* signs,
                                      const float* rnorms, int64_t M, const float* Pi, const float* centroids,
                                      const float* S, int mse_bits, float qjl_scale, void* out, int out_dtype,
                                      void* stream) {
  LKV_REQUIRE(mse_bits >= 1 && mse_bits <= 4, "tq_prod_dequantize: mse_bits=%d unsupported (1..4)", mse_bits);
  LKV_REQUIRE(M >= 0, "tq_prod_dequantize: negative M");
  LKV_REQUIRE(norm_dtype == LKV_DTYPE_F32 || norm_dtype == LKV_DTYPE_F16, "tq_prod_dequantize: bad norm dtype");
  LKV_REQUIRE(out_dtype == LKV_DTYPE_F32 || out_dtype == LKV_DTYPE_F16, "tq_prod_dequantize: bad out dtype");
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(codes && norms && signs && rnorms && Pi && centroids && S && out, "tq_prod_dequantize: null pointer");
  LKV_REQUIRE(aligned4(codes) && aligned4(signs) && aligned16(out) && aligned16(Pi) && aligned16(S),
              "tq_prod_dequantize: codes and signs 4-byte, out, Pi and S 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int g = prod_grid(M);
#define LKV_PDQ(NF16, OF16)                                                                                   \
  LKV_MB_SWITCH(mse_bits, hipLaunchKernelGGL((prod_dequantize_kernel<MB_, NF16, OF16>), dim3(g), dim3(kThreads), \
                                             0, st, codes, norms, signs, rnorms, M, Pi, centroids, S, qjl_scale, out))
  if (norm_dtype == LKV_DTYPE_F16) {
    if (out_dtype == LKV_DTYPE_F16) { LKV_PDQ(true, true) } else { LKV_PDQ(true, false) }
  } else {
    if (out_dtype == LKV_DTYPE_F16) { LKV_PDQ(false, true) } else { LKV_PDQ(false, false) }
  }
#undef LKV_PDQ
  LKV_LAUNCH_CHECK("tq_prod_dequantize");
  return LKV_OK;
}
