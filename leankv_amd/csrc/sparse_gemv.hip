// TEAL magnitude-thresholded sparse GEMV and the fused gate/up SwiGLU variant.
//
// Semantics: leankv/teal/kernels/sparse_gemv.py:61-87 (one program sums
// A[z, n] * x[z] over the rows z of its block whose |x[z]| > threshold) and the
// wrapper at :143-181.  The weight arrives in the column-major layout of
// prepare_weight_for_sparse_gemv (:229-234): row z of A[Z][N] is N contiguous
// fp16 values, so a surviving activation selects one contiguous weight row.
//
// Work decomposition (one launch, no host sync, no memset):
//   grid = (N / BN column slabs) x (Z / BZ row chunks), 256 threads per block.
//   1. Compaction: the block reads its BZ activations, tests |x| > t, and
//      builds the list of surviving rows in LDS with a wave ballot and
//      mbcnt lane prefix (plus a 4-entry cross-wave prefix).
//   2. Streaming: BN/8 lanes cover one row segment with 16-byte loads; the
//      256/(BN/8) row slots of the block walk the survivor list, U rows at a
//      time so that U independent 16-byte loads per lane are in flight.
//      Products and sums are fp32.
//   3. The row slots are reduced through LDS; the block writes its BN fp32
//      partial sums to the workspace.
//   4. Split-K ticket: the last block of a column slab to finish (agent-scope
//      release/acquire around an atomic counter) sums the partials of all
//      chunks in chunk order, converts to fp16 once, writes y and resets the
//      counter to zero.  The result is therefore deterministic, unlike the
//      reference's fp16 atomic_add accumulation (:87).
#include <stdlib.h>

#include "common.h"

namespace lkv {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;

__device__ __forceinline__ void fma8(float (&acc)[8], const uint4& w, float xv) {
  const uint32_t p[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] = fmaf(h2f(static_cast<uint16_t>(p[i] & 0xffffu)), xv, acc[2 * i]);
    acc[2 * i + 1] = fmaf(h2f(static_cast<uint16_t>(p[i] >> 16)), xv, acc[2 * i + 1]);
  }
}

template <int SLOTS>
__device__ __forceinline__ void stream_rows(const uint16_t* __restrict__ A, size_t N, int col,
                                            bool colok, const int* __restrict__ idx,
                                            const float* __restrict__ xv, int total, int slot,
                                            float (&acc)[8]) {
  const uint4 zero = make_uint4(0, 0, 0, 0);
  int s = slot;
  for (; s + (kUnroll - 1) * SLOTS < total; s += kUnroll * SLOTS) {
    uint4 w[kUnroll];
    float xs[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = idx[s + u * SLOTS];
      xs[u] = xv[s + u * SLOTS];
      w[u] = colok ? *reinterpret_cast<const uint4*>(A + static_cast<size_t>(r) * N + col) : zero;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) fma8(acc, w[u], xs[u]);
  }
  for (; s < total; s += SLOTS) {
    const int r = idx[s];
    const uint4 w = colok ? *reinterpret_cast<const uint4*>(A + static_cast<size_t>(r) * N + col) : zero;
    fma8(acc, w, xv[s]);
  }
}

// Reduce the SLOTS row-slot accumulators of the block into out[0..BN).
template <int BN, int SLOTS>
__device__ __forceinline__ void block_reduce_cols(float* s_red, const float (&acc)[8], int slot,
                                                  int c, float* out_cols /*BN/kThreads per thread*/) {
  float4* dst = reinterpret_cast<float4*>(s_red + slot * BN + c * 8);
  dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < BN / kThreads; ++j) {
    const int cc = threadIdx.x + j * kThreads;
    float s = 0.f;
#pragma unroll
    for (int sl = 0; sl < SLOTS; ++sl) s += s_red[sl * BN + cc];
    out_cols[j] = s;
  }
  __syncthreads();
}

// SwiGLU epilogue with the rounding of the eager fp16 torch sequence
// silu(fp16 g) -> fp16, times fp16 u -> fp16.
__device__ __forceinline__ uint16_t swiglu_f16(float g, float u) {
  const float g16 = h2f(f2h(g));
  const float u16 = h2f(f2h(u));
  const float s16 = h2f(f2h(g16 / (1.0f + expf(-g16))));
  return f2h(s16 * u16);
}

template <int BN, int BZ, bool DUAL>
__global__ __launch_bounds__(kThreads) void sparse_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ A0,
    const uint16_t* __restrict__ A1, float t0, float t1, int N, int Z, int nchunk,
    uint16_t* __restrict__ y, float* __restrict__ partials, unsigned* __restrict__ tickets) {
  constexpr int LPR = BN / 8;            // lanes per row segment
  constexpr int SLOTS = kThreads / LPR;  // rows processed side by side
  constexpr int NL = DUAL ? 2 : 1;
  static_assert(BN % kThreads == 0 && LPR <= kThreads, "BN must be 256..2048");

  __shared__ int s_idx[NL][BZ];
  __shared__ float s_xv[NL][BZ];
  __shared__ int s_cnt[NL][kThreads / kWave];
  __shared__ __align__(16) float s_red[SLOTS * BN];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int slab = blockIdx.x;
  const int chunk = blockIdx.y;
  const int nslab = gridDim.x;
  const int n0 = slab * BN;
  const int z0 = chunk * BZ;

  // ---- 1. compaction of surviving activation rows
  int total[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) total[l] = 0;
  for (int base = 0; base < BZ; base += kThreads) {
    const int z = z0 + base + tid;
    const bool valid = (base + tid < BZ) && (z < Z);
    const float v = valid ? h2f(x[z]) : 0.f;
    const float a = fabsf(v);
    bool pred[NL];
    uint64_t mask[NL];
    pred[0] = valid && (a > t0);
    if (DUAL) pred[NL - 1] = valid && (a > t1);
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      mask[l] = wave_ballot(pred[l]);
      if (lane == 0) s_cnt[l][wave] = __popcll(mask[l]);
    }
    __syncthreads();
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      int off = total[l], tot = 0;
#pragma unroll
      for (int w = 0; w < kThreads / kWave; ++w) {
        const int cw = s_cnt[l][w];
        off += (w < wave) ? cw : 0;
        tot += cw;
      }
      if (pred[l]) {
        const int pos = off + lane_prefix(mask[l]);
        s_idx[l][pos] = z;
        s_xv[l][pos] = v;
      }
      total[l] += tot;
    }
    __syncthreads();
  }

  // ---- 2. stream surviving weight rows
  const int c = tid % LPR;
  const int slot = tid / LPR;
  const int col = n0 + c * 8;
  const bool colok = col < N;
  float acc[NL][8];
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[l][j] = 0.f;
  stream_rows<SLOTS>(A0, static_cast<size_t>(N), col, colok, s_idx[0], s_xv[0], total[0], slot, acc[0]);
  if (DUAL)
    stream_rows<SLOTS>(A1, static_cast<size_t>(N), col, colok, s_idx[NL - 1], s_xv[NL - 1],
                       total[NL - 1], slot, acc[NL - 1]);

  // ---- 3. cross-slot reduction through LDS
  float sums[NL][BN / kThreads];
#pragma unroll
  for (int l = 0; l < NL; ++l) block_reduce_cols<BN, SLOTS>(s_red, acc[l], slot, c, sums[l]);

  if (nchunk == 1) {
#pragma unroll
    for (int j = 0; j < BN / kThreads; ++j) {
      const int n = n0 + tid + j * kThreads;
      if (n < N) y[n] = DUAL ? swiglu_f16(sums[0][j], sums[NL - 1][j]) : f2h(sums[0][j]);
    }
    return;
  }

  // ---- 4. split-K: partials, ticket, last block reduces in chunk order
  const size_t mat_stride = static_cast<size_t>(nslab) * nchunk * BN;
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float* P = partials + l * mat_stride + (static_cast<size_t>(slab) * nchunk + chunk) * BN;
#pragma unroll
    for (int j = 0; j < BN / kThreads; ++j) P[tid + j * kThreads] = sums[l][j];
  }
  fence_release_agent();
  __syncthreads();
  if (tid == 0) s_last = (ticket_add(&tickets[slab]) == static_cast<unsigned>(nchunk - 1));
  __syncthreads();
  if (!s_last) return;
  fence_acquire_agent();
#pragma unroll
  for (int j = 0; j < BN / kThreads; ++j) {
    const int cc = tid + j * kThreads;
    const int n = n0 + cc;
    float r[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      const float* P = partials + l * mat_stride + static_cast<size_t>(slab) * nchunk * BN + cc;
      float s = 0.f;
      for (int k = 0; k < nchunk; ++k) s += P[static_cast<size_t>(k) * BN];
      r[l] = s;
    }
    if (n < N) y[n] = DUAL ? swiglu_f16(r[0], r[NL - 1]) : f2h(r[0]);
  }
  if (tid == 0) ticket_reset(&tickets[slab]);
}

struct GemvCfg {
  int bn;
  int bz;
};

// Shapes are chosen so that the grid holds at least ~2 blocks per CU while
// each block streams as many rows as possible (fewer partials to reduce).
GemvCfg pick_cfg(int64_t N, int64_t Z, bool dual) {
  const char* env = getenv(dual ? "LKV_GATEUP_CFG" : "LKV_GEMV_CFG");
  if (env) {
    int bn = 0, bz = 0;
    if (sscanf(env, "%d,%d", &bn, &bz) == 2) return {bn, bz};
  }
  const int64_t target = 2 * static_cast<int64_t>(device_cu_count());
  const int bn = (N >= 2048) ? 512 : 256;
  const int64_t nslab = (N + bn - 1) / bn;
  static const int bzs[] = {512, 256, 128, 64};
  for (int bz : bzs) {
    const int64_t nchunk = (Z + bz - 1) / bz;
    if (nslab * nchunk >= target) return {bn, bz};
  }
  return {bn, 64};
}

size_t ws_bytes_for(const GemvCfg& c, int64_t N, int64_t Z, bool dual) {
  const int64_t nslab = (N + c.bn - 1) / c.bn;
  const int64_t nchunk = Z > 0 ? (Z + c.bz - 1) / c.bz : 1;
  const size_t tick = ((static_cast<size_t>(nslab) * 4 + 255) / 256) * 256;
  return tick + static_cast<size_t>(dual ? 2 : 1) * nslab * nchunk * c.bn * sizeof(float);
}

template <bool DUAL>
int launch(const GemvCfg& cfg, const void* x, const void* A0, const void* A1, float t0, float t1,
           int64_t N, int64_t Z, void* y, void* ws, hipStream_t st) {
  const int64_t nslab = (N + cfg.bn - 1) / cfg.bn;
  const int64_t nchunk = Z > 0 ? (Z + cfg.bz - 1) / cfg.bz : 1;
  const size_t tick = ((static_cast<size_t>(nslab) * 4 + 255) / 256) * 256;
  unsigned* tickets = static_cast<unsigned*>(ws);
  float* partials = reinterpret_cast<float*>(static_cast<char*>(ws) + tick);
  dim3 grid(static_cast<unsigned>(nslab), static_cast<unsigned>(nchunk));
  const uint16_t* xx = static_cast<const uint16_t*>(x);
  const uint16_t* a0 = static_cast<const uint16_t*>(A0);
  const uint16_t* a1 = static_cast<const uint16_t*>(A1);
  uint16_t* yy = static_cast<uint16_t*>(y);
  const int n = static_cast<int>(N), z = static_cast<int>(Z), nc = static_cast<int>(nchunk);
#define LKV_GEMV_CASE(BN_, BZ_)                                                                 \
  if (cfg.bn == BN_ && cfg.bz == BZ_) {                                                         \
    hipLaunchKernelGGL((sparse_gemv_kernel<BN_, BZ_, DUAL>), grid, dim3(kThreads), 0, st, xx, a0, \
                       a1, t0, t1, n, z, nc, yy, partials, tickets);                             \
    LKV_LAUNCH_CHECK("sparse_gemv");                                                            \
    return LKV_OK;                                                                              \
  }
  LKV_GEMV_CASE(256, 64)
  LKV_GEMV_CASE(256, 128)
  LKV_GEMV_CASE(256, 256)
  LKV_GEMV_CASE(256, 512)
  LKV_GEMV_CASE(512, 64)
  LKV_GEMV_CASE(512, 128)
  LKV_GEMV_CASE(512, 256)
  LKV_GEMV_CASE(512, 512)
  LKV_GEMV_CASE(1024, 128)
  LKV_GEMV_CASE(1024, 256)
  LKV_GEMV_CASE(1024, 512)
#undef LKV_GEMV_CASE
  set_error("sparse_gemv: no kernel instantiated for BN=%d BZ=%d", cfg.bn, cfg.bz);
  return LKV_ERR_INVALID;
}

int check_common(const void* x, const void* A, int64_t N, int64_t Z, const void* y) {
  LKV_REQUIRE(N >= 0 && Z >= 0, "sparse_gemv: negative size N=%lld Z=%lld", (long long)N, (long long)Z);
  LKV_REQUIRE(N <= (1ll << 30) && Z <= (1ll << 30), "sparse_gemv: size too large");
  LKV_REQUIRE(N % 8 == 0, "sparse_gemv: N=%lld must be a multiple of 8 (16-byte weight rows)",
              (long long)N);
  LKV_REQUIRE(x && A && y, "sparse_gemv: null pointer");
  LKV_REQUIRE((aligned16(A) && aligned16(y)) || (N == 0),
              "sparse_gemv: weight and output must be 16-byte aligned");
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_sparse_gemv_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return 256;
  return ws_bytes_for(pick_cfg(N, Z, false), N, Z, false);
}

extern "C" size_t lkv_sparse_gateup_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return 256;
  return ws_bytes_for(pick_cfg(N, Z, true), N, Z, true);
}

extern "C" int lkv_sparse_gemv(const void* x, const void* w, float threshold, int64_t N, int64_t Z,
                               void* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_common(x, w, N, Z, y)) return e;
  if (N == 0) return LKV_OK;
  const GemvCfg cfg = pick_cfg(N, Z, false);
  const size_t need = ws_bytes_for(cfg, N, Z, false);
  LKV_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
              "sparse_gemv: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
              workspace_bytes);
  return launch<false>(cfg, x, w, w, threshold, threshold, N, Z, y, workspace,
                       static_cast<hipStream_t>(stream));
}

extern "C" int lkv_sparse_gateup_swiglu(const void* x, const void* wg, const void* wu, float t_gate,
                                        float t_up, int64_t N, int64_t Z, void* h, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  if (int e = check_common(x, wg, N, Z, h)) return e;
  LKV_REQUIRE(wu && (aligned16(wu) || N == 0), "sparse_gateup: up weight must be 16-byte aligned");
  if (N == 0) return LKV_OK;
  const GemvCfg cfg = pick_cfg(N, Z, true);
  const size_t need = ws_bytes_for(cfg, N, Z, true);
  LKV_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
              "sparse_gateup: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
              workspace_bytes);
  return launch<true>(cfg, x, wg, wu, t_gate, t_up, N, Z, h, workspace,
                      static_cast<hipStream_t>(stream));
}
