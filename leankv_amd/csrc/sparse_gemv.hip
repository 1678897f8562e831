// TEAL magnitude-thresholded sparse GEMV and the fused gate/up SwiGLU variant.
//
// Semantics: leankv/teal/kernels/sparse_gemv.py:61-87 (one program sums
// A[z, n] * x[z] over the rows z of its block whose |x[z]| > threshold) and the
// wrapper at :143-181.  The weight arrives in the column-major layout of
// prepare_weight_for_sparse_gemv (:229-234): row z of A[Z][N] is N contiguous
// fp16 values, so a surviving activation selects one contiguous weight row.
//
// Work decomposition:
//   grid = (N / BN column slabs) x (Z / BZ row chunks), 256 threads per block.
//   1. Compaction: the block reads its BZ activations, tests |x| > t, and
//      builds the list of surviving rows in LDS with a wave ballot and mbcnt
//      lane prefix (plus a 4-entry cross-wave prefix).  The list is padded to
//      a whole number of streaming batches with copies of its last row and a
//      zero activation: padded loads hit the line just fetched and add 0.
//   2. Streaming: BN/8 lanes cover one row segment with 16-byte buffer loads
//      (SGPR descriptor + 32-bit offset); the 256/(BN/8) row slots of the
//      block walk the list U rows at a time, so U independent 16-byte loads
//      per lane are in flight.  fp16 x fp32 -> fp32 FMAs.
//   3. The row slots are reduced through LDS into BN fp32 column sums.
//   4. Split-K over the row chunks, two variants:
//      * ticket: the block writes its partials, one thread releases them at
//        agent scope (one L2 write-back per block) and takes a ticket; the
//        last block of the slab sums all chunks in chunk order and writes fp16.
//      * two kernels: the block only writes partials; gemv_reduce_kernel sums
//        them after the kernel boundary.
//      Both reduce in a fixed order, so y is deterministic (the reference
//      accumulates with fp16 atomic_add, :87).
#include <stdlib.h>

#include "common.h"

namespace lkv {
namespace {

constexpr int kThreads = 256;

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void fma8(float (&acc)[8], const u32x4v& w, float xv) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] = fmaf(h2f(static_cast<uint16_t>(w[i] & 0xffffu)), xv, acc[2 * i]);
    acc[2 * i + 1] = fmaf(h2f(static_cast<uint16_t>(w[i] >> 16)), xv, acc[2 * i + 1]);
  }
}

// Buffer descriptor over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Stream the padded survivor list: total is a multiple of kUnroll * SLOTS.
template <int SLOTS, int kUnroll>
__device__ __forceinline__ void stream_rows(__amdgpu_buffer_rsrc_t A, uint32_t row_bytes, uint32_t col_bytes,
                                            const int* __restrict__ idx, const float* __restrict__ xv,
                                            int total, int slot, int aux, float (&acc)[8]) {
  for (int s = slot; s < total; s += kUnroll * SLOTS) {
    int r[kUnroll];
    float xs[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      r[u] = idx[s + u * SLOTS];
      xs[u] = xv[s + u * SLOTS];
    }
    u32x4v w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      w[u] = aux ? __builtin_amdgcn_raw_buffer_load_b128(A, static_cast<uint32_t>(r[u]) * row_bytes + col_bytes, 0, 2)
                 : __builtin_amdgcn_raw_buffer_load_b128(A, static_cast<uint32_t>(r[u]) * row_bytes + col_bytes, 0, 0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) fma8(acc, w[u], xs[u]);
  }
}

// Reduce the SLOTS row-slot accumulators of the block into out[0..BN/256).
template <int BN, int SLOTS>
__device__ __forceinline__ void block_reduce_cols(float* s_red, const float (&acc)[8], int slot, int c,
                                                  float* out_cols) {
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

// Sum nchunk partials spaced `stride` floats apart, in chunk order.  Loads are
// issued 16 at a time so the sum costs ceil(nchunk / 16) memory round trips
// instead of nchunk.
__device__ __forceinline__ float sum_chunks(const float* __restrict__ P, size_t stride, int nchunk) {
  constexpr int kBatch = 16;
  float s = 0.f;
  for (int k0 = 0; k0 < nchunk; k0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) v[i] = (k0 + i < nchunk) ? P[static_cast<size_t>(k0 + i) * stride] : 0.f;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) s += v[i];
  }
  return s;
}

// SwiGLU epilogue with the rounding of the eager fp16 torch sequence
// silu(fp16 g) -> fp16, times fp16 u -> fp16.
__device__ __forceinline__ uint16_t swiglu_f16(float g, float u) {
  const float g16 = h2f(f2h(g));
  const float u16 = h2f(f2h(u));
  const float s16 = h2f(f2h(g16 / (1.0f + expf(-g16))));
  return f2h(s16 * u16);
}

template <int BN, int BZ, bool DUAL, bool TICKET, int kUnroll>
__global__ __launch_bounds__(kThreads) void sparse_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ A0, const uint16_t* __restrict__ A1,
    uint32_t a_bytes, float t0, float t1, int N, int Z, int nchunk, uint16_t* __restrict__ y,
    float* __restrict__ partials, unsigned* __restrict__ tickets, int aux) {
  constexpr int LPR = BN / 8;            // lanes per row segment
  constexpr int SLOTS = kThreads / LPR;  // rows processed side by side
  constexpr int NL = DUAL ? 2 : 1;
  constexpr int PAD = kUnroll * SLOTS;   // list granularity
  static_assert(BN % kThreads == 0 && LPR <= kThreads, "BN must be 256..2048");

  __shared__ int s_idx[NL][BZ + PAD];
  __shared__ float s_xv[NL][BZ + PAD];
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
  // pad each list to a multiple of PAD with (last row, 0)
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const int padded = (total[l] + PAD - 1) / PAD * PAD;
    if (total[l] > 0 && tid < padded - total[l]) {
      s_idx[l][total[l] + tid] = s_idx[l][total[l] - 1];
      s_xv[l][total[l] + tid] = 0.f;
    }
    total[l] = padded;
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
  stream_rows<SLOTS, kUnroll>(make_rsrc(A0, a_bytes), row_bytes, col_bytes, s_idx[0], s_xv[0], total[0], slot,
                              aux, acc[0]);
  if (DUAL)
    stream_rows<SLOTS, kUnroll>(make_rsrc(A1, a_bytes), row_bytes, col_bytes, s_idx[NL - 1], s_xv[NL - 1],
                                total[NL - 1], slot, aux, acc[NL - 1]);

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

  // ---- 4. split-K partials
  const size_t mat_stride = static_cast<size_t>(nslab) * nchunk * BN;
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    float* P = partials + l * mat_stride + (static_cast<size_t>(slab) * nchunk + chunk) * BN;
#pragma unroll
    for (int j = 0; j < BN / kThreads; ++j) P[tid + j * kThreads] = sums[l][j];
  }
  if (!TICKET) return;
  // The barrier completes every thread's partial stores (to this XCD's L2);
  // one agent-scope release by thread 0 then publishes them all.  Only the
  // block that takes the last ticket pays the acquire (L1/L2 invalidate).
  __syncthreads();
  if (tid == 0) {
    fence_release_agent();
    const bool last = ticket_add(&tickets[slab]) == static_cast<unsigned>(nchunk - 1);
    if (last) fence_acquire_agent();
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
#pragma unroll
  for (int j = 0; j < BN / kThreads; ++j) {
    const int cc = tid + j * kThreads;
    const int n = n0 + cc;
    float r[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l)
      r[l] = sum_chunks(partials + l * mat_stride + static_cast<size_t>(slab) * nchunk * BN + cc, BN, nchunk);
    if (n < N) y[n] = DUAL ? swiglu_f16(r[0], r[NL - 1]) : f2h(r[0]);
  }
  if (tid == 0) ticket_reset(&tickets[slab]);
}

// Second kernel of the two-kernel split-K: y[n] = sum over chunks, in order.
template <int BN, bool DUAL>
__global__ __launch_bounds__(kThreads) void gemv_reduce_kernel(const float* __restrict__ partials, int N, int nslab,
                                                               int nchunk, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  if (n >= N) return;
  const int slab = n / BN, cc = n % BN;
  const size_t mat_stride = static_cast<size_t>(nslab) * nchunk * BN;
  const float* P = partials + static_cast<size_t>(slab) * nchunk * BN + cc;
  const float g = sum_chunks(P, BN, nchunk);
  if (DUAL)
    y[n] = swiglu_f16(g, sum_chunks(P + mat_stride, BN, nchunk));
  else
    y[n] = f2h(g);
}

struct GemvCfg {
  int bn;
  int bz;
  bool ticket;
  int unroll;
  int aux;
};

// Shapes are chosen so the grid holds ~1.5-2 blocks per CU while each block
// streams as many rows as possible (fewer partials, fewer per-block costs).
GemvCfg pick_cfg(int64_t N, int64_t Z, bool dual) {
  GemvCfg cfg{256, 512, false, 8, 0};
  const char* mode = getenv("LKV_GEMV_SPLITK");  // "two" (default) or "ticket"
  if (mode && mode[0] == 't' && mode[1] == 'i') cfg.ticket = true;
  if (const char* u = getenv("LKV_GEMV_UNROLL")) cfg.unroll = atoi(u) == 16 ? 16 : 8;
  if (const char* a = getenv("LKV_GEMV_NT")) cfg.aux = atoi(a) ? 1 : 0;
  const char* env = getenv(dual ? "LKV_GATEUP_CFG" : "LKV_GEMV_CFG");
  if (env) {
    int bn = 0, bz = 0;
    if (sscanf(env, "%d,%d", &bn, &bz) == 2) {
      cfg.bn = bn;
      cfg.bz = bz;
      return cfg;
    }
  }
  const int64_t target = 3 * static_cast<int64_t>(device_cu_count()) / 2;
  const int64_t nslab = (N + cfg.bn - 1) / cfg.bn;
  static const int bzs[] = {1024, 512, 256};
  for (int bz : bzs) {
    const int64_t nchunk = (Z + bz - 1) / bz;
    if (nslab * nchunk >= target) {
      cfg.bz = bz;
      return cfg;
    }
  }
  cfg.bz = 256;
  return cfg;
}

size_t ws_bytes_for(const GemvCfg& c, int64_t N, int64_t Z, bool dual) {
  const int64_t nslab = (N + c.bn - 1) / c.bn;
  const int64_t nchunk = Z > 0 ? (Z + c.bz - 1) / c.bz : 1;
  return kTicketBytes + static_cast<size_t>(dual ? 2 : 1) * nslab * nchunk * c.bn * sizeof(float);
}

template <bool DUAL>
int launch(const GemvCfg& cfg, const void* x, const void* A0, const void* A1, float t0, float t1, int64_t N,
           int64_t Z, void* y, void* ws, hipStream_t st) {
  const int64_t nslab = (N + cfg.bn - 1) / cfg.bn;
  const int64_t nchunk = Z > 0 ? (Z + cfg.bz - 1) / cfg.bz : 1;
  if (nslab > kMaxTickets) {
    set_error("sparse_gemv: N=%lld needs %lld column slabs, more than %lld tickets", (long long)N,
              (long long)nslab, (long long)kMaxTickets);
    return LKV_ERR_INVALID;
  }
  unsigned* tickets = static_cast<unsigned*>(ws);
  float* partials = reinterpret_cast<float*>(static_cast<char*>(ws) + kTicketBytes);
  dim3 grid(static_cast<unsigned>(nslab), static_cast<unsigned>(nchunk));
  const uint16_t* xx = static_cast<const uint16_t*>(x);
  const uint16_t* a0 = static_cast<const uint16_t*>(A0);
  const uint16_t* a1 = static_cast<const uint16_t*>(A1);
  uint16_t* yy = static_cast<uint16_t*>(y);
  const uint32_t a_bytes = static_cast<uint32_t>(N * Z * 2);
  const int n = static_cast<int>(N), z = static_cast<int>(Z), nc = static_cast<int>(nchunk);
  const bool ticket = cfg.ticket || nchunk == 1;
  bool launched = false;
#define LKV_GEMV_LAUNCH(BN_, BZ_, T_, U_)                                                                    \
  hipLaunchKernelGGL((sparse_gemv_kernel<BN_, BZ_, DUAL, T_, U_>), grid, dim3(kThreads), 0, st, xx, a0, a1,      \
                     a_bytes, t0, t1, n, z, nc, yy, partials, tickets, cfg.aux)
#define LKV_GEMV_CASE(BN_, BZ_)                                                                              \
  if (!launched && cfg.bn == BN_ && cfg.bz == BZ_) {                                                          \
    if (ticket) {                                                                                            \
      if (cfg.unroll == 16) LKV_GEMV_LAUNCH(BN_, BZ_, true, 16); else LKV_GEMV_LAUNCH(BN_, BZ_, true, 8);    \
    } else {                                                                                                 \
      if (cfg.unroll == 16) LKV_GEMV_LAUNCH(BN_, BZ_, false, 16); else LKV_GEMV_LAUNCH(BN_, BZ_, false, 8);  \
    }                                                                                                        \
    launched = true;                                                                                         \
  }
  LKV_GEMV_CASE(256, 256)
  LKV_GEMV_CASE(256, 512)
  LKV_GEMV_CASE(256, 1024)
  LKV_GEMV_CASE(512, 512)
  LKV_GEMV_CASE(1024, 256)
#undef LKV_GEMV_CASE
#undef LKV_GEMV_LAUNCH
  if (!launched) {
    set_error("sparse_gemv: no kernel instantiated for BN=%d BZ=%d", cfg.bn, cfg.bz);
    return LKV_ERR_INVALID;
  }
  LKV_LAUNCH_CHECK("sparse_gemv");
  if (!ticket) {
    const unsigned rgrid = static_cast<unsigned>((N + kThreads - 1) / kThreads);  // kReduceThreads per block
    switch (cfg.bn) {
      case 256:
        hipLaunchKernelGGL((gemv_reduce_kernel<256, DUAL>), dim3(rgrid), dim3(kThreads), 0, st, partials, n,
                           static_cast<int>(nslab), nc, yy);
        break;
      case 512:
        hipLaunchKernelGGL((gemv_reduce_kernel<512, DUAL>), dim3(rgrid), dim3(kThreads), 0, st, partials, n,
                           static_cast<int>(nslab), nc, yy);
        break;
      case 1024:
        hipLaunchKernelGGL((gemv_reduce_kernel<1024, DUAL>), dim3(rgrid), dim3(kThreads), 0, st, partials, n,
                           static_cast<int>(nslab), nc, yy);
        break;
      default:
        hipLaunchKernelGGL((gemv_reduce_kernel<2048, DUAL>), dim3(rgrid), dim3(kThreads), 0, st, partials, n,
                           static_cast<int>(nslab), nc, yy);
        break;
    }
    LKV_LAUNCH_CHECK("sparse_gemv reduce");
  }
  return LKV_OK;
}

int check_common(const void* x, const void* A, int64_t N, int64_t Z, const void* y) {
  LKV_REQUIRE(N >= 0 && Z >= 0, "sparse_gemv: negative size N=%lld Z=%lld", (long long)N, (long long)Z);
  LKV_REQUIRE(N % 8 == 0, "sparse_gemv: N=%lld must be a multiple of 8 (16-byte weight rows)", (long long)N);
  LKV_REQUIRE(N * Z * 2 < (1ll << 32),
              "sparse_gemv: weight of %lld bytes exceeds the 4 GiB buffer-descriptor range", (long long)(N * Z * 2));
  LKV_REQUIRE(x && A && y, "sparse_gemv: null pointer");
  LKV_REQUIRE((aligned16(A) && aligned16(y)) || (N == 0), "sparse_gemv: weight and output must be 16-byte aligned");
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_sparse_gemv_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return kTicketBytes;
  return ws_bytes_for(pick_cfg(N, Z, false), N, Z, false);
}

extern "C" size_t lkv_sparse_gateup_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return kTicketBytes;
  return ws_bytes_for(pick_cfg(N, Z, true), N, Z, true);
}

extern "C" int lkv_sparse_gemv(const void* x, const void* w, float threshold, int64_t N, int64_t Z, void* y,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_common(x, w, N, Z, y)) return e;
  if (N == 0) return LKV_OK;
  const GemvCfg cfg = pick_cfg(N, Z, false);
  const size_t need = ws_bytes_for(cfg, N, Z, false);
  LKV_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
              "sparse_gemv: workspace of %zu bytes (16-byte aligned) required, got %zu", need, workspace_bytes);
  return launch<false>(cfg, x, w, w, threshold, threshold, N, Z, y, workspace, static_cast<hipStream_t>(stream));
}

extern "C" int lkv_sparse_gateup_swiglu(const void* x, const void* wg, const void* wu, float t_gate, float t_up,
                                        int64_t N, int64_t Z, void* h, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  if (int e = check_common(x, wg, N, Z, h)) return e;
  LKV_REQUIRE(wu && (aligned16(wu) || N == 0), "sparse_gateup: up weight must be 16-byte aligned");
  if (N == 0) return LKV_OK;
  const GemvCfg cfg = pick_cfg(N, Z, true);
  const size_t need = ws_bytes_for(cfg, N, Z, true);
  LKV_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
              "sparse_gateup: workspace of %zu bytes (16-byte aligned) required, got %zu", need, workspace_bytes);
  return launch<true>(cfg, x, wg, wu, t_gate, t_up, N, Z, h, workspace, static_cast<hipStream_t>(stream));
}
