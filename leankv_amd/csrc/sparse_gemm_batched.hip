// TEAL sparse GEMM for B > 1 decode rows, each with its own activation mask.
//
// Semantics: leankv/teal/kernels/sparse_gemv.py:92-138 (_batched_sparse_gemm_kernel:
// per (output block, input block, batch item) program, rows with
// |x[b][z]| > threshold contribute A[z, :] * x[b][z], fp32 tile sums) and its
// wrapper :184-226 (x [B, Z], weight [N, Z] column-major, output fp16
// [B, N]).  The reference accumulates with atomic_add into an output it does
// not zero; here every output is the deterministic chunk-ordered sum, equal to
// B independent lkv_sparse_gemv calls up to fp32 summation order (rows are
// accumulated in pairs by v_dot2_f32_f16).
//
// A weight row is needed by a block as soon as one of its batch items keeps
// that activation, and then serves all of them: grid = (column slabs of 256) x
// (row chunks of BZ) x (groups of up to 8 batch rows).  The block compacts the
// union of its rows' masks into an LDS list (per row, the NB activations with
// the ones at or below the threshold zeroed), streams each listed 512-byte
// row segment once with 16-byte buffer loads (batches of 4 rows per lane, the
// next batch in flight while the current one is summed; non-temporal) and
// accumulates NB x 8 fp32 column sums per lane, two rows per
// v_dot2_f32_f16; row slots
// are reduced through LDS and the block writes fp32 partials per batch row,
// summed over chunks in chunk order by batched_reduce_kernel (or written as
// fp16 directly when there is one chunk).  At 40 % sparsity and B = 4 the
// union keeps ~97 % of the rows: one pass over ~the dense weight instead of
// 4 x 60 % of it.
#include "kernels.h"

namespace lkv {
namespace {

constexpr int kNT = 256;
constexpr int kBN = kGemvBN;    // columns per slab
constexpr int kLPR = kBN / 8;   // lanes per row segment
constexpr int kSlots = kNT / kLPR;
constexpr int kU = 4;           // rows per lane per batch (8, pipelined: 27.6 vs 26.2 us at B = 8, config-1 shape)
constexpr int kPad = kU * kSlots;

typedef uint32_t u32x4b __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

struct BatchedArgs {
  const uint16_t* x;  // [B][Z] fp16
  const uint16_t* A;  // [Z][N] fp16 (column-major weight)
  uint32_t a_bytes;
  float t;
  int B, N, Z, nchunk, nslab;
  float* part;        // [B][nslab][nchunk][256] fp32 (nchunk > 1)
  uint16_t* y;        // [B][N] fp16 (written directly when nchunk == 1)
};

template <int NB, int BZ>
__global__ __launch_bounds__(kNT) void sparse_gemm_batched_kernel(BatchedArgs P) {
  static_assert(BZ % kNT == 0, "BZ must be a multiple of the block size");
  __shared__ float s_x[NB][BZ];
  __shared__ int s_idx[BZ + kPad];
  __shared__ __align__(4) uint16_t s_xh[NB][BZ + kPad];  // fp16 activations of the listed rows (0 if dropped)
  __shared__ int s_cnt[kNT / kWave];
  __shared__ __align__(16) float s_red[kSlots * kBN];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int slab = blockIdx.x, chunk = blockIdx.y;
  const int b0 = blockIdx.z * NB;
  const int nb = min(NB, P.B - b0);
  const int z0 = chunk * BZ, n0 = slab * kBN;
  const int Z = P.Z, N = P.N;

  // ---- 0. the group's activations (0 past Z and past the last batch row).
  // Every load is issued before the first is used (address clamped to element
  // 0, value selected afterwards): a conditional load compiles to a branch and
  // a wait per element, NB x BZ / kNT memory round trips in a row.
  {
    constexpr int E = BZ / kNT;
    uint16_t raw[NB][E];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int z = z0 + e * kNT + tid;
        const bool ok = b < nb && z < Z;
        raw[b][e] = P.x[ok ? static_cast<size_t>(b0 + b) * Z + z : 0];
      }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int z = z0 + e * kNT + tid;
        s_x[b][e * kNT + tid] = (b < nb && z < Z) ? h2f(raw[b][e]) : 0.f;
      }
  }
  __syncthreads();

  // ---- 1. compaction of the rows some batch row keeps (strict |x| > t)
  int total = 0;
#pragma unroll
  for (int base = 0; base < BZ; base += kNT) {
    const int z = z0 + base + tid;
    bool keep = false;
    float v[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float xv = s_x[b][base + tid];
      const bool k = fabsf(xv) > P.t;
      v[b] = k ? xv : 0.f;
      keep = keep || k;
    }
    keep = keep && z < Z;
    const uint64_t mask = wave_ballot(keep);
    if (lane == 0) s_cnt[wave] = __popcll(mask);
    __syncthreads();
    int off = total, tot = 0;
#pragma unroll
    for (int w = 0; w < kNT / kWave; ++w) {
      const int cw = s_cnt[w];
      off += (w < wave) ? cw : 0;
      tot += cw;
    }
    if (keep) {
      const int pos = off + lane_prefix(mask);
      s_idx[pos] = z;
#pragma unroll
      for (int b = 0; b < NB; ++b) s_xh[b][pos] = f2h(v[b]);  // exact: fp16 inputs
    }
    total += tot;
    __syncthreads();
  }
  // pad to a multiple of kPad with (last row, zero activations)
  const int padded = (total + kPad - 1) / kPad * kPad;
  if (total > 0 && tid < padded - total) {
    s_idx[total + tid] = s_idx[total - 1];
#pragma unroll
    for (int b = 0; b < NB; ++b) s_xh[b][total + tid] = 0;
  }
  __syncthreads();

  // ---- 2. stream the listed weight rows once for all NB activations
  const int c = tid % kLPR, slot = tid / kLPR;
  const int col = n0 + 8 * c;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * 2u;
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : P.a_bytes;  // past N: past the end (reads 0)
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.A), 0, P.a_bytes,
                                                                      0x00020000);
  float acc[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[b][j] = 0.f;
  // The list is walked in pairs of neighbouring entries: pair q = slot + v *
  // kSlots (v < kU / 2) holds rows s_idx[2q], s_idx[2q + 1].  v_perm_b32 gathers
  // a column's two weights into one fp16 pair, the two activations are one
  // 32-bit LDS read, and v_dot2_f32_f16 adds both products into the fp32 sum:
  // about half the VALU work of a conversion plus an FMA per weight and row.
  // The next batch of kU rows is loaded before the current one is computed on,
  // so its memory round trip overlaps the dot products (padded is a multiple of
  // kPad, so every slot runs the same number of batches).
  static_assert(kU % 2 == 0, "rows are streamed in pairs");
  {
    const int iters = padded / kPad;
    constexpr int kStep = (kU / 2) * kSlots;
    u32x4b w[kU];
    int q = slot;
    if (iters > 0) {
#pragma unroll
      for (int u = 0; u < kU; ++u)
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(
            rs, static_cast<uint32_t>(s_idx[2 * (q + (u >> 1) * kSlots) + (u & 1)]) * row_bytes + col_bytes, 0, 2);
    }
    for (int it = 0; it < iters; ++it, q += kStep) {
      u32x4b cur[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) cur[u] = w[u];
      if (it + 1 < iters) {
#pragma unroll
        for (int u = 0; u < kU; ++u)
          w[u] = __builtin_amdgcn_raw_buffer_load_b128(
              rs, static_cast<uint32_t>(s_idx[2 * (q + kStep + (u >> 1) * kSlots) + (u & 1)]) * row_bytes + col_bytes,
              0, 2);
      }
#pragma unroll
      for (int v = 0; v < kU / 2; ++v) {
        half2_t wp[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wp[2 * i] = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(cur[2 * v + 1][i], cur[2 * v][i], 0x05040100u));
          wp[2 * i + 1] =
              __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(cur[2 * v + 1][i], cur[2 * v][i], 0x07060302u));
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const half2_t xp = *reinterpret_cast<const half2_t*>(&s_xh[b][2 * (q + v * kSlots)]);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[b][j] = __builtin_amdgcn_fdot2(wp[j], xp, acc[b][j], false);
        }
      }
    }
  }

  // ---- 3. per batch row: slots reduced through LDS, then partials or fp16 out
  for (int b = 0; b < NB; ++b) {
    float4* dst = reinterpret_cast<float4*>(s_red + slot * kBN + 8 * c);
    dst[0] = make_float4(acc[b][0], acc[b][1], acc[b][2], acc[b][3]);
    dst[1] = make_float4(acc[b][4], acc[b][5], acc[b][6], acc[b][7]);
    __syncthreads();
    if (tid < kBN && b < nb) {
      float sum = 0.f;
#pragma unroll
      for (int sl = 0; sl < kSlots; ++sl) sum += s_red[sl * kBN + tid];
      if (P.nchunk == 1) {
        if (n0 + tid < N) P.y[static_cast<size_t>(b0 + b) * N + n0 + tid] = f2h(sum);
      } else {
        P.part[((static_cast<size_t>(b0 + b) * P.nslab + slab) * P.nchunk + chunk) * kBN + tid] = sum;
      }
    }
    __syncthreads();
  }
}

// y[b][n] = fp16 of the chunk partials summed in chunk order.
__global__ __launch_bounds__(kNT) void batched_reduce_kernel(const float* __restrict__ part, int N, int nslab,
                                                             int nchunk, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * kNT + threadIdx.x, b = blockIdx.y;
  if (n >= N) return;
  y[static_cast<size_t>(b) * N + n] = f2h(column_sum(part + static_cast<size_t>(b) * nslab * nchunk * kBN, n, nchunk));
}

template <int NB>
bool launch_nb(const BatchedArgs& P, int bz, dim3 grid, hipStream_t st) {
  switch (bz) {
    case 256: hipLaunchKernelGGL((sparse_gemm_batched_kernel<NB, 256>), grid, dim3(kNT), 0, st, P); return true;
    case 512: hipLaunchKernelGGL((sparse_gemm_batched_kernel<NB, 512>), grid, dim3(kNT), 0, st, P); return true;
    case 1024: hipLaunchKernelGGL((sparse_gemm_batched_kernel<NB, 1024>), grid, dim3(kNT), 0, st, P); return true;
    default: return false;
  }
}

// Batch rows per block: the next power of two up to 8.
int group_rows(int64_t B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8; }

// Chunk size: the largest giving ~1.5 blocks (of 256 threads) per CU, with the
// batch groups counted as extra blocks.
int batched_bz(int64_t B, int64_t N, int64_t Z) {
  const int64_t groups = (B + group_rows(B) - 1) / group_rows(B);
  return gemv_pick_bz(gemv_slabs(N) * groups, Z, 6);
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_sparse_gemm_batched_workspace_bytes(int64_t B, int64_t N, int64_t Z) {
  if (B <= 0 || N <= 0 || Z <= 0) return 256;
  const int64_t nchunk = gemv_chunks(Z, batched_bz(B, N, Z));
  return static_cast<size_t>(B) * gemv_part_floats(N, nchunk) * sizeof(float) + 256;
}

extern "C" int lkv_sparse_gemm_batched(const void* x, const void* w, float threshold, int64_t B, int64_t N,
                                       int64_t Z, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  LKV_REQUIRE(B >= 0 && N >= 0 && Z >= 0, "sparse_gemm_batched: negative size B=%lld N=%lld Z=%lld", (long long)B,
              (long long)N, (long long)Z);
  LKV_REQUIRE(N % 8 == 0, "sparse_gemm_batched: N=%lld must be a multiple of 8 (16-byte weight rows)", (long long)N);
  LKV_REQUIRE(N * Z * 2 < (1ll << 32), "sparse_gemm_batched: weight of %lld bytes exceeds the 4 GiB descriptor range",
              (long long)(N * Z * 2));
  LKV_REQUIRE(B < 65536, "sparse_gemm_batched: B=%lld too large", (long long)B);
  if (B == 0 || N == 0) return LKV_OK;
  LKV_REQUIRE(x && w && y, "sparse_gemm_batched: null pointer");
  LKV_REQUIRE(aligned16(w) && aligned16(y), "sparse_gemm_batched: weight and output must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (Z == 0) {  // empty sums: the reduce kernel over zero chunks writes 0 (a kernel, so graph capture stays safe)
    hipLaunchKernelGGL(batched_reduce_kernel, dim3(static_cast<unsigned>((N + kNT - 1) / kNT), static_cast<unsigned>(B)),
                       dim3(kNT), 0, st, static_cast<const float*>(y), static_cast<int>(N), 1, 0,  // never read
                       static_cast<uint16_t*>(y));
    LKV_LAUNCH_CHECK("sparse_gemm_batched zero");
    return LKV_OK;
  }
  const int bz = batched_bz(B, N, Z);
  const int64_t nslab = gemv_slabs(N), nchunk = gemv_chunks(Z, bz);
  const size_t need = lkv_sparse_gemm_batched_workspace_bytes(B, N, Z);
  LKV_REQUIRE(nchunk == 1 || (workspace && workspace_bytes >= need && aligned16(workspace)),
              "sparse_gemm_batched: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
              workspace_bytes);
  const int nbr = group_rows(B);
  BatchedArgs P;
  P.x = static_cast<const uint16_t*>(x);
  P.A = static_cast<const uint16_t*>(w);
  P.a_bytes = static_cast<uint32_t>(N * Z * 2);
  P.t = threshold;
  P.B = static_cast<int>(B);
  P.N = static_cast<int>(N);
  P.Z = static_cast<int>(Z);
  P.nchunk = static_cast<int>(nchunk);
  P.nslab = static_cast<int>(nslab);
  P.part = static_cast<float*>(workspace);
  P.y = static_cast<uint16_t*>(y);
  const dim3 grid(static_cast<unsigned>(nslab), static_cast<unsigned>(nchunk),
                  static_cast<unsigned>((B + nbr - 1) / nbr));
  const bool ok = nbr == 1 ? launch_nb<1>(P, bz, grid, st)
                : nbr == 2 ? launch_nb<2>(P, bz, grid, st)
                : nbr == 4 ? launch_nb<4>(P, bz, grid, st)
                           : launch_nb<8>(P, bz, grid, st);
  LKV_REQUIRE(ok, "sparse_gemm_batched: no kernel for chunk %d", bz);
  LKV_LAUNCH_CHECK("sparse_gemm_batched");
  if (nchunk > 1) {
    hipLaunchKernelGGL(batched_reduce_kernel, dim3(static_cast<unsigned>((N + kNT - 1) / kNT), static_cast<unsigned>(B)),
                       dim3(kNT), 0, st, P.part, static_cast<int>(N), static_cast<int>(nslab),
                       static_cast<int>(nchunk), P.y);
    LKV_LAUNCH_CHECK("sparse_gemm_batched reduce");
  }
  return LKV_OK;
}
