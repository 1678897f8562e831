// TEAL magnitude-thresholded sparse GEMV, the fused gate/up SwiGLU variant,
// and the input prologues the decode step fuses into them.
//
// Semantics: leankv/teal/kernels/sparse_gemv.py:61-87 (one program sums
// A[z, n] * x[z] over the rows z of its block whose |x[z]| > threshold) and the
// wrapper at :143-181.  The weight arrives in the column-major layout of
// prepare_weight_for_sparse_gemv (:229-234): row z of A[Z][N] is N contiguous
// fp16 values, so a surviving activation selects one contiguous weight row.
//
// Work decomposition: grid = (column slabs of 256) x (row chunks of BZ),
// 512 threads per block for chunks of 512 rows and more, else 256.
//   0. Input prologue: x as given, or computed from what produced it --
//      RMSNorm of the fp16 residual stream (each block reads the whole 8 KB
//      vector for the sum of squares), or SwiGLU of the gate/up partial sums
//      (each block sums the chunks of its own BZ inputs) -- so a projection
//      input never round-trips through a kernel of its own.
//   1. Compaction: the block tests |x| > t on its BZ activations and builds
//      the list of surviving rows in LDS with a wave ballot and mbcnt lane
//      prefix (plus a 4-entry cross-wave prefix).  The list is padded to a
//      whole number of streaming batches with copies of its last row and a
//      zero activation: padded loads hit the line just fetched and add 0.
//   2. Streaming: 32 lanes cover one 512-byte row segment with 16-byte buffer
//      loads (SGPR descriptor + 32-bit offset; loads past the end read 0,
//      non-temporal cache policy); the 8 row slots of the block walk the list
//      4 rows at a time, so 4 independent 16-byte loads per lane are in
//      flight.  fp16 x fp32 -> fp32.
//   3. The row slots are reduced through LDS into 256 fp32 column sums.
//   4. The block writes its partial sums.  The reduction over chunks happens
//      after the kernel boundary, in chunk order (so results are
//      deterministic, unlike the reference's fp16 atomic_add, :87): in
//      gemv_reduce_kernel for the standalone entry points, or in the
//      prologue of whichever decode-step kernel consumes the projection.
//   Weight matrices that share x (q/k/v of a layer) are one launch: column
//   slabs are numbered across the segments.
#include <stdlib.h>

#include <mutex>

#include "gemv_core.h"
#include "kernels.h"

namespace lkv {
namespace {

// The chunk's inputs for the three input modes, in registers: thread t gets
// x[z0 + E t + j], j < E = BZ / NT (0 past Z), the layout the compaction takes.
// Every load of a mode is issued before the first is used (addresses clamped
// into range, values selected afterwards): a conditional load compiles to a
// branch and a wait per element, one memory round trip each.  issue() runs
// once, with no branch around it: after the mode's first loads (raw, SwiGLU),
// so loads it issues return behind them (memory results retire in issue
// order), or before any (RMSNorm, whose sum of squares reads the whole vector).
template <int NT, int BZ, int MODE, bool HOOK, typename Issue>
__device__ __forceinline__ void input_prologue(const GemvArgs& G, int z0, float (&v)[BZ / NT], float* s_wsum,
                                               Issue&& issue) {
  constexpr int E = BZ / NT;  // inputs per thread
  const int zt = z0 + E * static_cast<int>(threadIdx.x);
  const int Z = G.Z;
  if (MODE == kInRmsNorm) {
    if constexpr (HOOK) issue();
    uint16_t xv[E], wv[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int z = min(zt + j, Z - 1);
      xv[j] = G.x[z];
      wv[j] = G.norm_w[z];
    }
    const float rstd = rms_rstd(G.x, Z, G.eps, s_wsum);
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = zt + j < Z ? rms_apply(xv[j], wv[j], rstd) : 0.f;
  } else if (MODE == kInSwiglu) {
    // h = SwiGLU(sum of gate chunks, sum of up chunks), chunks summed in order.  The thread's E inputs
    // are consecutive in one 256-column slab of the partials (Z a multiple of 256 here), so each chunk
    // is one E-float load per matrix, all of them issued 8 chunks deep.
    static_assert(E == 1 || E == 2 || E == 4, "SwiGLU inputs load as 1, 2 or 4 floats");
    typedef float fvec __attribute__((ext_vector_type(E)));
    const size_t mat = static_cast<size_t>(G.in_nslab) * G.in_nchunk * kGemvBN;
    const int nc = G.in_nchunk;
    const int zb = min(zt, Z - E);
    const float* pg = G.in_part + static_cast<size_t>(zb / kGemvBN) * nc * kGemvBN + (zb % kGemvBN);
    float g[E], u[E];
#pragma unroll
    for (int j = 0; j < E; ++j) g[j] = u[j] = 0.f;
    auto pass = [&](int k0, bool first) {
      fvec vg[8], vu[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const size_t k = static_cast<size_t>(min(k0 + i, nc - 1)) * kGemvBN;
        vg[i] = *reinterpret_cast<const fvec*>(pg + k);
        vu[i] = *reinterpret_cast<const fvec*>(pg + mat + k);
      }
      if (HOOK && first) {
        __builtin_amdgcn_sched_barrier(0);
        issue();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool ok = k0 + i < nc;
#pragma unroll
        for (int j = 0; j < E; ++j) {
          g[j] += ok ? vg[i][j] : 0.f;
          u[j] += ok ? vu[i][j] : 0.f;
        }
      }
    };
    if constexpr (HOOK) {
      pass(0, true);  // the first pass straight-line: issue() follows its loads with no branch between
      for (int k0 = 8; k0 < nc; k0 += 8) pass(k0, false);
    } else {
      for (int k0 = 0; k0 < nc; k0 += 8) pass(k0, false);
    }
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = zt + j < Z ? h2f(swiglu_f16(g[j], u[j])) : 0.f;
  } else {
    uint16_t xv[E];
#pragma unroll
    for (int j = 0; j < E; ++j) xv[j] = G.x[min(zt + j, Z - 1)];
    if constexpr (HOOK) {
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = zt + j < Z ? h2f(xv[j]) : 0.f;
  }
}

// v[seg] from a per-segment kernel-argument array without a dynamically
// indexed (serialised) scalar load: every entry is read, one is selected.
template <typename T>
__device__ __forceinline__ T seg_pick(const T (&v)[kMaxSeg], int seg) {
  T r = v[0];
#pragma unroll
  for (int s = 1; s < kMaxSeg; ++s) r = seg == s ? v[s] : r;
  return r;
}

#ifdef LKV_STAMPS
// Instrumented build only (build.py --stamps): per-block phase times on the
// 100 MHz real-time clock of the last launch of each kernel kind, [kind]
// [block][8 stamps]: 0 block start, 1 input prologue done, 2 column sums done
// (compaction, weight stream, slot reduction), 3 block end; 4 the XCC id and
// 5 the HW_ID register of the wave (CU, shader engine) at block start, 6 the
// global column slab and 7 the row chunk of the item.  Kinds: 0 raw
// input, 1 RMSNorm, 2 SwiGLU, 3 RMSNorm dual (gate|up); + 4 for the dense
// variant.  Thread 0 stores them (first work item of a block only).
constexpr int kGemvStampKinds = 8;
constexpr int kGemvStampBlocks = 16384;
__device__ uint64_t g_gemv_stamps[kGemvStampKinds * kGemvStampBlocks * 8];
#define LKV_GEMV_STAMP(i)                                                                                     \
  do {                                                                                                      \
    if (threadIdx.x == 0 && item == static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x) &&                \
        item < kGemvStampBlocks)                                                                            \
      __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(),                                         \
                                  g_gemv_stamps + (kStampKind * kGemvStampBlocks + item) * 8 + (i));        \
  } while (0)
#else
#define LKV_GEMV_STAMP(i) \
  do {                    \
  } while (0)
#endif

template <int NT, int BZ, bool DUAL, int MODE, int U, int CP, bool DENSE = false>
__global__ __launch_bounds__(NT) void sparse_gemv_kernel(GemvArgs G) {
#ifdef LKV_STAMPS
  constexpr int kStampKind = (DENSE ? 4 : 0) + (DUAL ? 3 : MODE);
#endif
  constexpr int BN = kGemvBN;
  constexpr int NL = DUAL ? 2 : 1;
  __shared__ GemvLds<NT, BZ, DUAL, U> sm;

  const int tid = threadIdx.x;
  // Work items are (slab, chunk) pairs.  The usual grid has one block per
  // item (the loop runs once); a persistent grid walks them with a stride.
  // gemv_launch sets slab0[s] = the total slab count for every s >= nseg
  const int nslab_tot = G.slab0[kMaxSeg];
  const int nitems = nslab_tot * G.nchunk;
  for (int item = blockIdx.y * gridDim.x + blockIdx.x; item < nitems; item += gridDim.x * gridDim.y) {
    int gslab, chunk;
    if (G.chunk_major) {  // consecutive items walk the chunks of one slab
      gslab = item / G.nchunk;
      chunk = item % G.nchunk;
    } else {
      gslab = item % nslab_tot;
      chunk = item / nslab_tot;
    }
    const int z0 = chunk * BZ;
    LKV_GEMV_STAMP(0);
#ifdef LKV_STAMPS
    if (threadIdx.x == 0 && item == static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x) && item < kGemvStampBlocks) {
      uint64_t* r = g_gemv_stamps + (kStampKind * kGemvStampBlocks + item) * 8;
      __builtin_nontemporal_store(static_cast<uint64_t>(__builtin_amdgcn_s_getreg(20 | (3 << 11))), r + 4);
      __builtin_nontemporal_store(static_cast<uint64_t>(__builtin_amdgcn_s_getreg(4 | (31 << 11))), r + 5);
      __builtin_nontemporal_store(static_cast<uint64_t>(gslab), r + 6);
      __builtin_nontemporal_store(static_cast<uint64_t>(chunk), r + 7);
    }
#endif

    int seg = 0;
#pragma unroll
    for (int s = 1; s < kMaxSeg; ++s) seg += gslab >= G.slab0[s] ? 1 : 0;
    const int slab = gslab - seg_pick(G.slab0_seg, seg);
    const int N = seg_pick(G.N, seg);
    const int n0 = slab * BN;

    float xin[BZ / NT];
    float sums[NL];
    if constexpr (DENSE) {
      gemv_u32x4 w0[U * kDensePf];
      input_prologue<NT, BZ, MODE, true>(G, z0, xin, sm.wsum, [&] {
        gemv_dense_first<NT, U, CP>(seg_pick(G.A, seg), seg_pick(G.a_bytes, seg), N, z0, G.Z, n0, w0);
      });
      LKV_GEMV_STAMP(1);
      gemv_core_dense<NT, BZ, DUAL, U, CP>(sm, xin, w0, seg_pick(G.A, seg), G.A_up, seg_pick(G.a_bytes, seg), N, z0,
                                           G.Z, n0, sums);
    } else {
      input_prologue<NT, BZ, MODE, false>(G, z0, xin, sm.wsum, [] {});
      LKV_GEMV_STAMP(1);
      gemv_core<NT, BZ, DUAL, U, CP>(sm, xin, seg_pick(G.A, seg), G.A_up, seg_pick(G.a_bytes, seg), N,
                                     seg_pick(G.t, seg), G.t_up, z0, G.Z, n0, sums);
    }
    LKV_GEMV_STAMP(2);

    // ---- 4. output (threads 0..255, one column each): fp16 directly (single chunk) or partial sums
    if (tid < BN) {
      if (G.y != nullptr) {
        if (n0 + tid < N) G.y[n0 + tid] = DUAL ? swiglu_f16(sums[0], sums[NL - 1]) : f2h(sums[0]);
      } else {
#pragma unroll
        for (int l = 0; l < NL; ++l) {
          float* P = G.part + (l == 0 ? seg_pick(G.part_off, seg) : G.part_up_off) +
                     (static_cast<size_t>(slab) * G.nchunk + chunk) * BN;
          P[tid] = sums[l];
        }
      }
    }
    LKV_GEMV_STAMP(3);
    if (item + static_cast<int>(gridDim.x * gridDim.y) < nitems) __syncthreads();  // uniform: LDS reused next
  }
}

// y[n] = sum over chunks of the partials, in chunk order (standalone entry points).
template <bool DUAL>
__global__ __launch_bounds__(kGemvThreads) void gemv_reduce_kernel(const float* __restrict__ partials, int N, int nslab,
                                                                   int nchunk, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * kGemvThreads + threadIdx.x;
  if (n >= N) return;
  const float g = column_sum(partials, n, nchunk);
  if (DUAL)
    y[n] = swiglu_f16(g, column_sum(partials + static_cast<size_t>(nslab) * nchunk * kGemvBN, n, nchunk));
  else
    y[n] = f2h(g);
}

// Several matrices that share x (lkv_sparse_gemv_multi): column n of the
// concatenated outputs belongs to segment s when n0[s] <= n < n0[s + 1].
struct MultiReduce {
  const float* part[kMaxSeg];
  uint16_t* y[kMaxSeg];
  int n0[kMaxSeg + 1];
  int nseg, nchunk;
};

__global__ __launch_bounds__(kGemvThreads) void gemv_reduce_multi_kernel(MultiReduce R) {
  const int n = blockIdx.x * kGemvThreads + threadIdx.x;
  if (n >= R.n0[R.nseg]) return;
  int s = 0;
#pragma unroll
  for (int i = 1; i < kMaxSeg; ++i)
    if (i < R.nseg && n >= R.n0[i]) s = i;
  const int c = n - R.n0[s];
  R.y[s][c] = f2h(column_sum(R.part[s], c, R.nchunk));
}

}  // namespace

// Row-chunk size for a GEMV with Z inputs over `slabs` column slabs: the
// largest chunk that still gives at least quarter_blocks / 4 blocks per CU
// (fewer partials and per-block costs), overridable with LKV_GEMV_BZ for
// tuning sweeps.  The split-K GEMV launches chunks of 512 rows and more as
// 512-thread blocks, so its default of 3 (0.75 blocks per CU) keeps ~6-7 waves
// per CU, as 1.5 blocks of 256 threads did; measured on one box: config 1
// 13.64 -> 13.23 us (1024-row chunks, 224 blocks), config-5 decode 419 -> 420
// tok/s (q|k|v in 512-row chunks, gate|up and down in 1024-row chunks).
int gemv_pick_bz(int64_t slabs, int64_t Z, int quarter_blocks) {
  if (const char* env = getenv("LKV_GEMV_BZ")) {
    const int bz = atoi(env);
    if (bz == 256 || bz == 512 || bz == 1024) return bz;
  }
  const int64_t target = quarter_blocks * static_cast<int64_t>(device_cu_count()) / 4;
  static const int bzs[] = {1024, 512};
  for (int bz : bzs)
    if (slabs * gemv_chunks(Z, bz) >= target) return bz;
  return 256;
}

namespace {

template <int NT, int BZ, int U, int CP>
bool launch_bz(const GemvArgs& G, bool dual, int mode, dim3 grid, hipStream_t st) {
  const dim3 blk(NT);
  switch (mode * 2 + (dual ? 1 : 0)) {
    case kInRaw * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInRaw, U, CP>), grid, blk, 0, st, G); return true;
    case kInRaw * 2 + 1: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, true, kInRaw, U, CP>), grid, blk, 0, st, G); return true;
    case kInRmsNorm * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInRmsNorm, U, CP>), grid, blk, 0, st, G); return true;
    case kInRmsNorm * 2 + 1: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, true, kInRmsNorm, U, CP>), grid, blk, 0, st, G); return true;
    case kInSwiglu * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInSwiglu, U, CP>), grid, blk, 0, st, G); return true;
    default: return false;
  }
}

// Every threshold 0: the dense variant (default launch shapes only).
template <int NT, int BZ, int U>
bool launch_dense(const GemvArgs& G, bool dual, int mode, dim3 grid, hipStream_t st) {
  const dim3 blk(NT);
  switch (mode * 2 + (dual ? 1 : 0)) {
    case kInRaw * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInRaw, U, 2, true>), grid, blk, 0, st, G); return true;
    case kInRmsNorm * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInRmsNorm, U, 2, true>), grid, blk, 0, st, G); return true;
    case kInRmsNorm * 2 + 1: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, true, kInRmsNorm, U, 2, true>), grid, blk, 0, st, G); return true;
    case kInSwiglu * 2: hipLaunchKernelGGL((sparse_gemv_kernel<NT, BZ, false, kInSwiglu, U, 2, true>), grid, blk, 0, st, G); return true;
    default: return false;
  }
}

// LKV_GEMV_DENSE=0 keeps zero-threshold launches on the compacting kernel (A/B sweeps).
bool gemv_dense_enabled() {
  static const bool d = [] {
    const char* env = getenv("LKV_GEMV_DENSE");
    return !(env && atoi(env) == 0);
  }();
  return d;
}

template <int NT, int BZ, int U>
bool launch_cp(const GemvArgs& G, bool dual, int mode, dim3 grid, hipStream_t st, int cp) {
  return cp == 2 ? launch_bz<NT, BZ, U, 2>(G, dual, mode, grid, st) : launch_bz<NT, BZ, U, 0>(G, dual, mode, grid, st);
}

// Tuning knobs, read once.  Weights are streamed with the nt (non-temporal)
// cache policy: each byte is read once per call, and keeping it out of the
// L2 leaves room for x and the partial sums (measured on MI355X: fused gate/up
// 27.7 -> 24.3 us, config-1 GEMV 15.7 -> 14.2 us); LKV_GEMV_CPOL=0 restores
// the default policy.  LKV_GEMV_ORDER=chunk makes consecutive blocks walk one
// slab's chunks instead of one chunk's slabs (slower: 17.5 vs 15.7 us).
int gemv_cpol() {
  static const int c = [] {
    const char* env = getenv("LKV_GEMV_CPOL");
    return env && atoi(env) == 0 ? 0 : 2;
  }();
  return c;
}
// LKV_GEMV_PERSIST=k: a grid of k blocks per CU walks the (slab, chunk) items.
int gemv_persist() {
  static const int k = [] {
    const char* env = getenv("LKV_GEMV_PERSIST");
    const int v = env ? atoi(env) : 0;
    return v > 0 && v <= 8 ? v : 0;
  }();
  return k;
}
bool gemv_chunk_major() {
  static const bool c = [] {
    const char* env = getenv("LKV_GEMV_ORDER");
    return env && env[0] == 'c';
  }();
  return c;
}

// Threads per GEMV block for chunks of 512 rows and more: 512 (LKV_GEMV_THREADS=256
// for tuning sweeps; 256-row chunks always run 256 threads).
int gemv_threads() {
  static const int t = [] {
    const char* env = getenv("LKV_GEMV_THREADS");
    return env && atoi(env) == 256 ? 256 : 512;
  }();
  return t;
}

// Rows each lane keeps in flight, chosen so a block keeps ~32 KB of weight
// rows in flight: 4 in 512-thread blocks, 8 in 256-thread blocks (256-row
// chunks); LKV_GEMV_UNROLL=4, 8 or 16 overrides for tuning sweeps.  Measured on
// one box, fused gate/up at the Mistral-7B shape: U = 2 / 3 / 4 / 6 / 8 ->
// 30.4 / 24.7 / 23.5 / 23.8 / 24.0 us, config-5 decode 355 / 407 / 419 / 416 /
// 415 tok/s; the 256-row o_proj chunks with 8 rather than 4: decode 419.4 ->
// 420.2 tok/s, dense fp16 step 298.3 -> 301.5 tok/s.
int gemv_unroll(int threads) {
  static const int u = [] {
    const char* env = getenv("LKV_GEMV_UNROLL");
    const int v = env ? atoi(env) : 0;
    return v == 4 || v == 8 || v == 16 ? v : 0;
  }();
  return u ? u : (threads == 512 ? 4 : 8);
}

}  // namespace

int gemv_launch(const GemvArgs& G, int bz, bool dual, int mode, int nslab_total, hipStream_t st) {
  if (nslab_total <= 0) return LKV_OK;
  dim3 grid(static_cast<unsigned>(nslab_total), static_cast<unsigned>(G.nchunk));
  if (const int k = gemv_persist()) {
    const int64_t items = static_cast<int64_t>(nslab_total) * G.nchunk;
    const int64_t blocks = static_cast<int64_t>(k) * device_cu_count();
    if (blocks < items) grid = dim3(static_cast<unsigned>(blocks), 1);
  }
  bool ok = false;
  const bool t512 = gemv_threads() == 512 && bz >= 512;
  const int cp = gemv_cpol();
  GemvArgs Gx = G;
  Gx.chunk_major = gemv_chunk_major() ? 1 : 0;
  // the kernel selects per-segment values without dynamic indexing: segments
  // past nseg start at the total slab count (never selected) and copy seg 0
  for (int s = 0; s < kMaxSeg; ++s) Gx.slab0_seg[s] = G.slab0[s];
  for (int s = G.nseg; s <= kMaxSeg; ++s) Gx.slab0[s] = nslab_total;
  for (int s = G.nseg; s < kMaxSeg; ++s) {
    Gx.A[s] = G.A[0];
    Gx.a_bytes[s] = G.a_bytes[0];
    Gx.N[s] = G.N[0];
    Gx.t[s] = G.t[0];
    Gx.part_off[s] = G.part_off[0];
    Gx.slab0_seg[s] = nslab_total;
  }
  const int unroll = gemv_unroll(t512 ? 512 : 256);
  bool zero_t = !dual || G.t_up == 0.f;
  for (int s = 0; s < G.nseg; ++s) zero_t = zero_t && G.t[s] == 0.f;
  if (zero_t && gemv_dense_enabled() && cp == 2 && unroll == (t512 ? 4 : 8) && !gemv_persist() &&
      !Gx.chunk_major) {
    if (bz == 256) ok = launch_dense<256, 256, 8>(Gx, dual, mode, grid, st);
    else if (bz == 512) ok = t512 ? launch_dense<512, 512, 4>(Gx, dual, mode, grid, st) : launch_dense<256, 512, 8>(Gx, dual, mode, grid, st);
    else if (bz == 1024) ok = t512 ? launch_dense<512, 1024, 4>(Gx, dual, mode, grid, st) : launch_dense<256, 1024, 8>(Gx, dual, mode, grid, st);
  } else if (unroll == 4) {
    if (bz == 256) ok = launch_cp<256, 256, 4>(Gx, dual, mode, grid, st, cp);
    else if (bz == 512) ok = t512 ? launch_cp<512, 512, 4>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 512, 4>(Gx, dual, mode, grid, st, cp);
    else if (bz == 1024) ok = t512 ? launch_cp<512, 1024, 4>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 1024, 4>(Gx, dual, mode, grid, st, cp);
  } else if (unroll == 16) {
    if (bz == 256) ok = launch_cp<256, 256, 16>(Gx, dual, mode, grid, st, cp);
    else if (bz == 512) ok = t512 ? launch_cp<512, 512, 16>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 512, 16>(Gx, dual, mode, grid, st, cp);
    else if (bz == 1024) ok = t512 ? launch_cp<512, 1024, 16>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 1024, 16>(Gx, dual, mode, grid, st, cp);
  } else {
    if (bz == 256) ok = launch_cp<256, 256, 8>(Gx, dual, mode, grid, st, cp);
    else if (bz == 512) ok = t512 ? launch_cp<512, 512, 8>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 512, 8>(Gx, dual, mode, grid, st, cp);
    else if (bz == 1024) ok = t512 ? launch_cp<512, 1024, 8>(Gx, dual, mode, grid, st, cp) : launch_cp<256, 1024, 8>(Gx, dual, mode, grid, st, cp);
  }
  if (!ok) {
    set_error("sparse_gemv: no kernel for chunk %d, mode %d, dual %d", bz, mode, dual ? 1 : 0);
    return LKV_ERR_INVALID;
  }
  LKV_LAUNCH_CHECK("sparse_gemv");
  return LKV_OK;
}

#ifdef LKV_STAMPS
// Instrumented build only: copy the stamps of GEMV kind `kind` (n <= 8 * 16384
// words) to host memory, or zero every kind's with clear = 1.  Not declared
// in the public header.
extern "C" int lkv_debug_gemv_stamps(int kind, uint64_t* host, int64_t n, int clear) {
  LKV_REQUIRE(kind >= 0 && kind < kGemvStampKinds && n >= 0 && n <= 8 * kGemvStampBlocks && (clear || host),
              "debug_gemv_stamps: bad arguments");
  hipError_t e;
  if (clear) {
    static uint64_t zeros[kGemvStampKinds * kGemvStampBlocks * 8];
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_gemv_stamps), zeros, sizeof(zeros));
  } else {
    e = hipMemcpyFromSymbol(host, HIP_SYMBOL(g_gemv_stamps), static_cast<size_t>(n) * 8,
                            static_cast<size_t>(kind) * kGemvStampBlocks * 8 * 8);
  }
  LKV_REQUIRE(e == hipSuccess, "debug_gemv_stamps: %s", hipGetErrorString(e));
  return LKV_OK;
}
#endif

namespace {

size_t ws_bytes_for(int64_t N, int64_t Z, bool dual) {
  const int bz = gemv_pick_bz(gemv_slabs(N), Z);
  return kTicketBytes + (dual ? 2 : 1) * gemv_part_floats(N, gemv_chunks(Z, bz)) * sizeof(float);
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

int standalone(const void* x, const void* A0, const void* A1, float t0, float t1, int64_t N, int64_t Z, void* y,
               void* ws, size_t ws_bytes, hipStream_t st, bool dual) {
  const int64_t nslab = gemv_slabs(N);
  const int bz = gemv_pick_bz(nslab, Z);
  const int64_t nchunk = gemv_chunks(Z, bz);
  const size_t need = ws_bytes_for(N, Z, dual);
  LKV_REQUIRE(ws && ws_bytes >= need && aligned16(ws),
              "sparse_gemv: workspace of %zu bytes (16-byte aligned) required, got %zu", need, ws_bytes);
  GemvArgs G{};
  G.x = static_cast<const uint16_t*>(x);
  G.nseg = 1;
  G.A[0] = static_cast<const uint16_t*>(A0);
  G.A_up = static_cast<const uint16_t*>(A1);
  G.a_bytes[0] = static_cast<uint32_t>(N * Z * 2);
  G.N[0] = static_cast<int>(N);
  G.t[0] = t0;
  G.t_up = t1;
  G.slab0[0] = 0;
  G.slab0[1] = static_cast<int>(nslab);
  G.Z = static_cast<int>(Z);
  G.nchunk = static_cast<int>(nchunk);
  G.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kTicketBytes);
  G.part_off[0] = 0;
  G.part_up_off = gemv_part_floats(N, nchunk);
  G.y = nchunk == 1 ? static_cast<uint16_t*>(y) : nullptr;
  if (int e = gemv_launch(G, bz, dual, kInRaw, static_cast<int>(nslab), st)) return e;
  if (nchunk > 1) {
    const unsigned rgrid = static_cast<unsigned>((N + kGemvThreads - 1) / kGemvThreads);
    if (dual)
      hipLaunchKernelGGL((gemv_reduce_kernel<true>), dim3(rgrid), dim3(kGemvThreads), 0, st, G.part,
                         static_cast<int>(N), static_cast<int>(nslab), static_cast<int>(nchunk),
                         static_cast<uint16_t*>(y));
    else
      hipLaunchKernelGGL((gemv_reduce_kernel<false>), dim3(rgrid), dim3(kGemvThreads), 0, st, G.part,
                         static_cast<int>(N), static_cast<int>(nslab), static_cast<int>(nchunk),
                         static_cast<uint16_t*>(y));
    LKV_LAUNCH_CHECK("sparse_gemv reduce");
  }
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_sparse_gemv_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return kTicketBytes;
  return ws_bytes_for(N, Z, false);
}

extern "C" size_t lkv_sparse_gateup_workspace_bytes(int64_t N, int64_t Z) {
  if (N <= 0) return kTicketBytes;
  return ws_bytes_for(N, Z, true);
}

extern "C" int lkv_sparse_gemv_chunks(int64_t N, int64_t Z) {
  if (N <= 0 || Z <= 0) return 1;
  return static_cast<int>(gemv_chunks(Z, gemv_pick_bz(gemv_slabs(N), Z)));
}

extern "C" int lkv_sparse_gemv_partials(const void* x, const void* w_gate, const void* w_up, float t_gate, float t_up,
                                        int64_t N, int64_t Z, float* partials, size_t partials_bytes, void* stream) {
  if (int e = check_common(x, w_gate, N, Z, partials)) return e;
  LKV_REQUIRE(w_up == nullptr || aligned16(w_up), "sparse_gemv_partials: up weight must be 16-byte aligned");
  if (N == 0 || Z == 0) return LKV_OK;
  const bool dual = w_up != nullptr;
  const int64_t nslab = gemv_slabs(N);
  const int bz = gemv_pick_bz(nslab, Z);
  const int64_t nchunk = gemv_chunks(Z, bz);
  const size_t need = (dual ? 2 : 1) * gemv_part_floats(N, nchunk) * sizeof(float);
  LKV_REQUIRE(partials_bytes >= need, "sparse_gemv_partials: %zu bytes of partials required, got %zu", need,
              partials_bytes);
  GemvArgs G{};
  G.x = static_cast<const uint16_t*>(x);
  G.nseg = 1;
  G.A[0] = static_cast<const uint16_t*>(w_gate);
  G.A_up = static_cast<const uint16_t*>(w_up);
  G.a_bytes[0] = static_cast<uint32_t>(N * Z * 2);
  G.N[0] = static_cast<int>(N);
  G.t[0] = t_gate;
  G.t_up = t_up;
  G.slab0[1] = static_cast<int>(nslab);
  G.Z = static_cast<int>(Z);
  G.nchunk = static_cast<int>(nchunk);
  G.part = partials;
  G.part_up_off = gemv_part_floats(N, nchunk);
  return gemv_launch(G, bz, dual, kInRaw, static_cast<int>(nslab), static_cast<hipStream_t>(stream));
}

namespace {

int multi_check(int n, const int64_t* N, int64_t Z) {
  LKV_REQUIRE(n >= 1 && n <= kMaxSeg && N != nullptr, "sparse_gemv_multi: 1..%d matrices, got %d", kMaxSeg, n);
  LKV_REQUIRE(Z > 0 && Z < (1 << 30), "sparse_gemv_multi: Z=%lld out of range", (long long)Z);
  for (int s = 0; s < n; ++s) {
    LKV_REQUIRE(N[s] > 0 && N[s] % 8 == 0 && N[s] < (1 << 30),
                "sparse_gemv_multi: N[%d]=%lld must be a positive multiple of 8", s, (long long)N[s]);
    LKV_REQUIRE(N[s] * Z * 2 < (1ll << 32), "sparse_gemv_multi: matrix %d exceeds the 4 GiB descriptor range", s);
  }
  return LKV_OK;
}

struct MultiPlan {
  int bz, nchunk, nslab;
  size_t part_off[kMaxSeg];
  size_t bytes;
};

// The fused decode step's q|k|v plan (decode.hip): one chunk size for the
// slabs of all segments together, partials of segment s after those of s - 1.
MultiPlan multi_plan(int n, const int64_t* N, int64_t Z) {
  MultiPlan p{};
  for (int s = 0; s < n; ++s) p.nslab += static_cast<int>(gemv_slabs(N[s]));
  p.bz = gemv_pick_bz(p.nslab, Z);
  p.nchunk = static_cast<int>(gemv_chunks(Z, p.bz));
  size_t off = 0;
  for (int s = 0; s < n; ++s) {
    p.part_off[s] = off;
    off += gemv_part_floats(N[s], p.nchunk);
  }
  p.bytes = off * sizeof(float);
  return p;
}

}  // namespace

extern "C" size_t lkv_sparse_gemv_multi_workspace_bytes(int n, const int64_t* N, int64_t Z) {
  if (multi_check(n, N, Z) != LKV_OK) return 0;
  return multi_plan(n, N, Z).bytes;
}

extern "C" int lkv_sparse_gemv_multi(const void* x, int n, const void* const* w, const float* thresholds,
                                     const int64_t* N, int64_t Z, void* const* y, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (int e = multi_check(n, N, Z)) return e;
  LKV_REQUIRE(x && w && thresholds && y, "sparse_gemv_multi: null pointer");
  for (int s = 0; s < n; ++s)
    LKV_REQUIRE(w[s] && y[s] && aligned16(w[s]) && aligned16(y[s]),
                "sparse_gemv_multi: matrix and output %d must be non-null and 16-byte aligned", s);
  const MultiPlan p = multi_plan(n, N, Z);
  LKV_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= p.bytes,
              "sparse_gemv_multi: workspace of %zu bytes (16-byte aligned) required, got %zu", p.bytes,
              workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemvArgs G{};
  G.x = static_cast<const uint16_t*>(x);
  G.nseg = n;
  MultiReduce R{};
  R.nseg = n;
  R.nchunk = p.nchunk;
  int slab = 0, col = 0;
  for (int s = 0; s < n; ++s) {
    G.A[s] = static_cast<const uint16_t*>(w[s]);
    G.a_bytes[s] = static_cast<uint32_t>(N[s] * Z * 2);
    G.N[s] = static_cast<int>(N[s]);
    G.t[s] = thresholds[s];
    G.slab0[s] = slab;
    G.part_off[s] = p.part_off[s];
    slab += static_cast<int>(gemv_slabs(N[s]));
    R.part[s] = static_cast<float*>(workspace) + p.part_off[s];
    R.y[s] = static_cast<uint16_t*>(y[s]);
    R.n0[s] = col;
    col += static_cast<int>(N[s]);
  }
  G.slab0[n] = slab;
  R.n0[n] = col;
  G.Z = static_cast<int>(Z);
  G.nchunk = p.nchunk;
  G.part = static_cast<float*>(workspace);
  if (int e = gemv_launch(G, p.bz, false, kInRaw, slab, st)) return e;
  hipLaunchKernelGGL(gemv_reduce_multi_kernel, dim3(static_cast<unsigned>((col + kGemvThreads - 1) / kGemvThreads)),
                     dim3(kGemvThreads), 0, st, R);
  LKV_LAUNCH_CHECK("sparse_gemv_multi reduce");
  return LKV_OK;
}

extern "C" int lkv_sparse_gemv(const void* x, const void* w, float threshold, int64_t N, int64_t Z, void* y,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_common(x, w, N, Z, y)) return e;
  if (N == 0) return LKV_OK;
  return standalone(x, w, w, threshold, threshold, N, Z, y, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream), false);
}

// ---------------------------------------------------------------- no-alloc variant
// lkv_sparse_gemv with its split-K partials in a library-owned device array
// instead of a caller workspace.  Each GPU holds its own copy of `scratch`;
// the host-side name is only a stand-in for that memory, so the device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only the looked-up pointer is handed to kernels.  Every call
// on a device shares its array: calls that overlap on one GPU race.
namespace lkv {
namespace {

constexpr size_t kScratchBytes = size_t(8) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (nullptr + error text on failure).
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("sparse_gemv_noalloc: no current HIP device (hipGetDevice -> %d)", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("sparse_gemv_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace lkv

extern "C" size_t lkv_sparse_gemv_noalloc_max_bytes(void) { return lkv::kScratchBytes; }

extern "C" int lkv_sparse_gemv_noalloc(const void* x, const void* w, float threshold, int64_t N, int64_t Z, void* y,
                                       void* stream) {
  if (int e = check_common(x, w, N, Z, y)) return e;
  if (N == 0) return LKV_OK;
  const size_t need = ws_bytes_for(N, Z, false);
  LKV_REQUIRE(need <= kScratchBytes,
              "sparse_gemv_noalloc: N=%lld Z=%lld needs %zu bytes of split-K partials, above the %zu-byte "
              "scratch array (use lkv_sparse_gemv with a workspace)",
              (long long)N, (long long)Z, need, kScratchBytes);
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return LKV_ERR_HIP;
  return standalone(x, w, w, threshold, threshold, N, Z, y, ws, kScratchBytes, static_cast<hipStream_t>(stream),
                    false);
}

extern "C" int lkv_sparse_gateup_swiglu(const void* x, const void* wg, const void* wu, float t_gate, float t_up,
                                        int64_t N, int64_t Z, void* h, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  if (int e = check_common(x, wg, N, Z, h)) return e;
  LKV_REQUIRE(wu && (aligned16(wu) || N == 0), "sparse_gateup: up weight must be 16-byte aligned");
  if (N == 0) return LKV_OK;
  return standalone(x, wg, wu, t_gate, t_up, N, Z, h, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                    true);
}
