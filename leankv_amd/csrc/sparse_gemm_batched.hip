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
// (row chunks of BZ) x (groups of up to 8 batch rows; of 16 on the
// matrix-core kernel below, used from 8 rows on).  The block compacts the
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
//
// The decode step of B > 1 sequences also groups products of one x in one
// launch (q, k, v; gate, up), each product keeping its own chunking, and gives
// the chunk reduce an epilogue: HF's SwiGLU, the fp16 residual add, RoPE with
// the new token's hot-ring write, or (in a one-block-per-row kernel of its
// own) the residual add and the next RMSNorm.
#include <stdlib.h>

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

// A launch covers up to kMaxSeg products of the same x (the q, k and v
// projections of a layer, or gate and up): each segment owns grid slabs
// slab0 .. slab0 + nslab - 1 and computes exactly what a launch of its own
// would (same chunking, same summation order).  kMaxSeg (3) as for the GEMV.
enum { kEpiNone = 0, kEpiSwiglu = 1, kEpiResidual = 2, kEpiRope = 3, kEpiResidualNorm = 4 };

struct BatchedSeg {
  const uint16_t* A;  // [Z][N] fp16 (column-major weight)
  float* part;        // [B][nslab][nchunk][256] fp32 (unless direct)
  uint16_t* y;        // [B][N] fp16
  uint16_t* ring;     // kEpiRope: also into this hot ring, [B * N / 128][hot_cap][128] fp16 (or null)
  uint32_t a_bytes;
  float t;
  int N, nslab, slab0;
  int rope;           // kEpiRope: this product's heads are rotated (q, k; not v)
};

struct BatchedArgs {
  const uint16_t* x;    // [B][Z] fp16
  const uint16_t* res;  // [B][N] fp16 residual (kEpiResidual; may be seg[0].y)
  const uint16_t* cos;  // [128] fp16 RoPE factors of the position (kEpiRope)
  const uint16_t* sin;
  const uint16_t* norm_w;  // [N] fp16 RMSNorm weight, its epsilon and output [B][N] (kEpiResidualNorm)
  float eps;
  uint16_t* ynorm;
  const int32_t* pos;      // kEpiRope with a ring: the position whose slot pos % hot_cap takes the token
  int hot_cap;
  int B, Z, nchunk, nseg, epi;
  int direct;           // one chunk and no epilogue: fp16 written by the GEMM kernel, no reduce
  BatchedSeg seg[kMaxSeg];
};

// The segment owning grid slab gs.  Uniform selects over constant indices: a
// dynamic index into the argument struct would copy it to scratch memory.
__device__ __forceinline__ BatchedSeg seg_of(const BatchedArgs& P, int gs) {
  BatchedSeg S = P.seg[0];
  if (P.nseg > 1 && gs >= P.seg[1].slab0) S = P.seg[1];
  if (P.nseg > 2 && gs >= P.seg[2].slab0) S = P.seg[2];
  return S;
}

template <int NB, int BZ>
__global__ __launch_bounds__(kNT) void sparse_gemm_batched_kernel(BatchedArgs P) {
  static_assert(BZ % kNT == 0, "BZ must be a multiple of the block size");
  __shared__ float s_x[NB][BZ];
  __shared__ int s_idx[BZ + kPad];
  __shared__ __align__(4) uint16_t s_xh[NB][BZ + kPad];  // fp16 activations of the listed rows (0 if dropped)
  __shared__ int s_cnt[kNT / kWave];
  __shared__ __align__(16) float s_red[kSlots * kBN];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const BatchedSeg S = seg_of(P, blockIdx.x);
  const int slab = blockIdx.x - S.slab0, chunk = blockIdx.y;
  const int b0 = blockIdx.z * NB;
  const int nb = min(NB, P.B - b0);
  const int z0 = chunk * BZ, n0 = slab * kBN;
  const int Z = P.Z, N = S.N;

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
      const bool k = fabsf(xv) > S.t;
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
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : S.a_bytes;  // past N: past the end (reads 0)
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(S.A), 0, S.a_bytes,
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
      if (P.direct) {
        if (n0 + tid < N) S.y[static_cast<size_t>(b0 + b) * N + n0 + tid] = f2h(sum);
      } else {
        S.part[((static_cast<size_t>(b0 + b) * S.nslab + slab) * P.nchunk + chunk) * kBN + tid] = sum;
      }
    }
    __syncthreads();
  }
}

// Groups of 9 to 16 batch rows on the matrix cores: the same union compaction
// (activations of the listed rows, fp16, batch-major in LDS), then per block
// of 32 list entries the 256-column weight tile (16 KB) goes through LDS as
// row-pair dwords -- thread (column group c, entry quad q) loads its four
// 16-byte row segments, v_perm_b32 pairs entries (4q, 4q + 1) and (4q + 2,
// 4q + 3) column by column, and the pairs are stored [pair][column] -- so that
// v_mfma_f32_16x16x32_f16 reads its B operand (8 entries of one column) as
// four LDS words and its A operand (8 entries of one batch row) as one 16-byte
// word.  Wave w owns columns 64 w .. 64 w + 63 (four 16-column tiles) for all
// 16 batch rows, so no cross-wave reduction; two blocks of entries are in
// flight per thread while the previous one is multiplied.  fp16 products are
// exact in fp32 and the sums fp32, as in the v_dot2 kernel (summation order
// differs).
constexpr int kMB = 16;               // batch rows per MFMA tile (the MFMA's M)
constexpr int kKB = 32;               // list entries per block of entries (the MFMA's K)
constexpr int kPairs = kKB / 2;       // row pairs per block of entries
constexpr int kBRow = kBN + 4;        // words per pair row of the weight tile in LDS (bank spread)

// MT tiles of 16 batch rows per block (MT = 2 from 17 rows on: one weight pass
// serves 32 rows, each weight tile read from LDS feeding both tiles' MFMAs).
template <int BZ, int MT>
__global__ __launch_bounds__(kNT, 2) void sparse_gemm_mfma_kernel(BatchedArgs P) {
  static_assert(BZ % kNT == 0 && BZ % kKB == 0, "chunk shape");
  constexpr int E = BZ / kNT;
  constexpr int kRows = kMB * MT;
  constexpr int kXRow = BZ + kKB + 8;  // fp16 per batch row of the listed activations (16-byte rows)
  __shared__ int s_idx[BZ + kKB];
  __shared__ __align__(16) uint16_t s_xh[kRows][kXRow];
  __shared__ __align__(16) uint32_t s_w[2][kPairs * kBRow];
  __shared__ int s_cnt[kNT / kWave];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const BatchedSeg S = seg_of(P, blockIdx.x);
  const int slab = blockIdx.x - S.slab0, chunk = blockIdx.y;
  const int b0 = blockIdx.z * kRows;
  const int nb = min(kRows, P.B - b0);
  const int z0 = chunk * BZ, n0 = slab * kBN;
  const int Z = P.Z, N = S.N;

  // ---- 0. the group's activations into registers, every load issued before
  // the first is used (address clamped to element 0, value selected after)
  float xv[kRows][E];
  {
    uint16_t raw[kRows][E];
#pragma unroll
    for (int b = 0; b < kRows; ++b)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int z = z0 + e * kNT + tid;
        raw[b][e] = P.x[(b < nb && z < Z) ? static_cast<size_t>(b0 + b) * Z + z : 0];
      }
#pragma unroll
    for (int b = 0; b < kRows; ++b)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int z = z0 + e * kNT + tid;
        xv[b][e] = (b < nb && z < Z) ? h2f(raw[b][e]) : 0.f;
      }
  }

  // ---- 1. compaction of the rows some batch row keeps (strict |x| > t)
  int total = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int z = z0 + e * kNT + tid;
    bool keep = false;
#pragma unroll
    for (int b = 0; b < kRows; ++b) keep = keep || fabsf(xv[b][e]) > S.t;
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
      for (int b = 0; b < kRows; ++b) s_xh[b][pos] = f2h(fabsf(xv[b][e]) > S.t ? xv[b][e] : 0.f);  // exact
    }
    total += tot;
    __syncthreads();
  }
  // pad to whole blocks of entries with (last row, zero activations)
  const int padded = (total + kKB - 1) / kKB * kKB;
  if (total > 0 && tid < padded - total) {
    s_idx[total + tid] = s_idx[total - 1];
#pragma unroll
    for (int b = 0; b < kRows; ++b) s_xh[b][total + tid] = 0;
  }
  __syncthreads();

  // ---- 2. blocks of 32 entries: weight tile through LDS, MFMA
  const int nkb = padded / kKB;
  const int c = tid % (kBN / 8), q = tid / (kBN / 8);  // column group (8 columns), entry quad
  const int col = n0 + 8 * c;
  const uint32_t row_bytes = static_cast<uint32_t>(N) * 2u;
  const uint32_t col_bytes = col < N ? static_cast<uint32_t>(col) * 2u : S.a_bytes;  // past N: reads 0
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(S.A), 0, S.a_bytes,
                                                                      0x00020000);
  // Blocks past the list load through offsets past the descriptor's end (zeros,
  // no memory traffic): the loads stay unconditional, so no branch makes the
  // wait for the block in flight come early.
  auto load_tile = [&](u32x4b (&w)[4], int kb) {
    const bool ok = kb < nkb;
    const int kc = ok ? kb : 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t off = static_cast<uint32_t>(s_idx[kc * kKB + 4 * q + r]) * row_bytes + col_bytes;
      w[r] = __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? off : S.a_bytes, 0, 2);
    }
  };
  // pairs (4q, 4q + 1) -> pair row 2q, (4q + 2, 4q + 3) -> 2q + 1; columns 8c .. 8c + 7
  auto store_tile = [&](const u32x4b (&w)[4], int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4b o[2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        o[j >> 2][j & 3] = __builtin_amdgcn_perm(w[2 * h + 1][j >> 1], w[2 * h][j >> 1], sel);
      }
      uint32_t* dst = &s_w[buf][(2 * q + h) * kBRow + 8 * c];
      *reinterpret_cast<u32x4b*>(dst) = o[0];
      *reinterpret_cast<u32x4b*>(dst + 4) = o[1];
    }
  };
  f32x4 acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int m = lane & 15, kg = lane >> 4;
  auto multiply = [&](int kb, int buf) {
    u32x4b a[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) a[mt] = *reinterpret_cast<const u32x4b*>(&s_xh[kMB * mt + m][kb * kKB + 8 * kg]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int cc = 64 * wave + 16 * t + m;  // this lane's B column
      u32x4b bw;
#pragma unroll
      for (int i = 0; i < 4; ++i) bw[i] = s_w[buf][(4 * kg + i) * kBRow + cc];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt][t] = mfma16x16x32(__builtin_bit_cast(u32x4, a[mt]), __builtin_bit_cast(u32x4, bw), acc[mt][t]);
    }
  };
  if (nkb > 0) {
    u32x4b r0[4], r1[4];
    load_tile(r0, 0);
    load_tile(r1, 1);
    store_tile(r0, 0);
    __syncthreads();
    for (int kb = 0; kb < nkb; kb += 2) {
      // s_w[0] holds block kb, r1 block kb + 1 (in flight); stores of blocks
      // past the list write zeros nobody reads
      load_tile(r0, kb + 2);
      multiply(kb, 0);
      store_tile(r1, 1);
      __syncthreads();
      if (kb + 1 >= nkb) break;
      load_tile(r1, kb + 3);
      multiply(kb + 1, 1);
      store_tile(r0, 0);
      __syncthreads();
    }
  }

  // ---- 3. lane (m, kg) holds batch rows 16 mt + 4 kg + i of column 64 wave + 16 t + m
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int lc = 64 * wave + 16 * t + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = kMB * mt + 4 * kg + i;
      if (b < nb) {
        if (P.direct) {
          if (n0 + lc < N) S.y[static_cast<size_t>(b0 + b) * N + n0 + lc] = f2h(acc[mt][t][i]);
        } else {
          S.part[((static_cast<size_t>(b0 + b) * S.nslab + slab) * P.nchunk + chunk) * kBN + lc] = acc[mt][t][i];
        }
      }
    }
  }
}

// y[b][n] = fp16 of the chunk partials summed in chunk order, through the
// launch's epilogue: SwiGLU of the two segments' sums (gate, up; the grid
// covers the first segment's columns), the fp16 residual add
// fp16(res + fp16(sum)) (res may be the output: each element is read, then
// written, by one thread), or RoPE at one position on the heads of 128 dims of
// the segments marked rope (q, k; v is stored as it is): rope_pair, the fp16
// arithmetic of HF's apply_rotary_pos_emb, with the partner dim d +- 64 from
// the same block (a block's 256 columns are two whole heads); a segment with a
// ring (k, v) also stores its token in that hot ring.
static_assert(kBN == kNT && kBN % 128 == 0, "a reduce block covers one slab of whole heads");
// Element n of batch row b of a q/k/v product in its hot ring: row (b, head
// n / 128), slot pos % hot_cap, dim n % 128 (lkv_tq_cache_append's ring).
// A negative position stores nothing into the ring.
__device__ __forceinline__ size_t ring_index(const BatchedArgs& P, const BatchedSeg& S, int b, int n) {
  const int slot = *P.pos % P.hot_cap;
  const size_t r = static_cast<size_t>(b) * (S.N / 128) + n / 128;
  return (r * P.hot_cap + slot) * 128 + (n % 128);
}
__global__ __launch_bounds__(kNT) void batched_reduce_kernel(BatchedArgs P) {
  __shared__ float s_sum[kNT];
  const BatchedSeg S = seg_of(P, blockIdx.x);
  const int tid = threadIdx.x;
  const int n = (blockIdx.x - S.slab0) * kBN + tid, b = blockIdx.y;
  const size_t row = static_cast<size_t>(S.nslab) * P.nchunk * kBN;  // partial floats per batch row
  const size_t o = static_cast<size_t>(b) * S.N + n;
  if (P.epi == kEpiRope && S.rope) {
    // every thread reaches the barrier: columns past N (N % 128 == 0, so whole
    // heads) read the slab's partials, which exist, and store nothing
    const float sum = column_sum(S.part + b * row, n, P.nchunk);
    s_sum[tid] = sum;
    __syncthreads();
    const int d = tid & 127;
    const bool lo = d < 64;
    float o0, o1;
    rope_pair(lo ? sum : s_sum[tid - 64], lo ? s_sum[tid + 64] : sum, P.cos, P.sin, d & 63, o0, o1);
    if (n < S.N) {
      const uint16_t h = f2h(lo ? o0 : o1);
      S.y[o] = h;
      if (S.ring && *P.pos >= 0) S.ring[ring_index(P, S, b, n)] = h;
    }
    return;
  }
  if (n >= S.N) return;
  const float sum = column_sum(S.part + b * row, n, P.nchunk);
  if (S.ring) {  // v of a RoPE launch: its ring slot too
    const uint16_t h = f2h(sum);
    S.y[o] = h;
    if (*P.pos >= 0) S.ring[ring_index(P, S, b, n)] = h;
    return;
  }
  if (P.epi == kEpiSwiglu) {
    S.y[o] = swiglu_f16(sum, column_sum(P.seg[1].part + b * row, n, P.nchunk));
  } else if (P.epi == kEpiResidual) {
    S.y[o] = f2h(h2f(P.res[o]) + h2f(f2h(sum)));
  } else {
    S.y[o] = f2h(sum);
  }
}

// kEpiResidualNorm, one block per batch row: x_out = fp16(res + fp16(sum of
// the chunk partials in chunk order)) (batched_reduce_kernel's arithmetic for
// the residual epilogue; x_out may be res), then y = RMSNorm(x_out) * w with
// rms_rstd / rms_apply, the arithmetic of lkv_rmsnorm, from the row staged in
// LDS.  Thread t takes columns 4t .. 4t + 3 (and every 4096th after), all
// chunks of them in flight together: one memory round trip where the reduce
// and the RMSNorm launch took two launches.
constexpr int kNormThreads = 1024;
constexpr int kNormMaxN = 8192;
constexpr int kNormIt = kNormMaxN / (4 * kNormThreads);  // column quads per thread
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(BatchedArgs P) {
  __shared__ __align__(16) uint16_t s_x[kNormMaxN];
  __shared__ float s_wsum[kGemvThreads / kWave];
  const BatchedSeg& S = P.seg[0];
  const int b = blockIdx.x, tid = threadIdx.x, N = S.N, nchunk = P.nchunk;
  const float* part = S.part + static_cast<size_t>(b) * S.nslab * nchunk * kBN;
  const size_t ro = static_cast<size_t>(b) * N;
  // the residual and the norm weight of the thread's columns first (clamped
  // to the row: N % 8 == 0), then the partials
  uint2 r[kNormIt], wn[kNormIt];
#pragma unroll
  for (int it = 0; it < kNormIt; ++it) {
    const int cc = min(4 * tid + it * 4 * kNormThreads, N - 4);
    r[it] = *reinterpret_cast<const uint2*>(P.res + ro + cc);
    wn[it] = *reinterpret_cast<const uint2*>(P.norm_w + cc);
  }
  uint16_t xn[kNormIt][4];
#pragma unroll
  for (int it = 0; it < kNormIt; ++it) {
    const int c = 4 * tid + it * 4 * kNormThreads;
    if (c < N) {
      const float* p = part + static_cast<size_t>(c / kBN) * nchunk * kBN + (c % kBN);
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      constexpr int kB = 16;  // zeros past the last chunk leave the sum as it is (it is never -0)
      for (int k0 = 0; k0 < nchunk; k0 += kB) {
        f32x4 v[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i)  // clamped address, value selected after: the loads stay unconditional
          v[i] = *reinterpret_cast<const f32x4*>(p + static_cast<size_t>(min(k0 + i, nchunk - 1)) * kBN);
#pragma unroll
        for (int i = 0; i < kB; ++i) {
          const bool ok = k0 + i < nchunk;
#pragma unroll
          for (int j = 0; j < 4; ++j) sum[j] += ok ? v[i][j] : 0.f;
        }
      }
      const uint16_t rr[4] = {static_cast<uint16_t>(r[it].x & 0xffffu), static_cast<uint16_t>(r[it].x >> 16),
                              static_cast<uint16_t>(r[it].y & 0xffffu), static_cast<uint16_t>(r[it].y >> 16)};
#pragma unroll
      for (int j = 0; j < 4; ++j) xn[it][j] = f2h(h2f(rr[j]) + h2f(f2h(sum[j])));
      const uint2 o = make_uint2(xn[it][0] | (static_cast<uint32_t>(xn[it][1]) << 16),
                                 xn[it][2] | (static_cast<uint32_t>(xn[it][3]) << 16));
      *reinterpret_cast<uint2*>(S.y + ro + c) = o;
      *reinterpret_cast<uint2*>(s_x + c) = o;
    }
  }
  __syncthreads();
  const float rstd = rms_rstd(s_x, N, P.eps, s_wsum);
#pragma unroll
  for (int it = 0; it < kNormIt; ++it) {
    const int c = 4 * tid + it * 4 * kNormThreads;
    if (c < N) {
      const uint16_t ww[4] = {static_cast<uint16_t>(wn[it].x & 0xffffu), static_cast<uint16_t>(wn[it].x >> 16),
                              static_cast<uint16_t>(wn[it].y & 0xffffu), static_cast<uint16_t>(wn[it].y >> 16)};
      uint16_t yy[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) yy[j] = f2h(rms_apply(xn[it][j], ww[j], rstd));
      *reinterpret_cast<uint2*>(P.ynorm + ro + c) =
          make_uint2(yy[0] | (static_cast<uint32_t>(yy[1]) << 16), yy[2] | (static_cast<uint32_t>(yy[3]) << 16));
    }
  }
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

template <int MT>
bool launch_mfma(const BatchedArgs& P, int bz, dim3 grid, hipStream_t st) {
  switch (bz) {
    case 256: hipLaunchKernelGGL((sparse_gemm_mfma_kernel<256, MT>), grid, dim3(kNT), 0, st, P); return true;
    case 512: hipLaunchKernelGGL((sparse_gemm_mfma_kernel<512, MT>), grid, dim3(kNT), 0, st, P); return true;
    case 1024:
      if constexpr (MT == 1) {  // 32-row groups stop at 512-row chunks (batched_bz)
        hipLaunchKernelGGL((sparse_gemm_mfma_kernel<1024, MT>), grid, dim3(kNT), 0, st, P);
        return true;
      }
      return false;
    default: return false;
  }
}

// Batches of at least this many rows run on the matrix-core kernel in groups
// of 16 (LKV_BATCHED_MFMA=k for sweeps; 0 never).  Measured on one MI355X at
// the Mistral-7B shapes (us, VALU / matrix-core kernel): 2 rows at 40 %
// sparsity 18.1 / 21.2 (down), 6 rows 25.0 / 25.0, 8 rows 25.9 / 25.0, dense
// 16 rows 41.1 / 26.3 (down) and 38.9 / 24.8 (gate / up).
int64_t mfma_min_rows() {
  static const int64_t k = [] {
    const char* env = getenv("LKV_BATCHED_MFMA");
    return static_cast<int64_t>(env ? atoi(env) : 8);
  }();
  return k;
}
bool use_mfma(int64_t B) { return mfma_min_rows() > 0 && B >= mfma_min_rows(); }

// Batch rows per block: the next power of two up to 8 on the VALU kernel, 16
// on the matrix-core kernel, 32 (two MFMA tiles) above 16 rows.
int group_rows(int64_t B) {
  if (use_mfma(B)) return B > kMB ? 2 * kMB : kMB;
  return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;
}

// Chunk size: the largest giving ~1.5 blocks (of 256 threads) per CU, with the
// batch groups counted as extra blocks.
int batched_bz(int64_t B, int64_t N, int64_t Z) {
  const int64_t groups = (B + group_rows(B) - 1) / group_rows(B);
  const int bz = gemv_pick_bz(gemv_slabs(N) * groups, Z, 6);
  // 32-row groups: the 1024-row chunk's LDS would leave one block per CU
  return group_rows(B) > kMB && bz > 512 ? 512 : bz;
}

// What follows the chunk sums (the entry points' epilogue arguments).
struct EpiArgs {
  int kind = kEpiNone;
  const void* res = nullptr;     // residual (kEpiResidual, kEpiResidualNorm)
  const void* cos = nullptr;     // RoPE factors (kEpiRope)
  const void* sin = nullptr;
  const void* norm_w = nullptr;  // RMSNorm weight, epsilon and output (kEpiResidualNorm)
  float eps = 0.f;
  void* ynorm = nullptr;
  void* ring[kMaxSeg] = {nullptr, nullptr, nullptr};  // per product: its hot ring (kEpiRope), or null
  bool rope[kMaxSeg] = {true, true, false};            // kEpiRope: which products are rotated (q, k)
  const int32_t* pos = nullptr;
  int64_t hot_cap = 1;
};

// Partial floats of one product of B rows at its own chunk size.
size_t product_floats(int64_t B, int64_t N, int64_t Z) {
  return static_cast<size_t>(B) * gemv_part_floats(N, gemv_chunks(Z, batched_bz(B, N, Z)));
}

// One GEMM launch (none when Z == 0) and one reduce (none when direct) for n
// products of x whose chunk sizes agree; partials one product after another
// from ws.  Shapes are checked by the caller.
bool launch_products(const void* x, int64_t B, int64_t Z, int n, const void* const* w, const float* t,
                     const int64_t* N, void* const* y, const EpiArgs& E, float* ws, hipStream_t st) {
  const int epi = E.kind;
  const int bz = batched_bz(B, N[0], Z);
  const int64_t nchunk = Z > 0 ? gemv_chunks(Z, bz) : 0;
  BatchedArgs P = {};
  P.x = static_cast<const uint16_t*>(x);
  P.res = static_cast<const uint16_t*>(E.res);
  P.cos = static_cast<const uint16_t*>(E.cos);
  P.sin = static_cast<const uint16_t*>(E.sin);
  P.norm_w = static_cast<const uint16_t*>(E.norm_w);
  P.eps = E.eps;
  P.ynorm = static_cast<uint16_t*>(E.ynorm);
  P.pos = E.pos;
  P.hot_cap = static_cast<int>(E.hot_cap);
  P.B = static_cast<int>(B);
  P.Z = static_cast<int>(Z);
  P.nchunk = static_cast<int>(nchunk);
  P.nseg = n;
  P.epi = epi;
  P.direct = nchunk == 1 && epi == kEpiNone;
  int slabs = 0;
  size_t off = 0;
  for (int s = 0; s < n; ++s) {
    BatchedSeg& S = P.seg[s];
    S.A = static_cast<const uint16_t*>(w[s]);
    S.part = ws + off;
    S.y = s < (epi == kEpiSwiglu ? 1 : n) ? static_cast<uint16_t*>(y[s]) : nullptr;  // SwiGLU: one output
    S.ring = epi == kEpiRope ? static_cast<uint16_t*>(E.ring[s]) : nullptr;
    S.rope = epi == kEpiRope && E.rope[s];
    S.a_bytes = static_cast<uint32_t>(N[s] * Z * 2);
    S.t = t[s];
    S.N = static_cast<int>(N[s]);
    S.nslab = static_cast<int>(gemv_slabs(N[s]));
    S.slab0 = slabs;
    slabs += S.nslab;
    off += static_cast<size_t>(B) * gemv_part_floats(N[s], nchunk);
  }
  if (Z > 0) {
    const int nbr = group_rows(B);
    const dim3 grid(static_cast<unsigned>(slabs), static_cast<unsigned>(nchunk),
                    static_cast<unsigned>((B + nbr - 1) / nbr));
    bool ok;
    if (use_mfma(B)) {
      ok = nbr == kMB ? launch_mfma<1>(P, bz, grid, st) : launch_mfma<2>(P, bz, grid, st);
    } else {
      ok = nbr == 1 ? launch_nb<1>(P, bz, grid, st)
         : nbr == 2 ? launch_nb<2>(P, bz, grid, st)
         : nbr == 4 ? launch_nb<4>(P, bz, grid, st)
                    : launch_nb<8>(P, bz, grid, st);
    }
    if (!ok) return false;
  }
  if (epi == kEpiResidualNorm) {  // Z == 0: empty sums, the residual itself normalised
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(static_cast<unsigned>(B)), dim3(kNormThreads), 0, st, P);
  } else if (!P.direct) {  // Z == 0: the reduce over zero chunks writes the epilogue of empty sums (graph-safe)
    const int rslabs = epi == kEpiSwiglu ? P.seg[0].nslab : slabs;
    hipLaunchKernelGGL(batched_reduce_kernel, dim3(static_cast<unsigned>(rslabs), static_cast<unsigned>(B)), dim3(kNT),
                       0, st, P);
  }
  return true;
}

// The shared checks and launches of lkv_sparse_gemm_batched(_multi): products
// whose chunk sizes differ run as launches of their own (the epilogues pair
// products of one shape, which always agree).
int batched_products(const char* who, const void* x, int64_t B, int n, const void* const* w, const float* t,
                     const int64_t* N, int64_t Z, const EpiArgs& E, void* const* y, void* workspace,
                     size_t workspace_bytes, hipStream_t st) {
  const int epi = E.kind;
  LKV_REQUIRE(n >= 1 && n <= kMaxSeg, "%s: %d products (1 to %d)", who, n, kMaxSeg);
  LKV_REQUIRE(w && t && N && y, "%s: null product array", who);
  LKV_REQUIRE(epi == kEpiNone || (epi == kEpiSwiglu && n == 2) || (epi == kEpiResidual && n == 1) ||
                  (epi == kEpiRope && n >= 2) || (epi == kEpiResidualNorm && n == 1),
              "%s: epilogue %d with %d products (SwiGLU pairs 2, the residual add takes 1, RoPE q, k and v)", who,
              epi, n);
  LKV_REQUIRE(B >= 0 && Z >= 0, "%s: negative size B=%lld Z=%lld", who, (long long)B, (long long)Z);
  LKV_REQUIRE(B < 65536, "%s: B=%lld too large", who, (long long)B);
  for (int s = 0; s < n; ++s) {
    LKV_REQUIRE(N[s] >= 0, "%s: negative size N=%lld", who, (long long)N[s]);
    LKV_REQUIRE(N[s] % 8 == 0, "%s: N=%lld must be a multiple of 8 (16-byte weight rows)", who, (long long)N[s]);
    LKV_REQUIRE(N[s] * Z * 2 < (1ll << 32), "%s: weight of %lld bytes exceeds the 4 GiB descriptor range", who,
                (long long)(N[s] * Z * 2));
  }
  LKV_REQUIRE(epi != kEpiSwiglu || N[0] == N[1], "%s: SwiGLU of products of %lld and %lld columns", who,
              (long long)N[0], (long long)N[1]);
  for (int s = 0; s < n; ++s)
    LKV_REQUIRE(epi != kEpiRope || !(E.rope[s] || E.ring[s]) || N[s] % 128 == 0,
                "%s: RoPE / ring on a product of %lld columns (heads of 128 dims)", who, (long long)N[s]);
  int64_t total = 0;
  for (int s = 0; s < n; ++s) total += N[s];
  if (B == 0 || total == 0) return LKV_OK;
  // x and the weights are not read when Z == 0 (empty sums)
  LKV_REQUIRE(x || Z == 0, "%s: null pointer", who);
  const int nout = epi == kEpiSwiglu ? 1 : n;  // SwiGLU writes one output for its two products
  for (int s = 0; s < n; ++s)
    LKV_REQUIRE(N[s] == 0 || ((Z == 0 || (w[s] && aligned16(w[s]))) && (s >= nout || (y[s] && aligned16(y[s])))),
                "%s: weight and output must be non-null and 16-byte aligned", who);
  LKV_REQUIRE((epi != kEpiResidual && epi != kEpiResidualNorm) || E.res, "%s: null residual", who);
  LKV_REQUIRE(epi != kEpiRope || (E.cos && E.sin), "%s: null RoPE factors", who);
  if (epi == kEpiResidualNorm) {
    LKV_REQUIRE(N[0] <= kNormMaxN, "%s: N=%lld above the fused RMSNorm's %d columns", who, (long long)N[0],
                kNormMaxN);
    LKV_REQUIRE(E.norm_w && E.ynorm, "%s: null RMSNorm weight or output", who);
    LKV_REQUIRE(aligned16(E.res) && aligned16(y[0]) && aligned16(E.norm_w) && aligned16(E.ynorm),
                "%s: residual, RMSNorm weight and outputs must be 16-byte aligned", who);
  }
  // partials are written unless every product is one chunk without epilogue
  size_t floats = 0;
  bool same = true, need_ws = false;
  for (int s = 0; s < n && Z > 0; ++s) {
    if (N[s] == 0) continue;
    const int bz = batched_bz(B, N[s], Z);
    floats += product_floats(B, N[s], Z);
    same = same && bz == batched_bz(B, N[0], Z);
    need_ws = need_ws || gemv_chunks(Z, bz) > 1 || epi != kEpiNone;
  }
  const size_t need = floats * sizeof(float) + 256;
  LKV_REQUIRE(!need_ws || (workspace && workspace_bytes >= need && aligned16(workspace)),
              "%s: workspace of %zu bytes (16-byte aligned) required, got %zu", who, need, workspace_bytes);
  float* ws = static_cast<float*>(workspace);
  if (same && N[0] > 0) {
    LKV_REQUIRE(launch_products(x, B, Z, n, w, t, N, y, E, ws, st), "%s: no kernel for this chunk size", who);
  } else {
    for (int s = 0; s < n; ++s) {
      if (N[s] == 0) continue;
      EpiArgs e = E;  // this product's own epilogue
      e.ring[0] = E.ring[s];
      e.ring[1] = e.ring[2] = nullptr;
      e.rope[0] = E.rope[s];
      e.rope[1] = e.rope[2] = false;
      LKV_REQUIRE(launch_products(x, B, Z, 1, w + s, t + s, N + s, y + s, e, ws, st),
                  "%s: no kernel for this chunk size", who);
      ws += Z > 0 ? product_floats(B, N[s], Z) : 0;
    }
  }
  LKV_LAUNCH_CHECK(who);
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_sparse_gemm_batched_workspace_bytes(int64_t B, int64_t N, int64_t Z) {
  if (B <= 0 || N <= 0 || Z <= 0) return 256;
  return product_floats(B, N, Z) * sizeof(float) + 256;
}

extern "C" int lkv_sparse_gemm_batched(const void* x, const void* w, float threshold, int64_t B, int64_t N,
                                       int64_t Z, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  return batched_products("sparse_gemm_batched", x, B, 1, &w, &threshold, &N, Z, EpiArgs{}, &y, workspace,
                          workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" size_t lkv_sparse_gemm_batched_multi_workspace_bytes(int64_t B, int n, const int64_t* N, int64_t Z) {
  if (B <= 0 || Z <= 0 || n <= 0 || n > kMaxSeg || !N) return 256;
  size_t floats = 0;
  for (int s = 0; s < n; ++s)
    if (N[s] > 0) floats += product_floats(B, N[s], Z);
  return floats * sizeof(float) + 256;
}

extern "C" int lkv_sparse_gemm_batched_multi(const void* x, int64_t B, int n, const void* const* w,
                                             const float* thresholds, const int64_t* N, int64_t Z, int epilogue,
                                             const void* residual, const void* cos_row, const void* sin_row,
                                             void* const* y, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  EpiArgs E;
  E.kind = epilogue;
  E.res = residual;
  E.cos = cos_row;
  E.sin = sin_row;
  LKV_REQUIRE(epilogue >= kEpiNone && epilogue <= kEpiRope, "sparse_gemm_batched_multi: epilogue %d", epilogue);
  return batched_products("sparse_gemm_batched_multi", x, B, n, w, thresholds, N, Z, E, y, workspace,
                          workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int lkv_sparse_gemm_batched_qkv_rope(const void* x, int64_t B, const void* const* w,
                                                const float* thresholds, const int64_t* N, int64_t Z,
                                                const void* cos_row, const void* sin_row, void* const* y, void* k_hot,
                                                void* v_hot, const int32_t* pos, int64_t hot_cap, void* workspace,
                                                size_t workspace_bytes, void* stream) {
  const char* who = "sparse_gemm_batched_qkv_rope";
  LKV_REQUIRE(N, "%s: null product array", who);
  LKV_REQUIRE((k_hot == nullptr) == (v_hot == nullptr), "%s: both rings or neither", who);
  if (k_hot) {
    LKV_REQUIRE(pos && hot_cap >= 1 && hot_cap < (1 << 30), "%s: null position or bad hot_cap %lld", who,
                (long long)hot_cap);
    LKV_REQUIRE(N[1] == N[2], "%s: k and v of %lld and %lld columns", who, (long long)N[1], (long long)N[2]);
    LKV_REQUIRE(aligned16(k_hot) && aligned16(v_hot), "%s: rings must be 16-byte aligned", who);
  }
  EpiArgs E;
  E.kind = kEpiRope;
  E.cos = cos_row;
  E.sin = sin_row;
  E.ring[1] = k_hot;
  E.ring[2] = v_hot;
  E.pos = pos;
  E.hot_cap = hot_cap;
  return batched_products(who, x, B, 3, w, thresholds, N, Z, E, y, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream));
}

extern "C" int lkv_sparse_gemm_batched_residual_rmsnorm(const void* x, const void* w, float threshold, int64_t B,
                                                        int64_t N, int64_t Z, const void* residual,
                                                        const void* norm_w, float eps, void* x_out, void* y_out,
                                                        void* workspace, size_t workspace_bytes, void* stream) {
  EpiArgs E;
  E.kind = kEpiResidualNorm;
  E.res = residual;
  E.norm_w = norm_w;
  E.eps = eps;
  E.ynorm = y_out;
  return batched_products("sparse_gemm_batched_residual_rmsnorm", x, B, 1, &w, &threshold, &N, Z, E, &x_out,
                          workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
