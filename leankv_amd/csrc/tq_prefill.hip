// Causal prefill attention that reads the TurboQuant packed KV cache.
//
// Reference semantics: during a prefill (or any update of S > 1 tokens)
// TurboQuantCache.update returns cat(dequantize(cold).fp16, hot)
// (leankv/turboquant/cache.py:119-125, 169-189) and HF SDPA runs causal GQA
// attention of the S new queries over it (transformers/integrations/
// sdpa_attention.py:79-105): query i, at position kv_len - S + i, sees keys
// 0 .. kv_len - S + i, where keys below kv_len - hot_cap are the dequantized
// cold tokens and the rest the fp16 hot window.  As in the decode kernels no
// dequantized K/V is formed: with K_hat_t = n_t c[idx_t] PiK,
//   q . K_hat_t = n_t (q PiK^T) . c[idx_t],   sum_t p_t V_hat_t = (sum_t p_t n_t c[idx_t]) PiV,
// and hot tokens enter the same rotated domain as k PiK^T / v PiV^T (exact in
// real arithmetic, rounded to fp16 here), so one accumulator serves all keys
// and one un-rotation by PiV finishes each output row.
//
// Launches of lkv_tq_prefill_attn (two, on the caller's stream):
//   1. rotate16_kernel (fp16 MFMA, PiK / PiV split exactly into fp16 hi + lo
//      parts): the hot rings k @ PiK^T and v @ PiV^T (fp16);
//   2. tq_prefill_attn_kernel: grid (query tiles, kv heads, batch), 8 waves.
//      A block owns 256 (query, head) columns: 256 / G consecutive queries x
//      the G heads of one kv head, 32 columns per wave.  Its prologue rotates
//      the block's queries, q_rot = (q @ PiK^T) * scale * log2(e) in fp16 (the
//      score operand), on the same MFMA with PiK split as in 1 (PiK staged in
//      the tile buffers, each wave its own 32 columns).  It walks the keys in
//      tiles of 64; per tile the block decodes the codes once into LDS --
//      keys as [key][dim] fp16 centroid values (waves 0-3), values transposed
//      as [dim][key] (waves 4-7) -- and every wave runs, on
//      v_mfma_f32_16x16x32_f16,
//      * scores transposed, A = 16 keys x 32 dims from LDS, B = its rotated
//        queries (registers), so a lane holds 8 keys of one column;
//      * the online softmax per lane (key norms, causal mask, exp2 domain,
//        max and sum across the 4 lanes of a column by permlane swaps; the
//        offset keeps a headroom above the max, so most tiles skip the
//        rescale of the accumulators);
//      * values transposed, A = 16 dims x 32 keys from LDS, B = p * n_t from
//        the lane's own softmax registers.
//      Each thread loads its share of a tile's codes two tiles ahead into
//      registers and decodes them into one of two LDS buffers: one barrier
//      per tile.  In its epilogue the block un-rotates its normalised rows,
//      out = rows @ PiV on the same MFMA (PiV staged in the free tile buffers,
//      both operands split into hi + lo), and writes them as fp16.
#include "kernels.h"
#include "tq_attn_common.h"
#include "tq_common.h"

namespace lkv {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;   // rotate16_kernel
constexpr int kKT = 64;         // keys per tile
#ifndef LKV_PREFILL_WAVES
#define LKV_PREFILL_WAVES 8
#endif
// Waves of an attention block, 32 (query, head) columns each.  With 8, the
// key codes of a tile are decoded by waves 0-3 and the value codes by waves
// 4-7, so each decoded tile serves twice the columns of a 4-wave block.
constexpr int kPWaves = LKV_PREFILL_WAVES;
static_assert(kPWaves == 4 || kPWaves == 8, "4 or 8 waves per attention block");
constexpr int kPThreads = 64 * kPWaves;
constexpr bool kSplitDecode = kPWaves == 8;
constexpr int kCols = 32 * kPWaves;  // (query, head) columns per block
constexpr int kKRow = kD + 8;   // fp16 row of the decoded key tile (padded)
#ifndef LKV_PREFILL_VTR
#define LKV_PREFILL_VTR 1
#endif
// Value tile layout.  1: [key][column] rows as decoded (columns in the keys'
// dim order), the MFMA's V^T operand gathered by ds_read_b64_tr_b16; 0:
// transposed [dim][key] by v_perm in the decode.
constexpr bool kVTr = LKV_PREFILL_VTR;
constexpr int kVRow = kKT + 4;    // [dim][key] row (padded: conflict-free 8-byte reads)
// [key][column] row: 72 dwords, so the 8-byte chunks of a transposed read (rows 4 g + i, 4 chunks each)
// fall in distinct banks
constexpr int kVRowT = kD + 16;
constexpr int kVBuf = kVTr ? kKT * kVRowT : kD * kVRow;  // fp16 per value buffer
static_assert(kKT == 64, "the decode / compute lane maps assume 64-key tiles");
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, one L2 each

#ifndef LKV_PREFILL_QROT
#define LKV_PREFILL_QROT 1
#endif
// 1: the attention kernel rotates its own queries in its prologue; 0: one
// rotate16_kernel launch writes them first.  Same bits either way.
constexpr bool kQRotIn = LKV_PREFILL_QROT;

struct PrefillParams {
  const uint16_t* q16;     // [B, Hq, S, 128] fp16: q (kQRotIn) or (q @ PiK^T) * scale * log2(e)
  const float* PiK;        // [128, 128] (kQRotIn)
  float scale_log2;        // scale * log2(e) (kQRotIn)
  const float* PiV;        // [128, 128]: the output rows are un-rotated in the epilogue
  uint16_t* out;           // [B, Hq, S, 128] fp16
  const uint8_t* k_codes;  // [B, Hkv, cap, 64]
  const float* k_norms;    // [B, Hkv, cap]
  const uint8_t* v_codes;
  const float* v_norms;
  const uint16_t* hk;      // [B, Hkv, hot_cap, 128] fp16: hot keys @ PiK^T (ring slots)
  const uint16_t* hv;      // hot values @ PiV^T
  const float* centroids;  // [2^bits]
  int S, Hq, Hkv, G, cap, hot_cap, kv_len, cold_len, ncent;
};

// y = scale * (x @ Pi^T) (TRANS false) or scale * (x @ Pi) (TRANS true) for M
// rows of 128, on fp16 MFMA: Pi split exactly into hi + lo / 2048 fp16 parts,
// and x too when it is fp32, fp32 accumulate (error ~2^-22 relative, the
// x_lo * Pi_lo term dropped).  Wave w computes output dims 32 w .. 32 w + 31
// with its Pi operands in registers; a block takes 64-row tiles, staged
// through LDS both ways so every row is read once and written with 16-byte
// stores.
// Up to 3 independent row sets (segments) per launch, blockIdx.y picking one:
// the query and the two hot rings are rotated by a single launch.
constexpr int kRotRows = 64;
constexpr int kMaxRotSegs = 3;
struct RotSeg {
  const void* x;
  const float* Pi;
  void* y;
  int64_t M;
  float scale;
};
struct RotSegs {
  RotSeg s[kMaxRotSegs];
};
template <bool IN_F16, bool OUT_F16, bool TRANS>
__global__ __launch_bounds__(kThreads) void rotate16_kernel(RotSegs segs) {
  const RotSeg& sg = segs.s[blockIdx.y];
  const void* __restrict__ x = sg.x;
  const float* __restrict__ Pi = sg.Pi;
  void* __restrict__ y = sg.y;
  const int64_t M = sg.M;
  const float scale = sg.scale;
  if (static_cast<int64_t>(blockIdx.x) * kRotRows >= M) return;  // uniform: this segment has fewer tiles
  constexpr int kInB = IN_F16 ? 2 : 4, kOutB = OUT_F16 ? 2 : 4;
  constexpr int kInRow = kD * kInB + 16, kOutRow = kD * kOutB + 16;  // padded LDS rows (bytes)
  __shared__ __align__(16) uint8_t s_in[kRotRows * kInRow];
  __shared__ __align__(16) uint8_t s_out[kRotRows * kOutRow];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  // B operands: column d = 32 wave + 16 dt + c16, k = input dim e = 32 kb + 8 g + i
  u32x4 bh[2][4], bl[2][4];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int d = 32 * wave + 16 * dt + c16, e0 = 32 * kb + 8 * g;
      float p[8];
      if constexpr (!TRANS) {  // B[e][d] = Pi[d][e]
        const float4 u0 = *reinterpret_cast<const float4*>(Pi + d * kD + e0);
        const float4 u1 = *reinterpret_cast<const float4*>(Pi + d * kD + e0 + 4);
        p[0] = u0.x; p[1] = u0.y; p[2] = u0.z; p[3] = u0.w;
        p[4] = u1.x; p[5] = u1.y; p[6] = u1.z; p[7] = u1.w;
      } else {  // B[e][d] = Pi[e][d]
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = Pi[(e0 + i) * kD + d];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t h0 = f2h(p[2 * j]), h1 = f2h(p[2 * j + 1]);
        bh[dt][kb][j] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
        bl[dt][kb][j] = pack2h((p[2 * j] - h2f(h0)) * 2048.f, (p[2 * j + 1] - h2f(h1)) * 2048.f);
      }
    }
  constexpr int kInChunks = kRotRows * kD * kInB / 16 / kThreads;    // 16-byte loads per thread
  constexpr int kOutChunks = kRotRows * kD * kOutB / 16 / kThreads;  // 16-byte stores per thread
  constexpr int kInPerRow = kD * kInB / 16, kOutPerRow = kD * kOutB / 16;
  const int64_t ntiles = (M + kRotRows - 1) / kRotRows;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kRotRows;
    // ---- rows in (rows past M read row M - 1, never stored)
#pragma unroll
    for (int c = 0; c < kInChunks; ++c) {
      const int f = c * kThreads + tid, r = f / kInPerRow, q = f % kInPerRow;
      const int64_t gr = min(row0 + r, M - 1);
      const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(x) + gr * (kD * kInB) + 16 * q);
      *reinterpret_cast<uint4*>(s_in + r * kInRow + 16 * q) = u;
    }
    __syncthreads();
#pragma unroll
    for (int rg = 0; rg < kRotRows / 16; ++rg) {
      u32x4 ah[4], al[4];
      const uint8_t* arow = s_in + (16 * rg + c16) * kInRow;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        if constexpr (IN_F16) {
          const uint4 u = *reinterpret_cast<const uint4*>(arow + 2 * (32 * kb + 8 * g));
          ah[kb] = u32x4{u.x, u.y, u.z, u.w};
        } else {
          const float4 u0 = *reinterpret_cast<const float4*>(arow + 4 * (32 * kb + 8 * g));
          const float4 u1 = *reinterpret_cast<const float4*>(arow + 4 * (32 * kb + 8 * g) + 16);
          const float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint16_t h0 = f2h(v[2 * j]), h1 = f2h(v[2 * j + 1]);
            ah[kb][j] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
            al[kb][j] = pack2h((v[2 * j] - h2f(h0)) * 2048.f, (v[2 * j + 1] - h2f(h1)) * 2048.f);
          }
        }
      }
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f}, accl = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          acc = mfma16x16x32(ah[kb], bh[dt][kb], acc);
          accl = mfma16x16x32(ah[kb], bl[dt][kb], accl);
          if constexpr (!IN_F16) accl = mfma16x16x32(al[kb], bh[dt][kb], accl);
        }
        // D: column d = 32 wave + 16 dt + c16, rows 16 rg + 4 g + i
        const int d = 32 * wave + 16 * dt + c16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = (acc[i] + accl[i] * (1.f / 2048.f)) * scale;
          uint8_t* dst = s_out + (16 * rg + 4 * g + i) * kOutRow + kOutB * d;
          if constexpr (OUT_F16)
            *reinterpret_cast<uint16_t*>(dst) = f2h(v);
          else
            *reinterpret_cast<float*>(dst) = v;
        }
      }
    }
    __syncthreads();
    // ---- rows out
#pragma unroll
    for (int c = 0; c < kOutChunks; ++c) {
      const int f = c * kThreads + tid, r = f / kOutPerRow, q = f % kOutPerRow;
      if (row0 + r < M)
        *reinterpret_cast<uint4*>(static_cast<uint8_t*>(y) + (row0 + r) * (kD * kOutB) + 16 * q) =
            *reinterpret_cast<const uint4*>(s_out + r * kOutRow + 16 * q);
    }
    __syncthreads();  // s_in and s_out are rewritten by the next tile
  }
}

// One launch over n segments (n <= kMaxRotSegs; empty segments are skipped).
template <bool IN_F16, bool OUT_F16, bool TRANS>
int rotate16_segs(const RotSeg* segs, int n, hipStream_t st) {
  RotSegs S{};
  int k = 0;
  int64_t tiles = 0;
  for (int i = 0; i < n; ++i) {
    if (segs[i].M <= 0) continue;
    S.s[k++] = segs[i];
    tiles = std::max<int64_t>(tiles, (segs[i].M + kRotRows - 1) / kRotRows);
  }
  if (k == 0) return LKV_OK;
  const int64_t cap = 2 * static_cast<int64_t>(device_cu_count());
  const int64_t g = tiles < cap ? tiles : cap;
  hipLaunchKernelGGL((rotate16_kernel<IN_F16, OUT_F16, TRANS>), dim3(static_cast<unsigned>(g), static_cast<unsigned>(k)),
                     dim3(kThreads), 0, st, S);
  LKV_LAUNCH_CHECK("tq_prefill_attn rotation");
  return LKV_OK;
}

template <bool IN_F16, bool OUT_F16, bool TRANS>
int rotate16(const void* x, int64_t M, const float* Pi, float scale, void* y, hipStream_t st) {
  const RotSeg seg{x, Pi, y, M, scale};
  return rotate16_segs<IN_F16, OUT_F16, TRANS>(&seg, 1, st);
}

// fp16 positions 0..7 of a natural-order group reordered to kPermDim.
__device__ __forceinline__ uint4 perm_group(uint4 a) {
  return uint4{__builtin_amdgcn_perm(a.y, a.x, 0x05040100u), __builtin_amdgcn_perm(a.w, a.z, 0x05040100u),
               __builtin_amdgcn_perm(a.y, a.x, 0x07060302u), __builtin_amdgcn_perm(a.w, a.z, 0x07060302u)};
}

// Code rows of stored width CB (4: nibbles, 64 B per token; 2: four codes per
// byte; 1: eight per byte) widened to nibble dwords as they are loaded, so the
// decode after the load is the nibble one (bits 1 and 2 through the v_perm
// table, zero-padded past 2^bits centroids).
__device__ __forceinline__ uint32_t nib2(uint32_t x) {  // 8 two-bit codes -> 8 nibbles
  uint32_t t = x & 0xffffu;
  t = (t | (t << 8)) & 0x00ff00ffu;
  t = (t | (t << 4)) & 0x0f0f0f0fu;
  return (t | (t << 2)) & 0x33333333u;
}
__device__ __forceinline__ uint32_t nib1(uint32_t x) {  // 8 one-bit codes -> 8 nibbles
  uint32_t t = x & 0xffu;
  t = (t | (t << 12)) & 0x000f000fu;
  t = (t | (t << 6)) & 0x03030303u;
  return (t | (t << 3)) & 0x11111111u;
}
// dims 32k .. 32k + 31 of a row whose code bytes start at p (row byte 4 CB k)
template <int CB>
__device__ __forceinline__ uint4 codes32(const uint8_t* p) {
  if constexpr (CB == 4) {
    return *reinterpret_cast<const uint4*>(p);
  } else if constexpr (CB == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    return uint4{nib2(v.x), nib2(v.x >> 16), nib2(v.y), nib2(v.y >> 16)};
  } else {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    return uint4{nib1(v), nib1(v >> 8), nib1(v >> 16), nib1(v >> 24)};
  }
}
// dims 8k .. 8k + 7 (row byte CB k)
template <int CB>
__device__ __forceinline__ uint32_t codes8(const uint8_t* p) {
  if constexpr (CB == 4)
    return *reinterpret_cast<const uint32_t*>(p);
  else if constexpr (CB == 2)
    return nib2(*reinterpret_cast<const uint16_t*>(p));
  else
    return nib1(*p);
}

template <bool PERM, int CB>
__global__ __launch_bounds__(kPThreads, 8 / kPWaves) void tq_prefill_attn_kernel(PrefillParams P) {
  static_assert(CB == 4 || PERM, "narrow code rows use the v_perm decode");
  constexpr int RB = kD * CB / 8;  // code bytes per token
  __shared__ __align__(16) uint16_t sK[2 * kKT * kKRow];  // two buffers of decoded keys
  __shared__ __align__(16) uint16_t sVt[2 * kVBuf];  // two buffers of decoded values
  __shared__ __align__(16) float sN[2][2][kKT];           // [buffer][key, value] norms (1 hot, 0 past the end)
  __shared__ uint32_t s_lut[256];
  __shared__ uint16_t s_cent[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h16 = lane & 15, g = lane >> 4;
  const int G = P.G, QT = kCols / G;
  // The latest queries see the most keys: their tiles are dispatched first.
  // Workgroups go to the 8 XCDs round-robin by linear id and every query tile
  // of a (batch, kv head) reads the same cold store, so the tiles are placed
  // XCD by XCD: with I = B * Hkv items, XCD x serves items x, x + 8, .. (I a
  // multiple of 8) or every (8 / I)-th tile of item x % I (I = 1, 2, 4), its
  // own tiles heaviest first; other shapes keep the plain order.
  int qtile, kvh, b;
  {
    const int nx = static_cast<int>(gridDim.x), I = static_cast<int>(gridDim.y * gridDim.z);
    const int p = static_cast<int>(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
    const int x = p % kXcds, s = p / kXcds;
    int item, t;
    if (I % kXcds == 0) {
      const int per = I / kXcds;  // items per XCD
      item = x + kXcds * (s % per);
      t = s / per;
    } else if (kXcds % I == 0 && nx % (kXcds / I) == 0) {
      const int k = kXcds / I;  // XCDs per item
      item = x % I;
      t = s * k + x / I;
    } else {
      item = p / nx;
      t = p % nx;
    }
    qtile = nx - 1 - t;
    kvh = item % static_cast<int>(gridDim.y);
    b = item / static_cast<int>(gridDim.y);
  }
  const int q0 = qtile * QT;
  const int qpos0 = P.kv_len - P.S;  // position of query 0
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  const int cold_len = P.cold_len, kv_len = P.kv_len;

  // ---- centroid tables
  uint32_t tab[4] = {0u, 0u, 0u, 0u};
  if constexpr (PERM) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // fewer than 8 centroids (1, 2 bits): zero entries, never selected
      const float cj = P.centroids[min(j, P.ncent - 1)];
      const uint32_t c16 = f2h(j < P.ncent ? cj : 0.f);
      tab[j >> 2] |= (c16 & 0xffu) << (8 * (j & 3));
      tab[2 + (j >> 2)] |= (c16 >> 8) << (8 * (j & 3));
    }
  } else {
    const int cmax = P.ncent - 1;
    if (tid < 256) s_lut[tid] = pack2h(P.centroids[min(tid & 15, cmax)], P.centroids[min(tid >> 4, cmax)]);
  }
  if (tid < 16) s_cent[tid] = f2h(P.centroids[min(tid, P.ncent - 1)]);

  // ---- query operands: column c = 32 wave + 16 ct + lane % 16 is query
  // q0 + c / G, head c % G; B operand dims 32 kb + 8 (lane / 16) + position.
  int lim[2];  // keys [0, lim) visible to the lane's column (0: no such query)
  u32x4 qa[2][4];
  int wmin = 0x7fffffff;
  if constexpr (kQRotIn) {
    // q_rot = (q @ PiK^T) * scale * log2(e) on fp16 MFMA, rotate16_kernel's arithmetic (PiK split into
    // fp16 hi + lo / 2048, the same products in the same k order, so the same bits), transposed: A = 16
    // rows of PiK, B = the wave's 16 query rows of a column tile.  Staged row R = 32 kb + 16 hf + 4 g' + i
    // holds the PiK row of the key tile's column 32 kb + 8 g' + 4 hf + i (its dim in the decode's order),
    // so the output lane (h16, g) of row tile 2 kb + hf holds that column tile's score operand positions
    // 4 hf + i of dims block kb: qa[ct][kb] directly.  PiK hi in sK, lo in sVt (the tile buffers are free
    // until the first decode).
    {
      const int e4 = tid & 31;  // input dims 4 e4 .. +3
#pragma unroll
      for (int j = 0; j < kD / (kPThreads / 32); ++j) {
        const int R = tid / 32 + (kPThreads / 32) * j;
        const int C = (R & ~31) + 8 * ((R >> 2) & 3) + 4 * ((R >> 4) & 1) + (R & 3);
        const int dim = PERM ? (C & ~7) + ((C & 3) << 1) + ((C >> 2) & 1) : C;
        const float4 pv = *reinterpret_cast<const float4*>(P.PiK + dim * kD + 4 * e4);
        const float x[4] = {pv.x, pv.y, pv.z, pv.w};
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hi[i] = f2h(x[i]);
          lo[i] = f2h((x[i] - h2f(hi[i])) * 2048.f);
        }
        *reinterpret_cast<uint2*>(sK + R * kKRow + 4 * e4) =
            uint2{hi[0] | (static_cast<uint32_t>(hi[1]) << 16), hi[2] | (static_cast<uint32_t>(hi[3]) << 16)};
        *reinterpret_cast<uint2*>(sVt + R * kKRow + 4 * e4) =
            uint2{lo[0] | (static_cast<uint32_t>(lo[1]) << 16), lo[2] | (static_cast<uint32_t>(lo[3]) << 16)};
      }
    }
    u32x4 bq[2][4];  // B: the column's q row, dims 32 kb + 8 g .. +7
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int c = 32 * wave + 16 * ct + h16;
      const int qq = q0 + c / G, hh = c % G;
      const uint16_t* src =
          P.q16 + ((static_cast<size_t>(b) * P.Hq + kvh * G + hh) * P.S + min(qq, P.S - 1)) * kD + 8 * g;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint4 u = *reinterpret_cast<const uint4*>(src + 32 * kb);
        bq[ct][kb] = u32x4{u.x, u.y, u.z, u.w};
      }
    }
    __syncthreads();  // PiK staged
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      f32x4 accl[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 ah = *reinterpret_cast<const u32x4*>(sK + (16 * t + h16) * kKRow + 32 * kb + 8 * g);
        const u32x4 al = *reinterpret_cast<const u32x4*>(sVt + (16 * t + h16) * kKRow + 32 * kb + 8 * g);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          acc[ct] = mfma16x16x32(ah, bq[ct][kb], acc[ct]);
          accl[ct] = mfma16x16x32(al, bq[ct][kb], accl[ct]);
        }
      }
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (acc[ct][i] + accl[ct][i] * (1.f / 2048.f)) * P.scale_log2;
        qa[ct][t >> 1][2 * (t & 1)] = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
        qa[ct][t >> 1][2 * (t & 1) + 1] = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
      }
    }
    __syncthreads();  // every wave is past its PiK reads: the tile buffers are free
  }
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int c = 32 * wave + 16 * ct + h16;
    const int qq = q0 + c / G, hh = c % G;
    const bool ok = qq < P.S;
    lim[ct] = ok ? qpos0 + qq + 1 : 0;
    if (ok) wmin = min(wmin, lim[ct]);
    if constexpr (kQRotIn) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qa[ct][kb] = ok ? qa[ct][kb] : u32x4{0u, 0u, 0u, 0u};
    } else {
      const uint16_t* src =
          P.q16 + ((static_cast<size_t>(b) * P.Hq + kvh * G + hh) * P.S + min(qq, P.S - 1)) * kD + 8 * g;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        uint4 u = *reinterpret_cast<const uint4*>(src + 32 * kb);
        if constexpr (PERM) u = perm_group(u);
        const u32x4 v = u32x4{u.x, u.y, u.z, u.w};
        qa[ct][kb] = ok ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wmin = min(wmin, __shfl_xor(wmin, o));
  wmin = __builtin_amdgcn_readfirstlane(wmin);

  // keys [0, kend) are visible to some column of the block
  const int kend = qpos0 + min(q0 + QT, P.S);
  const int ntile = (kend + kKT - 1) / kKT;

  // ---- per-thread code registers of one key tile, loaded two tiles ahead:
  //   kw   key codes of key tid / 4, dims 32 (tid % 4) .. +32 (as nibbles)
  //   vw   value codes of keys 4 kp + e, dims 8 j4 .. +8 (as nibbles)
  //   nrm  threads < 128: key (tid < 64) or value norm of key tid % 64
  // with vt = tid; with the split decode, threads below 256 hold kw only and
  // threads vt + 256 hold vw only.
  const uint8_t* kcod = P.k_codes + bh * static_cast<size_t>(P.cap) * RB;
  const uint8_t* vcod = P.v_codes + bh * static_cast<size_t>(P.cap) * RB;
  const float* norms = ((tid >> 6) & 1 ? P.v_norms : P.k_norms) + bh * static_cast<size_t>(P.cap);
  const int kk = (tid & 255) >> 2, part = tid & 3;  // key decode
  // value decode: with the [key][column] tile, the 16 lanes of a row group take the 16 column chunks of
  // one row (conflict-free 16-byte stores, coalesced code loads); transposed, the 16 key quads of a column
  const int vt = tid & 255, kp = kVTr ? vt >> 4 : vt & 15, j4 = kVTr ? vt & 15 : vt >> 4;
  const bool key_thr = !kSplitDecode || tid < 256, val_thr = !kSplitDecode || tid >= 256;  // wave-uniform
  struct TileRegs {
    uint4 kw;
    uint32_t vw[4];
    float nrm;
  };
  auto load_tile = [&](TileRegs& R, int t0) {
    if (cold_len > 0) {  // rows past cold_len read the last cold row (valid memory), decoded from elsewhere
      if (key_thr) R.kw = codes32<CB>(kcod + static_cast<size_t>(min(t0 + kk, cold_len - 1)) * RB + 4 * CB * part);
      if (val_thr) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          R.vw[e] = codes8<CB>(vcod + static_cast<size_t>(min(t0 + 4 * kp + e, cold_len - 1)) * RB + CB * j4);
      }
    }
    if (tid < 128) {
      const int tk = t0 + (tid & 63);
      const float n = cold_len > 0 ? norms[min(tk, cold_len - 1)] : 0.f;
      R.nrm = tk < cold_len ? n : (tk < kv_len ? 1.f : 0.f);
    }
  };
  // decode a tile's registers into LDS buffer `buf`: keys [key][dim] (kPermDim
  // order within 8-dim groups with PERM), values transposed [dim][key]
  auto decode_tile = [&](const TileRegs& R, int t0, int buf) {
    uint16_t* sKb = sK + buf * (kKT * kKRow);
    uint16_t* sVb = sVt + buf * kVBuf;
    if (key_thr) {
      const int tk = t0 + kk;
      uint4 o[4];
      if (tk < cold_len) {
        const uint32_t w[4] = {R.kw.x, R.kw.y, R.kw.z, R.kw.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t d[4];
          decode_dw<PERM>(w[q], tab, s_lut, d);
          o[q] = uint4{d[0], d[1], d[2], d[3]};
        }
      } else if (tk < kv_len) {
        const uint4* src = reinterpret_cast<const uint4*>(
            P.hk + (bh * P.hot_cap + static_cast<size_t>(tk % P.hot_cap)) * kD + 32 * part);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          o[q] = src[q];
          if constexpr (PERM) o[q] = perm_group(o[q]);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = uint4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(sKb + kk * kKRow + 32 * part + 8 * q) = o[q];
    }
    if (val_thr && kVTr) {
      // keys tb .. tb + 3, columns 8 j4 .. 8 j4 + 7 (dims in the keys' order): one 16-byte chunk each
      const int tb = t0 + 4 * kp;
      uint4 o[4];
      if (tb + 4 <= cold_len) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t d[4];
          decode_dw<PERM>(R.vw[e], tab, s_lut, d);
          o[e] = uint4{d[0], d[1], d[2], d[3]};
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tk = tb + e;
          if (tk < cold_len) {
            uint32_t d[4];
            decode_dw<PERM>(R.vw[e], tab, s_lut, d);
            o[e] = uint4{d[0], d[1], d[2], d[3]};
          } else if (tk < kv_len) {
            o[e] = *reinterpret_cast<const uint4*>(P.hv + (bh * P.hot_cap + static_cast<size_t>(tk % P.hot_cap)) * kD +
                                                  8 * j4);
            if constexpr (PERM) o[e] = perm_group(o[e]);
          } else {
            o[e] = uint4{0u, 0u, 0u, 0u};
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) *reinterpret_cast<uint4*>(sVb + (4 * kp + e) * kVRowT + 8 * j4) = o[e];
    } else if (val_thr) {
      const int tb = t0 + 4 * kp;
      uint32_t pr[2][8];  // fp16 pairs (key tb + 2 hp, key tb + 2 hp + 1) of dim 8 j4 + dd
      if (tb + 4 <= cold_len) {
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
          const uint32_t w0 = R.vw[2 * hp], w1 = R.vw[2 * hp + 1];
          if constexpr (PERM) {
            // decode8 pairs: [0] dims (0, 2), [1] (4, 6), [2] (1, 3), [3] (5, 7)
            uint32_t a[4], c[4];
            decode8(w0, tab, a);
            decode8(w1, tab, c);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int dlo = (q & 1) * 4 + (q >> 1);  // first dim of pair q: 0, 4, 1, 5
              pr[hp][dlo] = __builtin_amdgcn_perm(c[q], a[q], 0x05040100u);
              pr[hp][dlo + 2] = __builtin_amdgcn_perm(c[q], a[q], 0x07060302u);
            }
          } else {
#pragma unroll
            for (int bt = 0; bt < 4; ++bt) {
              const uint32_t x0 = s_lut[(w0 >> (8 * bt)) & 0xffu], x1 = s_lut[(w1 >> (8 * bt)) & 0xffu];
              pr[hp][2 * bt] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
              pr[hp][2 * bt + 1] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
            }
          }
        }
      } else {
#pragma unroll
        for (int hp = 0; hp < 2; ++hp)
#pragma unroll
          for (int dd = 0; dd < 8; ++dd) pr[hp][dd] = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tk = tb + e;
          uint32_t v[8];
          if (tk < cold_len) {
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) v[dd] = s_cent[(R.vw[e] >> (4 * dd)) & 15u];
          } else if (tk < kv_len) {
            const uint4 h = *reinterpret_cast<const uint4*>(
                P.hv + (bh * P.hot_cap + static_cast<size_t>(tk % P.hot_cap)) * kD + 8 * j4);
            const uint32_t w[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) v[dd] = (w[dd >> 1] >> (16 * (dd & 1))) & 0xffffu;
          } else {
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) v[dd] = 0u;
          }
#pragma unroll
          for (int dd = 0; dd < 8; ++dd) pr[e >> 1][dd] |= v[dd] << (16 * (e & 1));
        }
      }
#pragma unroll
      for (int dd = 0; dd < 8; ++dd)
        *reinterpret_cast<uint2*>(sVb + (8 * j4 + dd) * kVRow + 4 * kp) = uint2{pr[0][dd], pr[1][dd]};
    }
    if (tid < 128) sN[buf][tid >> 6][tid & 63] = R.nrm;
  };

  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[ct][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // one key tile from LDS buffer `buf`: the lane's keys are t0 + 16 tt + 4 g + i
  // (tt 0..3, i 0..3); the value MFMA takes them in two halves of 32 keys
  auto compute_tile = [&](int t0, int buf) {
    const uint16_t* sKb = sK + buf * (kKT * kKRow);
    const uint16_t* sVb = sVt + buf * kVBuf;
    f32x4 sc[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) sc[ct][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(sKb + (16 * tt + h16) * kKRow + 32 * kb + 8 * g);
        sc[0][tt] = mfma16x16x32(a, qa[0][kb], sc[0][tt]);
        sc[1][tt] = mfma16x16x32(a, qa[1][kb], sc[1][tt]);
      }
    const bool masked = t0 + kKT > wmin;  // wave-uniform
    u32x4 pb[2][2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float s[16];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const f32x4 kn = *reinterpret_cast<const f32x4*>(&sN[buf][0][16 * tt + 4 * g]);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * tt + i] = sc[ct][tt][i] * kn[i];
      }
      if (masked) {
#pragma unroll
        for (int jj = 0; jj < 16; ++jj)
          s[jj] = t0 + 16 * (jj >> 2) + 4 * g + (jj & 3) < lim[ct] ? s[jj] : -INFINITY;
      }
      float mx = vmax3(s[0], s[1], s[2]);
#pragma unroll
      for (int jj = 3; jj < 16; jj += 2) mx = jj + 1 < 16 ? vmax3(mx, s[jj], s[jj + 1]) : vmax(mx, s[jj]);
      mx = xgroup_max(mx);
      const float mn = mx > m[ct] ? mx + kHeadroom : m[ct];  // -inf stays -inf
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m[ct] - mu);
      m[ct] = mn;
      float ps = 0.f;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        s[jj] = fast_exp2(s[jj] - mu);
        ps += s[jj];
      }
      l[ct] = l[ct] * alpha + ps;
      if (wave_ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[ct][dt] = o[ct][dt] * alpha;
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(&sN[buf][1][32 * hh + 4 * g]);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(&sN[buf][1][32 * hh + 16 + 4 * g]);
        const float* p = s + 8 * hh;
        pb[ct][hh] = u32x4{pack2h(p[0] * v0[0], p[1] * v0[1]), pack2h(p[2] * v0[2], p[3] * v0[3]),
                           pack2h(p[4] * v1[0], p[5] * v1[1]), pack2h(p[6] * v1[2], p[7] * v1[3])};
      }
    }
    // values: O^T tiles [ct][dt] += V^T (columns 16 dt .., the lane's 8 keys of half hh) x P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        u32x4 a;
        if constexpr (kVTr) {
          // ds_read_b64_tr_b16: in each 16-lane group, lane l receives element l % 4 of the 8 bytes that
          // lanes 4 i + l / 4 (i = 0..3) address.  Lane (h16, g) addresses key 32 hh + 4 g + h16 / 4 (+16),
          // columns 16 dt + 4 (h16 % 4) .. +3, so it receives column 16 dt + h16 of keys 32 hh + 4 g + i.
          const uint16_t* src = sVb + (32 * hh + 4 * g + (h16 >> 2)) * kVRowT + 16 * dt + 4 * (h16 & 3);
          typedef short v4s __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) v4s lds_v4s;
          const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(src));
          const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(src + 16 * kVRowT));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          a = u32x4{l2.x, l2.y, h2.x, h2.y};
        } else {
          const uint16_t* row = sVb + (16 * dt + h16) * kVRow;
          const uint2 lo = *reinterpret_cast<const uint2*>(row + 32 * hh + 4 * g);
          const uint2 hi = *reinterpret_cast<const uint2*>(row + 32 * hh + 16 + 4 * g);
          a = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
        o[0][dt] = mfma16x16x32(a, pb[0][hh], o[0][dt]);
        o[1][dt] = mfma16x16x32(a, pb[1][hh], o[1][dt]);
      }
    }
  };

  // Two register sets and two LDS buffers in turn: tile it decodes from the
  // registers loaded two tiles earlier into buffer it % 2, then the loads of
  // tile it + 2 go out, one barrier, and the tile is computed.  Buffer it % 2
  // was last read by the compute of tile it - 2, which every wave finished
  // before the barrier of tile it - 1.
  TileRegs ra, rb;
  ra.kw = uint4{0u, 0u, 0u, 0u};
  ra.vw[0] = ra.vw[1] = ra.vw[2] = ra.vw[3] = 0u;
  ra.nrm = 0.f;
  rb = ra;
  load_tile(ra, 0);
  if (ntile > 1) load_tile(rb, kKT);
  for (int it = 0;;) {
    decode_tile(ra, it * kKT, 0);
    if (it + 2 < ntile) load_tile(ra, (it + 2) * kKT);
    __syncthreads();
    compute_tile(it * kKT, 0);
    if (++it >= ntile) break;
    decode_tile(rb, it * kKT, 1);
    if (it + 2 < ntile) load_tile(rb, (it + 2) * kKT);
    __syncthreads();
    compute_tile(it * kKT, 1);
    if (++it >= ntile) break;
  }

  // ---- normalise, un-rotate (out = o_rot @ PiV) and write fp16 rows.  One MFMA
  // contraction per 16 output dims x 16 columns with the input dims in a
  // permuted k order: in 32-dim block kb, k slot 8 g + j stands for dim
  // 32 kb + 4 g + j (j < 4) or 32 kb + 16 + 4 g + j - 4 -- the dims this lane
  // holds in o[ct][2 kb] and o[ct][2 kb + 1] -- so the B operand (o^T, column =
  // the lane's column) is the lane's own registers, and A = PiV^T in the same k
  // order comes from LDS.  Both are split exactly into fp16 hi + lo / 2048
  // (hi.hi + hi.lo + lo.hi, the x_lo.Pi_lo term dropped: ~2^-22 relative).
  u32x4 obh[2][4], obl[2][4];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const float L = xgroup_sum(l[ct]);
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const f32x4 u = o[ct][2 * kb] * inv, w = o[ct][2 * kb + 1] * inv;
      const float v[8] = {u[0], u[1], u[2], u[3], w[0], w[1], w[2], w[3]};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t h0 = f2h(v[2 * j]), h1 = f2h(v[2 * j + 1]);
        obh[ct][kb][j] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
        obl[ct][kb][j] = pack2h((v[2 * j] - h2f(h0)) * 2048.f, (v[2 * j + 1] - h2f(h1)) * 2048.f);
      }
    }
  }
  __syncthreads();  // every wave is past its last tile: the key / value buffers are free
  // PiV^T into LDS, [e][c] rows of kKRow: hi in sK, lo in sVt (128 x 136 fp16 each).  Column c holds
  // input dim c, or with the [key][column] value tile under PERM the dim its column c of o carries
  // (8 (c / 8) + kPermDim[c % 8], the keys' dim order).
  static_assert(kD * kKRow <= 2 * kKT * kKRow && kD * kKRow <= 2 * kVBuf, "PiV staging fits the tile buffers");
  {
    // thread: output dim e = tid % 128, input dims kSpan (tid / 128) .. +kSpan - 1 four at a time
    // (global loads coalesced over e, one 8-byte LDS store per four dims)
    constexpr int kSpan = kD / (kPThreads / kD);
    const int e = tid % kD, dbase = (tid / kD) * kSpan;
#pragma unroll 4
    for (int d = dbase; d < dbase + kSpan; d += 4) {
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = d + i;
        const int dim = (kVTr && PERM) ? (c & ~7) + ((c & 3) << 1) + ((c >> 2) & 1) : c;
        const float pv = P.PiV[dim * kD + e];
        hi[i] = f2h(pv);
        lo[i] = f2h((pv - h2f(hi[i])) * 2048.f);
      }
      *reinterpret_cast<uint2*>(sK + e * kKRow + d) =
          uint2{hi[0] | (static_cast<uint32_t>(hi[1]) << 16), hi[2] | (static_cast<uint32_t>(hi[3]) << 16)};
      *reinterpret_cast<uint2*>(sVt + e * kKRow + d) =
          uint2{lo[0] | (static_cast<uint32_t>(lo[1]) << 16), lo[2] | (static_cast<uint32_t>(lo[3]) << 16)};
    }
  }
  __syncthreads();
#pragma unroll 2
  for (int et = 0; et < kD / 16; ++et) {
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    f32x4 accl[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const int er = (16 * et + h16) * kKRow;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int d0 = 32 * kb + 4 * g;
      const uint2 h0 = *reinterpret_cast<const uint2*>(sK + er + d0);
      const uint2 h1 = *reinterpret_cast<const uint2*>(sK + er + d0 + 16);
      const uint2 l0 = *reinterpret_cast<const uint2*>(sVt + er + d0);
      const uint2 l1 = *reinterpret_cast<const uint2*>(sVt + er + d0 + 16);
      const u32x4 ah = u32x4{h0.x, h0.y, h1.x, h1.y}, al = u32x4{l0.x, l0.y, l1.x, l1.y};
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        acc[ct] = mfma16x16x32(ah, obh[ct][kb], acc[ct]);
        accl[ct] = mfma16x16x32(ah, obl[ct][kb], accl[ct]);
        accl[ct] = mfma16x16x32(al, obh[ct][kb], accl[ct]);
      }
    }
    // D: output dims 16 et + 4 g + i of column 32 wave + 16 ct + h16
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int c = 32 * wave + 16 * ct + h16;
      const int qq = q0 + c / G, hh = c % G;
      if (qq < P.S) {
        uint16_t* dst = P.out + ((static_cast<size_t>(b) * P.Hq + kvh * G + hh) * P.S + qq) * kD + 16 * et + 4 * g;
        const float r0 = acc[ct][0] + accl[ct][0] * (1.f / 2048.f), r1 = acc[ct][1] + accl[ct][1] * (1.f / 2048.f);
        const float r2 = acc[ct][2] + accl[ct][2] * (1.f / 2048.f), r3 = acc[ct][3] + accl[ct][3] * (1.f / 2048.f);
        *reinterpret_cast<uint2*>(dst) = uint2{static_cast<uint32_t>(f2h(r0)) | (static_cast<uint32_t>(f2h(r1)) << 16),
                                              static_cast<uint32_t>(f2h(r2)) | (static_cast<uint32_t>(f2h(r3)) << 16)};
      }
    }
  }
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_tq_prefill_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                                      int64_t hot_cap) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || hot_cap <= 0) return 0;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const size_t rows = kQRotIn ? 0 : static_cast<size_t>(B * Hq * S) * kD;
  const size_t hot = static_cast<size_t>(B * Hkv * hot_cap) * kD * 2;
  return al(rows * 2) + 2 * al(hot);  // q_rot fp16 (without kQRotIn), hot rings (the output is un-rotated in the kernel)
}

extern "C" int lkv_tq_prefill_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                                   const uint8_t* v_codes, const float* v_norms, const void* k_hot,
                                   const void* v_hot, const float* PiK, const float* PiV, const float* centroids,
                                   int bits, int64_t kv_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                   int64_t cap, int64_t hot_cap, float scale, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  LKV_REQUIRE(bits >= 1 && bits <= 4, "tq_prefill_attn: bits=%d unsupported (1..4 are bit-packed)", bits);
  LKV_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "tq_prefill_attn: need Hq %% Hkv == 0 (Hq=%lld Hkv=%lld)",
              (long long)Hq, (long long)Hkv);
  const int64_t G = Hq / Hkv;
  LKV_REQUIRE(G <= 16 && (16 % G) == 0, "tq_prefill_attn: Hq/Hkv=%lld must be 1, 2, 4, 8 or 16", (long long)G);
  LKV_REQUIRE(hot_cap >= 1 && hot_cap <= (1 << 20), "tq_prefill_attn: hot_cap=%lld out of range", (long long)hot_cap);
  LKV_REQUIRE(S >= 0 && S <= kv_len, "tq_prefill_attn: need 0 <= S <= kv_len (S=%lld kv_len=%lld)", (long long)S,
              (long long)kv_len);
  LKV_REQUIRE(kv_len - hot_cap <= cap, "tq_prefill_attn: kv_len - hot_cap = %lld cold tokens exceed cap=%lld",
              (long long)(kv_len - hot_cap), (long long)cap);
  LKV_REQUIRE(kv_len < (1ll << 30) && cap < (1ll << 30) && B * Hq * S < (1ll << 31),
              "tq_prefill_attn: problem too large");
  if (B == 0 || S == 0) return LKV_OK;
  LKV_REQUIRE(q && k_codes && k_norms && v_codes && v_norms && k_hot && v_hot && PiK && PiV && centroids && out &&
                  workspace,
              "tq_prefill_attn: null pointer");
  LKV_REQUIRE(aligned16(q) && aligned16(k_codes) && aligned16(v_codes) && aligned16(k_hot) && aligned16(v_hot) &&
                  aligned16(PiK) && aligned16(PiV) && aligned16(out) && aligned16(workspace),
              "tq_prefill_attn: q, codes, hot, Pi, out and workspace must be 16-byte aligned");
  const size_t need = lkv_tq_prefill_attn_workspace_bytes(B, Hq, Hkv, S, hot_cap);
  LKV_REQUIRE(workspace_bytes >= need, "tq_prefill_attn: workspace of %zu bytes required, got %zu", need,
              workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const int64_t nrows = B * Hq * S;
  char* ws = static_cast<char*>(workspace);
  uint16_t* q16 = kQRotIn ? const_cast<uint16_t*>(static_cast<const uint16_t*>(q)) : reinterpret_cast<uint16_t*>(ws);
  uint16_t* hk = reinterpret_cast<uint16_t*>(ws + (kQRotIn ? 0 : al(static_cast<size_t>(nrows) * kD * 2)));
  uint16_t* hv = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(hk) +
                                             al(static_cast<size_t>(B * Hkv * hot_cap) * kD * 2));
  const int64_t cold_len = kv_len > hot_cap ? kv_len - hot_cap : 0;

  // q_rot * scale * log2(e) in fp16 (the score operand); the hot rings in the rotated domains
  // (one launch; every hot slot is rotated, only the current tokens' slots are read)
  {
    const int64_t nhot = kv_len > cold_len ? B * Hkv * hot_cap : 0;
    const RotSeg segs[3] = {{q, PiK, q16, kQRotIn ? 0 : nrows, scale * kLog2e}, {k_hot, PiK, hk, nhot, 1.f},
                            {v_hot, PiV, hv, nhot, 1.f}};
    if (int e = rotate16_segs<true, true, false>(segs, 3, st)) return e;
  }
  PrefillParams P;
  P.q16 = q16;
  P.PiK = PiK;
  P.scale_log2 = scale * kLog2e;
  P.PiV = PiV;
  P.out = static_cast<uint16_t*>(out);
  P.k_codes = k_codes;
  P.k_norms = k_norms;
  P.v_codes = v_codes;
  P.v_norms = v_norms;
  P.hk = hk;
  P.hv = hv;
  P.centroids = centroids;
  P.S = static_cast<int>(S);
  P.Hq = static_cast<int>(Hq);
  P.Hkv = static_cast<int>(Hkv);
  P.G = static_cast<int>(G);
  P.cap = static_cast<int>(cap);
  P.hot_cap = static_cast<int>(hot_cap);
  P.kv_len = static_cast<int>(kv_len);
  P.cold_len = static_cast<int>(cold_len);
  P.ncent = 1 << bits;
  const int64_t QT = kCols / G;
  const dim3 grid(static_cast<unsigned>((S + QT - 1) / QT), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
  switch (bits) {
    case 1: hipLaunchKernelGGL((tq_prefill_attn_kernel<true, 1>), grid, dim3(kPThreads), 0, st, P); break;
    case 2: hipLaunchKernelGGL((tq_prefill_attn_kernel<true, 2>), grid, dim3(kPThreads), 0, st, P); break;
    case 3: hipLaunchKernelGGL((tq_prefill_attn_kernel<true, 4>), grid, dim3(kPThreads), 0, st, P); break;
    default: hipLaunchKernelGGL((tq_prefill_attn_kernel<false, 4>), grid, dim3(kPThreads), 0, st, P);
  }
  LKV_LAUNCH_CHECK("tq_prefill_attn");
  return LKV_OK;
}
