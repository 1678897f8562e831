// Batch decode attention over a paged fp16 KV cache (one layer): the
// attention of the dense fp16 baseline decode step (lkv_decode_layer_step_f16kv).
//
// Reference: leankv/turboquant/paged_cache.py:194-257 (PagedKVCache.
// decode_attention: FlashInfer BatchDecodeWithPagedKVCacheWrapper.plan + run,
// NHD layout, no positional encoding, default scale 1/sqrt(128)) over the page
// pool kv_data[layer] = [max_pages][2 (K, V)][page_size][Hkv][128] fp16 and
// the CSR page table FlashInfer takes: sequence b owns pages
// indices[indptr[b] .. indptr[b + 1]) and its last page holds last_len[b]
// (1 .. page_size) tokens.  Output: softmax(q K^T * scale) V per query head,
// GQA (query head h reads kv head h / (Hq / Hkv)).
//
// Launches: split kernel, grid (splits, kv heads, batch), 4 waves; each wave
// walks 32-token chunks of its split:
//   * scores on v_mfma_f32_16x16x32_f16, transposed as in the packed decode
//     kernel: A = 16 tokens x 32 dims straight from the pages (one 16-byte
//     load per lane, page looked up per token), B = the query (16 head
//     columns, G used), so a lane holds one head's scores for 8 tokens;
//   * online softmax per lane (exp2 domain, max / sum across the 4 lanes of
//     a head by permlane swaps);
//   * values: at most 4 query heads per kv head (SMALLG) on MFMA as in the
//     packed decode kernel, A = 16 dims x 32 tokens of value rows (16-byte
//     loads, token pairs joined by v_perm), B = the probabilities in fp16
//     (fp32 accumulate); otherwise on the VALU from the wave's LDS slice of
//     probabilities, lane (8-dim group, head) accumulating p * v in fp32;
// the 4 waves merge through LDS into one (m, l, o[G][128]) record per split;
// then a combine kernel, one block per (batch, query head), merges the split
// records.  Page indices are clamped to the pool, lengths to the pages owned,
// so malformed tables cannot address memory outside the pool.
#include <stdlib.h>

#include "kernels.h"
#include "tq_attn_common.h"

namespace lkv {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kChunk = 32;
constexpr int kORow = kD + 4;
constexpr int kMaxSplits = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct PagedParams {
  const uint16_t* q;        // [B, Hq, 128] fp16
  const uint16_t* kv;       // [max_pages, 2, ps, Hkv, 128] fp16
  const int32_t* indptr;    // [B + 1]
  const int32_t* indices;   // page ids
  const int32_t* last_len;  // [B]
  float* partials;          // [B, Hkv, nsplit, G (2 + 128)]
  uint16_t* out;            // [B, Hq, 128] fp16
  float scale_log2;
  int Hq, Hkv, G, ps, nsplit, split_tokens, max_pages;
  // decode step (DECODE): q|k|v GEMV partials, RoPE tables, the position
  const float* pq;
  const float* pk;
  const float* pv;
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  const int32_t* pos;
  uint16_t* kv_new;  // the pool, written at the new token's slot
  int nchunk, max_len;
};

// A split record: G maxima, G sums, then (from a 16-byte boundary) G x 128
// value sums; records are whole 16-byte units.
__host__ __device__ __forceinline__ int rec_acc_off(int G) { return (2 * G + 3) & ~3; }
__host__ __device__ __forceinline__ int rec_floats(int G) { return rec_acc_off(G) + G * kD; }

// Tokens of sequence b (0 without pages); its first page-table entry.
__device__ __forceinline__ int seq_tokens(const PagedParams& P, int b, int& first) {
  first = P.indptr[b];
  const int np = P.indptr[b + 1] - first;
  if (np <= 0) return 0;
  const int last = min(max(P.last_len[b], 0), P.ps);
  return (np - 1) * P.ps + last;
}

// Element offset of (token t, kv head, K or V) in the pool.
__device__ __forceinline__ size_t kv_offset(const PagedParams& P, int first, int t, int kvh, int side) {
  const int page = min(max(P.indices[first + t / P.ps], 0), P.max_pages - 1);
  const int slot = t % P.ps;
  return ((static_cast<size_t>(page) * 2 + side) * P.ps + slot) * (static_cast<size_t>(P.Hkv) * kD) +
         static_cast<size_t>(kvh) * kD;
}

constexpr int kMaxPg = 256;  // page ids of one split staged in LDS (SMALLG path)

// SMALLG (at most 4 query heads per kv head, the split's pages staged in LDS):
// a chunk's key rows and value rows (lane: 8-dim group lane % 16, the 8
// tokens of its scores) are loaded together, one memory round trip per chunk,
// every value row once; the values go through MFMA with no LDS traffic, and
// each lane rescales the output column of the head whose running max it
// holds.  Otherwise: page offsets through LDS, value rows per (8-dim group,
// head) lane in batches of 8.
//
// DECODE (the dense fp16-KV decode step; SMALLG layout, B = 1): identity
// pages (token t in page t / ps), length *pos + 1.  The prologue sums the
// q|k|v GEMV partials of the new token and applies RoPE at *pos (query and
// key rounded to fp16, exactly as a separate epilogue kernel storing fp16
// would); the partial loads and the wave's first chunk are in flight
// together.  The block whose split holds *pos writes the new key and value
// into the pool and uses them, from LDS, in place of the rows it loads for
// that token: no block reads the slot written in this launch.
template <bool SMALLG, bool DECODE>
__global__ __launch_bounds__(kThreads) void paged_split_kernel(PagedParams P) {
  static_assert(SMALLG || !DECODE, "the decode step runs the SMALLG layout");
  __shared__ float s_p[SMALLG ? 1 : kWaves][16][kChunk];
  __shared__ size_t s_off[SMALLG ? 1 : kWaves][kChunk];  // pool offset of each chunk token's value row
  __shared__ int s_pg[SMALLG && !DECODE ? kMaxPg + 1 : 1];
  __shared__ float s_alpha[SMALLG ? 1 : kWaves][16];
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ __align__(16) float s_o[kWaves][16][kORow];
  __shared__ float s_q[DECODE ? 4 : 1][kD];                     // decode: the RoPE'd query heads
  __shared__ __align__(16) uint16_t s_new[DECODE ? 2 : 1][kD];  // decode: the new key and value

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = P.G;
  const int h = lane & 15, g = lane >> 4;  // score layout: head column, token group
  const int dg = lane >> 2, hq = lane & 3;  // value layout: 8-dim group, head slot
  float* rec = P.partials + ((static_cast<size_t>(b) * P.Hkv + kvh) * P.nsplit + split) * rec_floats(G);

  int first = 0, len, pos = 0;
  if constexpr (DECODE) {
    pos = min(max(__builtin_amdgcn_readfirstlane(*P.pos), 0), P.max_len - 1);
    len = pos + 1;
  } else {
    len = seq_tokens(P, b, first);
  }
  const int t_begin = split * P.split_tokens;
  const int t_end = min(t_begin + P.split_tokens, len);
  if (t_begin >= t_end) {  // uniform: nothing of this sequence in this split
    if (tid < G) {
      rec[tid] = -INFINITY;
      rec[G + tid] = 0.f;
    }
    return;
  }
  const int pg0 = t_begin / P.ps;  // SMALLG: first page of the split
  if constexpr (SMALLG && !DECODE) {
    const int np = P.indptr[b + 1] - first;
    const int npg = (t_end - 1) / P.ps - pg0 + 1;  // <= kMaxPg + 1 (host plan)
    for (int i = tid; i < npg; i += kThreads) {
      const int pi = min(pg0 + i, np - 1);
      s_pg[i] = min(max(P.indices[first + pi], 0), P.max_pages - 1);
    }
    __syncthreads();
  }
  // pool offset of (token t of the split's range, side) for SMALLG
  auto off_of = [&](int t, int side) -> size_t {
    int page;
    if constexpr (DECODE)
      page = t / P.ps;
    else
      page = s_pg[t / P.ps - pg0];
    return ((static_cast<size_t>(page) * 2 + side) * P.ps + t % P.ps) * (static_cast<size_t>(P.Hkv) * kD) +
           static_cast<size_t>(kvh) * kD;
  };

  // SMALLG chunk registers: key rows of tokens c + 16 tt + (lane % 16) (dims
  // 8 (lane / 16) + 32 kb ..), value rows j of tokens c + 16 (j / 4) +
  // 4 (lane / 16) + j % 4 (dims 8 (lane % 16) ..): clamped valid tokens, masked later
  u32x4 a[2][4];
  uint4 vr[8];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const uint16_t* kp = P.kv + off_of(min(c + 16 * tt + h, t_end - 1), 0) + 8 * g;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint4 u = *reinterpret_cast<const uint4*>(kp + 32 * kb);
        a[tt][kb] = u32x4{u.x, u.y, u.z, u.w};
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      vr[j] = *reinterpret_cast<const uint4*>(P.kv + off_of(min(c + 16 * (j >> 2) + 4 * g + (j & 3), t_end - 1), 1) +
                                              8 * h);
  };
  const int c_first = t_begin + kChunk * wave;

  // B operand: query x scale * log2(e), head h (rows h >= G zero), dims 32 kb + 8 g + i
  u32x4 qa[4];
  bool writer = false;  // DECODE: this block's split holds the new token
  if constexpr (DECODE) {
    const uint16_t* cos_row = P.rope_cos + static_cast<size_t>(pos) * kD;
    const uint16_t* sin_row = P.rope_sin + static_cast<size_t>(pos) * kD;
    writer = pos < t_begin + P.split_tokens;  // pos >= t_begin: the split is not empty
    // Thread e < G * 64: query head e / 64, dim pair (e % 64, e % 64 + 64);
    // threads 0..63 / 64..127 also the key / value pair (t % 64, t % 64 + 64)
    // of the new token (loaded by every block, without a branch).  The first
    // kPre chunk partials from clamped, always valid addresses.
    constexpr int kPre = 8;
    float pre0[kPre], pre1[kPre], prk0[kPre], prk1[kPre];
    const int e = min(tid, G * (kD / 2) - 1);
    const int hh = e / (kD / 2), dd = e % (kD / 2);
    const uint16_t rc0 = cos_row[dd], rc1 = cos_row[dd + kD / 2];
    const uint16_t rs0 = sin_row[dd], rs1 = sin_row[dd + kD / 2];
    const int col = (kvh * G + hh) * kD + dd;
    const int t = tid & (kD - 1);
    const float* ksrc = t < kD / 2 ? P.pk : P.pv;
    const int kc0 = kvh * kD + (t & (kD / 2 - 1));
    {
      const float* p0 = P.pq + static_cast<size_t>(col / kGemvBN) * P.nchunk * kGemvBN + (col % kGemvBN);
      const float* p1 = P.pq + static_cast<size_t>((col + kD / 2) / kGemvBN) * P.nchunk * kGemvBN +
                        ((col + kD / 2) % kGemvBN);
      const float* k0 = ksrc + static_cast<size_t>(kc0 / kGemvBN) * P.nchunk * kGemvBN + (kc0 % kGemvBN);
      const float* k1 = ksrc + static_cast<size_t>((kc0 + kD / 2) / kGemvBN) * P.nchunk * kGemvBN +
                        ((kc0 + kD / 2) % kGemvBN);
#pragma unroll
      for (int i = 0; i < kPre; ++i) {
        const size_t o = static_cast<size_t>(min(i, P.nchunk - 1)) * kGemvBN;
        pre0[i] = p0[o];
        pre1[i] = p1[o];
        prk0[i] = k0[o];
        prk1[i] = k1[o];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the chunk's (results retire in order)
    if (c_first < t_end) load_chunk(c_first);
    // sums in column_sum2's order (chunk order from 0)
    if (tid < G * (kD / 2)) {
      float x0 = 0.f, x1 = 0.f, o0, o1;
      if (P.nchunk <= kPre) {
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          x0 += i < P.nchunk ? pre0[i] : 0.f;
          x1 += i < P.nchunk ? pre1[i] : 0.f;
        }
        rope_pair_v(x0, x1, rc0, rc1, rs0, rs1, o0, o1);
      } else {
        column_sum2(P.pq, col, col + kD / 2, P.nchunk, x0, x1);
        rope_pair(x0, x1, cos_row, sin_row, dd, o0, o1);
      }
      s_q[hh][dd] = o0;
      s_q[hh][dd + kD / 2] = o1;
    }
    if (writer && tid < kD) {
      float x0 = 0.f, x1 = 0.f, o0, o1;
      if (P.nchunk <= kPre) {
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          x0 += i < P.nchunk ? prk0[i] : 0.f;
          x1 += i < P.nchunk ? prk1[i] : 0.f;
        }
      } else {
        column_sum2(ksrc, kc0, kc0 + kD / 2, P.nchunk, x0, x1);
      }
      const int side = tid < kD / 2 ? 0 : 1;
      if (side == 0) {  // key pair (tid, tid + 64), RoPE'd (the factors of query element tid)
        if (P.nchunk <= kPre)
          rope_pair_v(x0, x1, rc0, rc1, rs0, rs1, o0, o1);
        else
          rope_pair(x0, x1, cos_row, sin_row, tid, o0, o1);
      } else {  // value dims (t - 64, t): no RoPE
        o0 = x0;
        o1 = x1;
      }
      const int d0 = t & (kD / 2 - 1);
      const uint16_t h0 = f2h(o0), h1 = f2h(o1);
      s_new[side][d0] = h0;
      s_new[side][d0 + kD / 2] = h1;
      uint16_t* dst = P.kv_new + off_of(pos, side);
      dst[d0] = h0;
      dst[d0 + kD / 2] = h1;
    }
    __syncthreads();
    const float* qrow = s_q[min(h, G - 1)];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * kb + 8 * g + 2 * j;
        v[j] = pack2h(qrow[d] * P.scale_log2, qrow[d + 1] * P.scale_log2);
      }
      qa[kb] = h < G ? v : u32x4{0u, 0u, 0u, 0u};
    }
  } else {
    const uint16_t* qrow = P.q + (static_cast<size_t>(b) * P.Hq + kvh * G + min(h, G - 1)) * kD + 8 * g;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint4 u = *reinterpret_cast<const uint4*>(qrow + 32 * kb);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = pack2h(h2f(static_cast<uint16_t>(w[j] & 0xffffu)) * P.scale_log2,
                      h2f(static_cast<uint16_t>(w[j] >> 16)) * P.scale_log2);
      qa[kb] = h < G ? v : u32x4{0u, 0u, 0u, 0u};
    }
    if constexpr (SMALLG) {
      if (c_first < t_end) load_chunk(c_first);
    }
  }

  float m = -INFINITY, lsum = 0.f;  // per lane: head h
  float acc[4][8];                  // general path, per lane: heads hq + 4 k, dims 8 dg ..
  f32x4 ov[8];                      // SMALLG: the value MFMA tiles
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[k][j] = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) ov[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (SMALLG) {
    for (int c = c_first; c < t_end;) {
      if constexpr (DECODE) {
        if (writer) {  // the new token's rows come from LDS, not from the slot written above
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            if (min(c + 16 * tt + h, t_end - 1) == pos) {
#pragma unroll
              for (int kb = 0; kb < 4; ++kb) a[tt][kb] = *reinterpret_cast<const u32x4*>(&s_new[0][32 * kb + 8 * g]);
            }
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (min(c + 16 * (j >> 2) + 4 * g + (j & 3), t_end - 1) == pos)
              vr[j] = *reinterpret_cast<const uint4*>(&s_new[1][8 * h]);
        }
      }
      // ---- scores, online softmax (lane: head h, tokens c + 16 tt + 4 g + i)
      f32x4 sc[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        sc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sc[tt] = mfma16x16x32(a[tt][kb], qa[kb], sc[tt]);
      }
      float s[8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * tt + i] = c + 16 * tt + 4 * g + i < t_end ? sc[tt][i] : -INFINITY;
      float mx = s[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mx = vmax(mx, s[j]);
      mx = xgroup_max(mx);
      const float mn = fmaxf(m, mx);  // finite: the chunk holds at least one token
      const float alpha = fast_exp2(m - mn);
      m = mn;
      float ps = 0.f, pr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pr[j] = fast_exp2(s[j] - mn);  // 0 for tokens past the end
        ps += pr[j];
      }
      lsum = lsum * alpha + ps;
      // ---- values on MFMA, transposed: A = 16 dim rows (8 (lane % 16) + t)
      // x 32 tokens (the lane's value rows, paired by v_perm), B = the
      // probabilities in fp16 (lane: head lane % 16, the same 8 tokens as its
      // scores); ov[t] row 4 (lane / 16) + i holds dim 8 (4 (lane / 16) + i) + t
      // of head lane % 16, whose running max this lane holds: the rescale
      // needs no exchange.
      const u32x4 pb = u32x4{pack2h(pr[0], pr[1]), pack2h(pr[2], pr[3]), pack2h(pr[4], pr[5]), pack2h(pr[6], pr[7])};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
        u32x4 av;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint4& r0 = vr[2 * pp];
          const uint4& r1 = vr[2 * pp + 1];
          const uint32_t x0 = (t >> 1) == 0 ? r0.x : (t >> 1) == 1 ? r0.y : (t >> 1) == 2 ? r0.z : r0.w;
          const uint32_t x1 = (t >> 1) == 0 ? r1.x : (t >> 1) == 1 ? r1.y : (t >> 1) == 2 ? r1.z : r1.w;
          av[pp] = __builtin_amdgcn_perm(x1, x0, sel);
        }
        ov[t] = mfma16x16x32(av, pb, ov[t] * alpha);
      }
      __builtin_amdgcn_wave_barrier();
      c += kChunk * kWaves;
      if (c < t_end) load_chunk(c);
    }
  } else {
    for (int c = t_begin + kChunk * wave; c < t_end; c += kChunk * kWaves) {
      // ---- scores: tokens c + 16 tt + (lane % 16) as A rows
      f32x4 sc[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tok = min(c + 16 * tt + h, t_end - 1);  // clamped valid token, masked below
        const size_t off = kv_offset(P, first, tok, kvh, 0);
        if (g == 0) s_off[wave][16 * tt + h] = off + static_cast<size_t>(P.ps) * P.Hkv * kD;  // its value row
        const uint16_t* kp = P.kv + off + 8 * g;
        u32x4 a[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const uint4 u = *reinterpret_cast<const uint4*>(kp + 32 * kb);
          a[kb] = u32x4{u.x, u.y, u.z, u.w};
        }
        sc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sc[tt] = mfma16x16x32(a[kb], qa[kb], sc[tt]);
      }
      // D: lane holds head h, tokens c + 16 tt + 4 g + i
      float s[8];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * tt + i] = c + 16 * tt + 4 * g + i < t_end ? sc[tt][i] : -INFINITY;
      float mx = s[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mx = vmax(mx, s[j]);
      mx = xgroup_max(mx);
      const float mn = fmaxf(m, mx);  // finite: the chunk holds at least one token
      const float alpha = fast_exp2(m - mn);
      m = mn;
      float ps = 0.f;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(s[4 * tt + i] - mn);
          ps += p;
          s_p[wave][h][16 * tt + 4 * g + i] = p;
        }
      lsum = lsum * alpha + ps;
      if (g == 0) s_alpha[wave][h] = alpha;
      __builtin_amdgcn_wave_barrier();
      // ---- values: lane (dims 8 dg .., heads hq + 4 k) over the chunk's tokens
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float al = s_alpha[wave][hq + 4 * k];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[k][j] *= al;
      }
      // the chunk's 32 value rows, 8 loads in flight per group; tokens past the
      // end read the last valid row (clamped offsets) with p = 0
#pragma unroll
      for (int t0 = 0; t0 < kChunk; t0 += 8) {
        uint4 u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) u[i] = *reinterpret_cast<const uint4*>(P.kv + s_off[wave][t0 + i] + 8 * dg);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
          float v[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] = h2f(static_cast<uint16_t>(w[e] & 0xffffu));
            v[2 * e + 1] = h2f(static_cast<uint16_t>(w[e] >> 16));
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (hq + 4 * k < G) {  // lanes past the G heads skip
              const float p = s_p[wave][hq + 4 * k][t0 + i];
#pragma unroll
              for (int j = 0; j < 8; ++j) acc[k][j] = fmaf(p, v[j], acc[k][j]);
            }
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- merge the 4 waves (a wave without a chunk keeps m = -inf, l = 0, o = 0)
  const float ltot = xgroup_sum(lsum);
  if (g == 0) {
    s_m[wave][h] = m;
    s_l[wave][h] = ltot;
  }
  if constexpr (SMALLG) {  // lane: head h, dims 8 (4 g + i) + t
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4* dst = reinterpret_cast<float4*>(&s_o[wave][h][8 * (4 * g + i)]);
      dst[0] = make_float4(ov[0][i], ov[1][i], ov[2][i], ov[3][i]);
      dst[1] = make_float4(ov[4][i], ov[5][i], ov[6][i], ov[7][i]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float4* dst = reinterpret_cast<float4*>(&s_o[wave][hq + 4 * k][8 * dg]);
      dst[0] = make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
      dst[1] = make_float4(acc[k][4], acc[k][5], acc[k][6], acc[k][7]);
    }
  }
  __syncthreads();
  for (int e = tid; e < G * kD; e += kThreads) {
    const int hh = e / kD, d = e % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][hh]);
    float o = 0.f, l = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = s_m[w][hh] == -INFINITY ? 0.f : fast_exp2(s_m[w][hh] - M);
        o += wt * s_o[w][hh][d];
        l += wt * s_l[w][hh];
      }
    }
    rec[rec_acc_off(G) + hh * kD + d] = o;
    if (d == 0) {
      rec[hh] = M;
      rec[G + hh] = l;
    }
  }
}

// One block of 256 threads per (query head, batch): merge the split records.
// Thread s < nsplit reads split s's maximum and sum (block max / sum through
// the waves); thread (dg = tid % 32, grp = tid / 32) reads the value sums of
// splits grp, grp + 8, ... at dims 4 dg .. 4 dg + 3 (float4), all issued
// before the first wait; the 8 split groups are joined in LDS in order.
constexpr int kPcThreads = 256;
constexpr int kPcGroups = kPcThreads / 32;
constexpr int kPcDepth = 8;  // value sums per thread loaded up front: 64 splits in one pass (more: further passes)
__global__ __launch_bounds__(kPcThreads) void paged_combine_kernel(PagedParams P) {
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[kPcThreads / 64];
  __shared__ __align__(16) float s_o[kPcGroups][kD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hq = blockIdx.x, b = blockIdx.y;
  const int G = P.G, kvh = hq / G, hh = hq % G, ns = P.nsplit, RF = rec_floats(G);
  const float* recs = P.partials + (static_cast<size_t>(b) * P.Hkv + kvh) * ns * RF;
  const int dg = tid & 31, grp = tid >> 5;
  float ms, ls;
  {
    const size_t sr = static_cast<size_t>(min(tid, ns - 1)) * RF;
    const float m_ = recs[sr + hh], l_ = recs[sr + G + hh];
    ms = tid < ns ? m_ : -INFINITY;
    ls = tid < ns ? l_ : 0.f;
  }
  float4 ov[kPcDepth];
#pragma unroll
  for (int i = 0; i < kPcDepth; ++i)
    ov[i] = *reinterpret_cast<const float4*>(recs + static_cast<size_t>(min(grp + kPcGroups * i, ns - 1)) * RF +
                                             rec_acc_off(G) + hh * kD + 4 * dg);
  float v = wave_max(ms);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kPcThreads / 64; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const float w_s = (tid < ns && ms != -INFINITY) ? fast_exp2(ms - M) : 0.f;
  if (tid < ns) s_w[tid] = w_s;
  float lv = wave_sum(w_s * ls);
  if (lane == 0) s_red[wave] = lv;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kPcThreads / 64; ++w) L += s_red[w];
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += kPcGroups * kPcDepth) {
#pragma unroll
    for (int i = 0; i < kPcDepth; ++i) {
      const int sp = s0 + grp + kPcGroups * i;
      if (s0 > 0)
        ov[i] = *reinterpret_cast<const float4*>(recs + static_cast<size_t>(min(sp, ns - 1)) * RF + rec_acc_off(G) +
                                                 hh * kD + 4 * dg);
      const float w = sp < ns ? s_w[sp] : 0.f;
      if (w != 0.f) {  // a split with no tokens left its sums unwritten: select, never multiply
        o.x = fmaf(w, ov[i].x, o.x);
        o.y = fmaf(w, ov[i].y, o.y);
        o.z = fmaf(w, ov[i].z, o.z);
        o.w = fmaf(w, ov[i].w, o.w);
      }
    }
  }
  *reinterpret_cast<float4*>(&s_o[grp][4 * dg]) = o;
  __syncthreads();
  if (tid < kD) {
    float r = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < kPcGroups; ++g2) r += s_o[g2][tid];
    P.out[(static_cast<size_t>(b) * P.Hq + hq) * kD + tid] = f2h(L > 0.f ? r / L : 0.f);
  }
}

// Fewest tokens per split (LKV_PAGED_MIN_SPLIT_TOKENS overrides, tuning sweeps).
int64_t paged_min_split_tokens() {
  static const int64_t k = [] {
    const char* env = getenv("LKV_PAGED_MIN_SPLIT_TOKENS");
    const long v = env ? atol(env) : 128;
    return static_cast<int64_t>(v > 0 && v <= (1 << 20) ? v : 128);
  }();
  return k;
}

struct PagedPlan {
  int nsplit, split_tokens;
  size_t bytes;
};

PagedPlan paged_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len) {
  PagedPlan p{};
  const int64_t target = 2 * static_cast<int64_t>(device_cu_count());
  int64_t ns = (target + B * Hkv - 1) / (B * Hkv);
  ns = ns < 1 ? 1 : (ns > kMaxSplits ? kMaxSplits : ns);
  constexpr int64_t gran = kChunk * kWaves;
  int64_t ts = (max(max_len, int64_t{1}) + ns - 1) / ns;
  if (ts < paged_min_split_tokens()) ts = paged_min_split_tokens();
  ts = (ts + gran - 1) / gran * gran;
  ns = (max(max_len, int64_t{1}) + ts - 1) / ts;
  p.nsplit = static_cast<int>(ns);
  p.split_tokens = static_cast<int>(ts);
  p.bytes = static_cast<size_t>(B * Hkv * ns) * rec_floats(static_cast<int>(Hq / Hkv)) * 4 + 256;
  return p;
}

}  // namespace

int f16kv_step_attn(const F16kvStepAttn& a, hipStream_t st) {
  LKV_REQUIRE(a.Hq > 0 && a.Hkv > 0 && a.Hq % a.Hkv == 0 && a.Hq / a.Hkv <= 4,
              "f16kv_step_attn: need Hq %% Hkv == 0 and Hq/Hkv <= 4 (Hq=%lld Hkv=%lld)", (long long)a.Hq,
              (long long)a.Hkv);
  LKV_REQUIRE(a.max_len >= 1 && a.max_len < (1ll << 30) && a.page_size >= 1 && a.max_pages >= 1 &&
                  a.max_len <= a.max_pages * a.page_size && a.nchunk >= 1,
              "f16kv_step_attn: max_len=%lld page_size=%lld max_pages=%lld nchunk=%d out of range",
              (long long)a.max_len, (long long)a.page_size, (long long)a.max_pages, a.nchunk);
  const PagedPlan pl = paged_plan(1, a.Hq, a.Hkv, a.max_len);
  LKV_REQUIRE(a.records && a.record_bytes >= pl.bytes, "f16kv_step_attn: %zu record bytes required, got %zu",
              pl.bytes, a.record_bytes);
  PagedParams P{};
  P.kv = a.kv;
  P.partials = static_cast<float*>(a.records);
  P.out = a.out;
  P.scale_log2 = a.scale * kLog2e;
  P.Hq = static_cast<int>(a.Hq);
  P.Hkv = static_cast<int>(a.Hkv);
  P.G = static_cast<int>(a.Hq / a.Hkv);
  P.ps = static_cast<int>(a.page_size);
  P.nsplit = pl.nsplit;
  P.split_tokens = pl.split_tokens;
  P.max_pages = static_cast<int>(a.max_pages);
  P.pq = a.pq;
  P.pk = a.pk;
  P.pv = a.pv;
  P.rope_cos = a.rope_cos;
  P.rope_sin = a.rope_sin;
  P.pos = a.pos;
  P.kv_new = a.kv;
  P.nchunk = a.nchunk;
  P.max_len = static_cast<int>(a.max_len);
  hipLaunchKernelGGL((paged_split_kernel<true, true>), dim3(static_cast<unsigned>(pl.nsplit), static_cast<unsigned>(a.Hkv)),
                     dim3(kThreads), 0, st, P);
  LKV_LAUNCH_CHECK("f16kv_step_attn split");
  hipLaunchKernelGGL(paged_combine_kernel, dim3(static_cast<unsigned>(a.Hq)), dim3(kPcThreads), 0, st, P);
  LKV_LAUNCH_CHECK("f16kv_step_attn combine");
  return LKV_OK;
}

}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_paged_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0) return 256;
  return paged_plan(B, Hq, Hkv, max_len).bytes;
}

extern "C" int lkv_paged_decode_attn(const void* q, const void* kv_data, const int32_t* kv_indptr,
                                     const int32_t* kv_indices, const int32_t* kv_last_page_len, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t page_size, int64_t max_pages,
                                     int64_t max_len, float scale, void* out, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  LKV_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16,
              "paged_decode_attn: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%lld Hkv=%lld)", (long long)Hq,
              (long long)Hkv);
  LKV_REQUIRE(page_size >= 1 && page_size <= 65536 && max_pages >= 1,
              "paged_decode_attn: page_size=%lld / max_pages=%lld out of range", (long long)page_size,
              (long long)max_pages);
  LKV_REQUIRE(max_len >= 0 && max_len < (1ll << 30), "paged_decode_attn: max_len=%lld out of range",
              (long long)max_len);
  LKV_REQUIRE(max_pages * 2 * page_size * Hkv * kD < (1ll << 40), "paged_decode_attn: pool too large");
  if (B == 0) return LKV_OK;
  LKV_REQUIRE(q && kv_data && kv_indptr && kv_indices && kv_last_page_len && out && workspace,
              "paged_decode_attn: null pointer");
  LKV_REQUIRE(aligned16(q) && aligned16(kv_data) && aligned16(out) && aligned16(workspace),
              "paged_decode_attn: q, kv_data, out and workspace must be 16-byte aligned");
  const PagedPlan pl = paged_plan(B, Hq, Hkv, max_len);
  LKV_REQUIRE(workspace_bytes >= pl.bytes, "paged_decode_attn: workspace of %zu bytes required, got %zu", pl.bytes,
              workspace_bytes);
  PagedParams P;
  P.q = static_cast<const uint16_t*>(q);
  P.kv = static_cast<const uint16_t*>(kv_data);
  P.indptr = kv_indptr;
  P.indices = kv_indices;
  P.last_len = kv_last_page_len;
  P.partials = static_cast<float*>(workspace);
  P.out = static_cast<uint16_t*>(out);
  P.scale_log2 = scale * kLog2e;
  P.Hq = static_cast<int>(Hq);
  P.Hkv = static_cast<int>(Hkv);
  P.G = static_cast<int>(Hq / Hkv);
  P.ps = static_cast<int>(page_size);
  P.nsplit = pl.nsplit;
  P.split_tokens = pl.split_tokens;
  P.max_pages = static_cast<int>(max_pages);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(pl.nsplit), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
  // the SMALLG path stages a split's pages in LDS: (ts - 1) / ps + 2 of them at most
  const bool small = Hq / Hkv <= 4 && (pl.split_tokens - 1) / page_size + 2 <= kMaxPg + 1;
  if (small)
    hipLaunchKernelGGL((paged_split_kernel<true, false>), grid, dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((paged_split_kernel<false, false>), grid, dim3(kThreads), 0, st, P);
  LKV_LAUNCH_CHECK("paged_decode_attn split");
  hipLaunchKernelGGL(paged_combine_kernel, dim3(static_cast<unsigned>(Hq), static_cast<unsigned>(B)),
                     dim3(kPcThreads), 0, st, P);
  LKV_LAUNCH_CHECK("paged_decode_attn combine");
  return LKV_OK;
}
