// Split-K flash-decode attention that reads the TurboQuant packed KV cache.
//
// Reference semantics: TurboQuantCache._get_full_cache (leankv/turboquant/
// cache.py:169-189) dequantizes every cold token to fp16 and concatenates the
// fp16 hot window; HF SDPA (transformers/integrations/sdpa_attention.py:79-105)
// then runs GQA attention for the single decode query.  Here no dequantized
// K/V ever exists.  With K_hat_t = n_t * c[idx_t] @ PiK (quantizer.py:131-137):
//   q . K_hat_t = n_t * (q @ PiK^T) . c[idx_t]
//   sum_t p_t V_hat_t = (sum_t p_t n_t c[idx_t]) @ PiV
// so the query is rotated once, cold scores and the cold value sum stay in the
// rotated domain, and PiV is applied once per query head at the end.
//
// Launches (all on the caller's stream, no inter-block waits):
//   1. split kernel, grid splits x kv_heads x batch, 4 waves per block, each
//      block owning a contiguous range of cold tokens.  Its prologue rotates
//      the G query heads of its kv head, q_rot = q @ PiK^T on fp32 MFMA
//      (the decode step passes q_rot from its own QKV epilogue instead),
//      while the first token blocks load.  Each wave then walks 32-token
//      blocks with two register sets in turn (the next block's codes and
//      norms load while the current one is computed):
//      * scores, transposed: v_mfma_f32_16x16x32_f16 with A = 16 tokens x 32
//        dims of centroid values and B = the rotated query (16 head
//        columns, G used), so a lane holds one head's scores for 8 tokens.
//        3-bit codes are decoded on the VALU with v_perm_b32 table lookups;
//        4-bit codes through a 256-entry LDS table (byte -> fp16 pair);
//      * online softmax in the exp2 domain, per lane, with the max taken
//        across the 4 lanes of a head by two permlane swaps; the offset keeps
//        a headroom above the max, so the rescale of the accumulators runs
//        only when some head's score passes it;
//      * values, transposed: the same MFMA with A = 16 dims x 32 tokens of
//        centroid values (a lane's 8 tokens of one dim, transposed from the
//        decoded code dwords with v_perm_b32) and B = p * n_t taken straight
//        from the lane's own softmax registers (same 8 tokens);
//      * the 4 waves merge through LDS and the block writes
//        (m, l, acc[G][128]) per head to the workspace;
//   2. combine kernel, one block of 8 waves per (batch, query head): issues
//      every load it needs at once (split maxima and sums, the rotated
//      partial sums, the fp16 hot window and the PiV column slice), then
//      computes the hot scores, merges hot and cold softmax statistics,
//      applies PiV to the cold sum, adds the hot sum, normalises, writes fp16.
#include <stdlib.h>

#include "kernels.h"
#include "tq_attn_common.h"
#include "tq_common.h"

namespace lkv {
namespace {

#ifdef LKV_STAMPS
// Instrumented build only (build.py --stamps): per-block phase times on the
// 100 MHz real-time clock, [block][8 stamps] for the split kernel (0 block
// start, 1 token loop start, 2 token loop end, 3 block end; inside the
// prologue 4 = query ready for the rotation, 5 = rotation done) and the
// combine kernel (0 start, 3 end), block = linear id in the grid.  Thread 0
// stores them.
constexpr int kStampBlocks = 16384;
constexpr int kStampSlots = 8;
__device__ uint64_t g_split_stamps[kStampBlocks * kStampSlots];
__device__ uint64_t g_comb_stamps[kStampBlocks * kStampSlots];
__device__ __forceinline__ void stamp(uint64_t* arr, int i) {
  if (threadIdx.x == 0) {
    const unsigned id = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (id < kStampBlocks)
      __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(), arr + kStampSlots * id + i);
  }
}
#define LKV_SPLIT_STAMP(i) stamp(g_split_stamps, i)
#define LKV_COMB_STAMP(i) stamp(g_comb_stamps, i)
#else
#define LKV_SPLIT_STAMP(i) \
  do {                     \
  } while (0)
#define LKV_COMB_STAMP(i) \
  do {                    \
  } while (0)
#endif

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kBlk = 32;    // tokens per wave step
constexpr int kHotMax = 256;  // hot-window slots the combine walks (64 per slot group)
constexpr float kLog2e = 1.4426950408889634f;

// Max / sum across the 16 lanes of a row group (lanes with equal lane/16).
__device__ __forceinline__ float group16_max(float v) { return row16_max(v); }
__device__ __forceinline__ float group16_sum(float v) { return row16_sum(v); }

struct AttnParams {
  const float* qrot;        // [B, Hq, 128] fp32 = q @ PiK^T
  const uint16_t* q;        // [B, Hq, 128] fp16 (the hot window uses the unrotated query)
  const uint8_t* k_codes;   // [B, Hkv, cap, 64]
  const float* k_norms;     // [B, Hkv, cap]
  const uint8_t* v_codes;
  const float* v_norms;
  const uint16_t* k_hot;    // [B, Hkv, hot_cap, 128]
  const uint16_t* v_hot;
  const float* PiV;         // [128, 128]
  const float* PiK;         // non-null: the split kernel rotates q itself (qrot unused)
  const float* centroids;   // [2^bits]
  const int32_t* seq_len;
  float* partials;          // [B, Hkv, nsplit, rec]
  uint16_t* out;            // [B, Hq, 128]
  float scale_log2;         // scale * log2(e)
  int max_len, Hq, Hkv, G, cap, hot_cap, nsplit, split_tokens, ncent;
  // paged cold store only: FlashInfer's CSR page table over pools of
  // [max_pages][Hkv][page_size] rows, seq_len holding one length per sequence
  const int32_t* indptr;
  const int32_t* indices;
  int page_shift, max_pages;
  uint32_t pool_code_bytes, pool_norm_bytes;
  // decode step only (AttnCall: q|k|v partials, RoPE, ring write)
  const float* pq;
  const float* pk;
  const float* pv;
  int nchunk;
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  const int32_t* pos;
  uint16_t* q16;
  uint16_t* k_ring;
  uint16_t* v_ring;
};

// A split record: G maxima, G sums, then (from a 16-byte boundary) G x 128
// rotated value sums; records are whole 16-byte units.
__host__ __device__ __forceinline__ int rec_acc_off(int G) { return (2 * G + 3) & ~3; }
__host__ __device__ __forceinline__ int rec_floats(int G) { return rec_acc_off(G) + G * kD; }

// Code rows by stored width CB: 4 = nibble rows (3- and 4-bit codes, 64 B per
// token), 2 = four 2-bit codes per byte (32 B), 1 = eight 1-bit codes per byte
// (16 B), the packings of leankv/turboquant/quantizer.py:38-62.  Narrow rows
// are widened to nibbles in registers as they arrive, so the decode after
// that (v_perm over a centroid table padded with zeros) is the 3-bit one.
template <int CB>
__host__ __device__ constexpr int code_row_bytes() {
  return kD * CB / 8;
}
// 16 bits of 2-bit codes (dims 0..7 at bits 2d) -> dims at bits 4d.
__device__ __forceinline__ uint32_t nib_from2(uint32_t x) {
  uint32_t t = x & 0xffffu;
  t = (t | (t << 8)) & 0x00ff00ffu;
  t = (t | (t << 4)) & 0x0f0f0f0fu;
  return (t | (t << 2)) & 0x33333333u;
}
// 8 bits of 1-bit codes (dim d at bit d) -> dims at bits 4d.
__device__ __forceinline__ uint32_t nib_from1(uint32_t x) {
  uint32_t t = x & 0xffu;
  t = (t | (t << 12)) & 0x000f000fu;
  t = (t | (t << 6)) & 0x03030303u;
  return (t | (t << 3)) & 0x11111111u;
}
// Dims 32k .. 32k+31 of a code row as 4 nibble dwords; voff/soff address the
// row's byte 4*CB*k.
template <int CB>
__device__ __forceinline__ u32x4 load_codes32(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  if constexpr (CB == 4) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  } else if constexpr (CB == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    const uint32_t lo = v[0], hi = v[1];
    return u32x4{nib_from2(lo), nib_from2(lo >> 16), nib_from2(hi), nib_from2(hi >> 16)};
  } else {
    const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    return u32x4{nib_from1(v), nib_from1(v >> 8), nib_from1(v >> 16), nib_from1(v >> 24)};
  }
}
// Dims 8k .. 8k+7 of a code row as one nibble dword (row byte CB*k).
template <int CB>
__device__ __forceinline__ uint32_t load_codes8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  if constexpr (CB == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  else if constexpr (CB == 2)
    return nib_from2(__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
  else
    return nib_from1(__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0));
}

// Buffer resource over `bytes` bytes at base (raw addressing, stride 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// The (batch, kv head) slice of the cold store as four buffer resources.
struct ColdRsrc {
  __amdgpu_buffer_rsrc_t kc, vc, kn, vn;
};

// Registers of one 32-token block t0 .. t0+31 (two 16-token tiles tt) for
// lane l = 16g + w:
//   kraw[tt]    code bytes 16g .. 16g+15 of token t0 + 16tt + w  (score operand)
//   kn[tt][i]   key norm   of token t0 + 16tt + 4g + i
//   vn[tt][i]   value norm of token t0 + 16tt + 4g + i
//   vdw[4tt+i]  code dword w (dims 8w .. 8w+7) of token t0 + 16tt + 4g + i
// The score MFMA leaves the score of token t0 + 16tt + 4g + i for head w in
// lane l, element i of tile tt, so the softmax weights, the value norms and
// the value codes a lane needs all belong to the same eight tokens: the value
// MFMA takes its probability operand straight from the lane's registers.
struct BlockRegs {
  u32x4 kraw[2];
  f32x4 kn[2], vn[2];
  uint32_t vdw[8];
};

// Token -> row of the buffer resources.  Dense: the (batch, kv head) slice is
// contiguous, row = token.  Paged: token t of the split lies in page
// s_pg[(t - t_begin) >> shift] at slot t % page_size, and the pools hold rows
// (page * Hkv + kv head) * page_size + slot, so a 16-token tile (page size a
// multiple of 16, tiles 16-aligned) is 16 consecutive rows.
struct DenseRows {
  __device__ __forceinline__ int operator()(int t) const { return t; }
};
struct PagedRows {
  const int* s_pg;
  int t_begin, shift, kvh, Hkv;
  __device__ __forceinline__ int operator()(int t) const {
    const int pg = s_pg[(t - t_begin) >> shift];
    return ((pg * Hkv + kvh) << shift) + (t & ((1 << shift) - 1));
  }
};

// A block entirely below the valid end.  Each load's voffset is one of two
// lane bases; everything that depends on the block or the load is in the
// scalar soffset (so no per-load vector address registers stay live).
template <int CB, typename Rows>
__device__ __forceinline__ void load_full(BlockRegs& R, const ColdRsrc& rs, int t0, int lane, const Rows& rows) {
  constexpr int RB = code_row_bytes<CB>();
  const int g = lane >> 4, w = lane & 15;
  const int vk = w * RB + 4 * CB * g;  // key codes: token w, dims 32g..
  const int vv = 4 * g * RB + CB * w;  // value codes: token 4g, dims 8w..
  const int vnrm = 16 * g;             // norms: token 4g
  const int r0 = __builtin_amdgcn_readfirstlane(rows(t0)), r1 = __builtin_amdgcn_readfirstlane(rows(t0 + 16));
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int sc = (tt ? r1 : r0) * RB, sn = (tt ? r1 : r0) * 4;
    R.kraw[tt] = load_codes32<CB>(rs.kc, vk, sc);
    R.kn[tt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.kn, vnrm, sn, 0));
    R.vn[tt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.vn, vnrm, sn, 0));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) R.vdw[j] = load_codes8<CB>(rs.vc, vv, ((j >> 2) ? r1 : r0) * RB + (j & 3) * RB);
}

// load_full for a block that may reach past the cold store (the prologue's
// unconditional loads): the row offset goes into the vector offset, which the
// buffer descriptor range-checks (rows at or past the end read 0), and the
// scalar offset is 0.  Dense layout only.
template <int CB>
__device__ __forceinline__ void load_full_checked(BlockRegs& R, const ColdRsrc& rs, int t0, int lane) {
  constexpr int RB = code_row_bytes<CB>();
  const int g = lane >> 4, w = lane & 15;
  const int vk = w * RB + 4 * CB * g, vv = 4 * g * RB + CB * w, vnrm = 16 * g;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int r = t0 + 16 * tt;
    R.kraw[tt] = load_codes32<CB>(rs.kc, vk + r * RB, 0);
    R.kn[tt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.kn, vnrm + r * 4, 0, 0));
    R.vn[tt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.vn, vnrm + r * 4, 0, 0));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) R.vdw[j] = load_codes8<CB>(rs.vc, vv + (t0 + 16 * (j >> 2) + (j & 3)) * RB, 0);
}

// A block reaching past t_lim: tokens at or past t_lim read token t_lim - 1
// (valid memory); the caller masks them.
template <int CB, typename Rows>
__device__ __forceinline__ void load_clamped(BlockRegs& R, const ColdRsrc& rs, int t0, int t_lim, int lane,
                                             const Rows& rows) {
  constexpr int RB = code_row_bytes<CB>();
  const int g = lane >> 4, w = lane & 15;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tk = min(t0 + 16 * tt + w, t_lim - 1);
    R.kraw[tt] = load_codes32<CB>(rs.kc, rows(tk) * RB + 4 * CB * g, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tn = min(t0 + 16 * tt + 4 * g + i, t_lim - 1);
      const int rn = rows(tn);
      R.kn[tt][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs.kn, rn * 4, 0, 0));
      R.vn[tt][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs.vn, rn * 4, 0, 0));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int tv = min(t0 + 16 * (j >> 2) + 4 * g + (j & 3), t_lim - 1);
    R.vdw[j] = load_codes8<CB>(rs.vc, rows(tv) * RB + CB * w, 0);
  }
}

template <int CB, typename Rows>
__device__ __forceinline__ void fetch_block(BlockRegs& R, const ColdRsrc& rs, int t0, int t_addr_end, int lane,
                                            const Rows& rows) {
  t0 = __builtin_amdgcn_readfirstlane(t0);  // wave-uniform: keeps the token offset scalar
  if (t0 + kBlk <= t_addr_end)
    load_full<CB>(R, rs, t0, lane, rows);
  else
    load_clamped<CB>(R, rs, t0, t_addr_end, lane, rows);
}

// Online-softmax state of one lane: head w = lane % 16, output dims
// 32g + 8i + dim(t) in o[t][i] (dim(t) = kPermDim[t] with PERM, else t).
struct SoftmaxState {
  float m, l;  // running max (log2 domain) and this lane's share of the sum
  f32x4 o[8];
};

// One 32-token block.  MASKED: tokens at or past t_end take no part.
template <bool PERM, bool MASKED>
__device__ __forceinline__ void attend_block(const BlockRegs& R, int t0, int t_end, const u32x4 (&qa)[4],
                                             const uint32_t (&tab)[4], const uint32_t* s_lut, int lane,
                                             SoftmaxState& S) {
  const int g = lane >> 4;
  // ---- scores, transposed: A = 16 tokens x 32 dims of centroids, B = the
  // rotated query (16 heads); lane gets head lane%16, tokens 4g+i of tile tt.
  float s[8];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint32_t dd[4];
      decode_dw<PERM>(R.kraw[tt][kb], tab, s_lut, dd);
      acc = mfma16x16x32(u32x4{dd[0], dd[1], dd[2], dd[3]}, qa[kb], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = acc[i] * R.kn[tt][i];
      s[4 * tt + i] = (!MASKED || t0 + 16 * tt + 4 * g + i < t_end) ? v : -INFINITY;
    }
  }
  // ---- online softmax; the rescale runs only when some head's score passes
  // its offset (the max plus kHeadroom when it last moved)
  float bm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
  bm = xgroup_max(bm);  // finite: token t0 of the block is always valid
  if (__builtin_amdgcn_ballot_w64(bm > S.m) != 0) {
    const float mn = bm > S.m ? bm + kHeadroom : S.m;
    const float alpha = fast_exp2(S.m - mn);  // 0 on the first block (m = -inf)
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) S.o[t][i] *= alpha;
    S.l *= alpha;
    S.m = mn;
  }
  float pv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = fast_exp2(s[j] - S.m);  // masked: exp2(-inf) = 0
    S.l += p;
    const float v = p * R.vn[j >> 2][j & 3];
    pv[j] = (!MASKED || t0 + 16 * (j >> 2) + 4 * g + (j & 3) < t_end) ? v : 0.f;
  }
  const u32x4 pb = u32x4{pack2h(pv[0], pv[1]), pack2h(pv[2], pv[3]), pack2h(pv[4], pv[5]), pack2h(pv[6], pv[7])};
  // ---- values, transposed: A = 16 dims x 32 tokens of centroids (the
  // lane's 8 tokens of dim 8w + dim(t)), B = p * n_v (the lane's 8 tokens).
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    uint32_t r[8][2];  // r[token j][q] = fp16 pair of positions 4half+2q, 4half+2q+1 of dims 8w..8w+7
#pragma unroll
    for (int j = 0; j < 8; ++j) decode_half<PERM>(R.vdw[j], half, tab, s_lut, r[j]);
#pragma unroll
    for (int tq = 0; tq < 4; ++tq) {
      const int t = 4 * half + tq, q = tq >> 1;
      u32x4 a;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t x0 = r[2 * pp][q], x1 = r[2 * pp + 1][q];
        a[pp] = (t & 1) ? __builtin_amdgcn_perm(x1, x0, 0x07060302u) : __builtin_amdgcn_perm(x1, x0, 0x05040100u);
      }
      S.o[t] = mfma16x16x32(a, pb, S.o[t]);
    }
  }
}

template <bool PERM>
__device__ __forceinline__ void attend(const BlockRegs& R, int t0, int t_end, const u32x4 (&qa)[4],
                                       const uint32_t (&tab)[4], const uint32_t* s_lut, int lane, SoftmaxState& S) {
  if (t0 + kBlk <= t_end)
    attend_block<PERM, false>(R, t0, t_end, qa, tab, s_lut, lane, S);
  else
    attend_block<PERM, true>(R, t0, t_end, qa, tab, s_lut, lane, S);
}

constexpr int kORow = kD + 4;  // padded LDS row of the per-wave outputs
#ifndef LKV_ATTN_BLOCKS_PER_CU
#define LKV_ATTN_BLOCKS_PER_CU 2
#endif
// Resident split blocks per CU (one wave per SIMD each): sets the register
// budget and the split count.
constexpr int kSplitBlocksPerCU = LKV_ATTN_BLOCKS_PER_CU;

constexpr int kMaxPg = 256;  // pages of one split in the paged layout

// QPRE (decode mode): q|k|v partial chunks loaded ahead of the codes, at least
// the q|k|v GEMV's chunk count for the fast path (8 or 16).
template <bool PERM, bool DECODE, bool PAGED, int CB, int QPRE = 16>
__global__ __launch_bounds__(kThreads, kSplitBlocksPerCU) void tq_attn_split_kernel(AttnParams P) {
  static_assert(!(PAGED && DECODE), "the fused decode step uses the dense layout");
  static_assert(CB == 4 || PERM, "narrow code rows (1, 2 bits) decode through v_perm");
  constexpr int RB = code_row_bytes<CB>();
  __shared__ uint32_t s_lut[256];
  __shared__ int s_pg[PAGED ? kMaxPg : 1];
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ __align__(16) float s_o[kWaves][16][kORow];  // all 16 heads: rows >= G are never read

  LKV_SPLIT_STAMP(0);
  // wave index made wave-uniform (scalar) so block offsets become scalar soffsets
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = P.G;
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  float* rec = P.partials + (bh * P.nsplit + split) * rec_floats(G);

  // The split's token range is static; the current length only masks it.
  // So the length load, the wave's first token block, the centroids and the
  // rotated query are all in flight before the first wait.
  const int t_begin = split * P.split_tokens;
  int t_addr_end, seq_len;  // valid memory: tokens below t_addr_end
  ColdRsrc rs;
  const PagedRows prow{s_pg, t_begin, P.page_shift, kvh, P.Hkv};
  if constexpr (PAGED) {
    // Sequence b owns pages indices[indptr[b] .. indptr[b + 1]); the split's
    // pages go to LDS, clamped to the pool; tokens past the sequence's pages
    // are past t_addr_end (the page of a clamped load is always one it owns).
    seq_len = __builtin_amdgcn_readfirstlane(P.seq_len[b]);
    const int pbeg = P.indptr[b], npg_seq = max(0, P.indptr[b + 1] - pbeg);
    t_addr_end = min(t_begin + P.split_tokens, npg_seq << P.page_shift);
    const int first = t_begin >> P.page_shift, npg = P.split_tokens >> P.page_shift;
    for (int i = tid; i < npg; i += kThreads) {
      const int pi = min(first + i, npg_seq - 1);
      const int pg = pi >= 0 ? P.indices[pbeg + pi] : 0;
      s_pg[i] = min(max(pg, 0), P.max_pages - 1);
    }
    rs.kc = make_rsrc(P.k_codes, P.pool_code_bytes);
    rs.vc = make_rsrc(P.v_codes, P.pool_code_bytes);
    rs.kn = make_rsrc(P.k_norms, P.pool_norm_bytes);
    rs.vn = make_rsrc(P.v_norms, P.pool_norm_bytes);
    __syncthreads();  // page ids
  } else {
    t_addr_end = min(t_begin + P.split_tokens, P.cap);
    seq_len = __builtin_amdgcn_readfirstlane(*P.seq_len);
    rs.kc = make_rsrc(P.k_codes + bh * static_cast<size_t>(P.cap) * RB, static_cast<uint32_t>(P.cap) * RB);
    rs.vc = make_rsrc(P.v_codes + bh * static_cast<size_t>(P.cap) * RB, static_cast<uint32_t>(P.cap) * RB);
    rs.kn = make_rsrc(P.k_norms + bh * static_cast<size_t>(P.cap), static_cast<uint32_t>(P.cap) * 4);
    rs.vn = make_rsrc(P.v_norms + bh * static_cast<size_t>(P.cap), static_cast<uint32_t>(P.cap) * 4);
  }
  auto fetch = [&](BlockRegs& R, int t) {
    if constexpr (PAGED)
      fetch_block<CB>(R, rs, t, t_addr_end, lane, prow);
    else
      fetch_block<CB>(R, rs, t, t_addr_end, lane, DenseRows{});
  };
  // The wave's first token block.  Dense layout: always the straight-line
  // full-block load, whatever t is: rows past the cold store read 0 through
  // the range-checked vector offset, and tokens at or past t_end are masked
  // by selects in attend_block, so no branch separates these loads from the
  // query's and the query's wait need not drain them.  Paged: page ids past
  // the split are not staged, so the load keeps its guard.
  auto fetch_first = [&](BlockRegs& R, int t) {
    if constexpr (PAGED) {
      if (t < t_addr_end) fetch(R, t);
    } else {
      load_full_checked<CB>(R, rs, __builtin_amdgcn_readfirstlane(t), lane);
    }
  };
  BlockRegs ra, rb;
  constexpr int kStep = kWaves * kBlk;  // tokens between a wave's consecutive blocks
  int t0 = t_begin + wave * kBlk;
  // The first token block is fetched right after the query's own loads are
  // issued: memory results retire in issue order, so the query rotation then
  // waits only for the (cached) rotation matrix and query, not for the first
  // codes from HBM, and the codes keep streaming in while it computes.
  float c_lo = 0.f, c_hi = 0.f;
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
    c_lo = P.centroids[min(tid & 15, cmax)];
    c_hi = P.centroids[min(tid >> 4, cmax)];
  }
  // B operand of the score MFMA: rotated query x scale*log2(e), head
  // h = lane%16, dims 32*(lane/16) + 8*kb + position (permuted with PERM).
  const int h = lane & 15, g = lane >> 4;
  u32x4 qa[4];
  {
    // rows h >= G read head G - 1 and are zeroed: unconditional loads
    float4 f[8];
    if constexpr (DECODE) {
      // The G query heads from the q|k|v partials: sums, fp16, RoPE at pos,
      // then the rotation below.  Thread pairs (head e / 64, dims e % 64 and
      // e % 64 + 64).  The last split block also publishes the RoPE'd query
      // (fp16, for the combine's hot-window scores) and puts the new key and
      // value into their ring slot; evict_kernel has already quantized the
      // token that slot held.
      __shared__ float s_q[16][kD];
      float4 pik[8][2];
      load_pik_operand(P.PiK, wave, lane, pik);  // in flight while the partials are summed
      const int pos = __builtin_amdgcn_readfirstlane(*P.pos);
      const uint16_t* cos_row = P.rope_cos + static_cast<size_t>(pos) * kD;
      const uint16_t* sin_row = P.rope_sin + static_cast<size_t>(pos) * kD;
      const bool writer = split == P.nsplit - 1;
      // this thread's first query element: its first kPre chunk partials (both
      // dims of the RoPE pair) from clamped, always valid addresses, ahead of
      // the codes; the rest of the chunks and elements are loaded after them
      constexpr int kPre = QPRE;
      float pre0[kPre], pre1[kPre];
      uint16_t rc0, rc1, rs0, rs1;  // its RoPE factors
      {
        const int e = min(tid, G * (kD / 2) - 1);
        const int dd = e % (kD / 2);
        rc0 = cos_row[dd];
        rc1 = cos_row[dd + kD / 2];
        rs0 = sin_row[dd];
        rs1 = sin_row[dd + kD / 2];
        const int col = (kvh * G + e / (kD / 2)) * kD + dd;
        const float* p0 = P.pq + static_cast<size_t>(col / kGemvBN) * P.nchunk * kGemvBN + (col % kGemvBN);
        const float* p1 = P.pq + static_cast<size_t>((col + kD / 2) / kGemvBN) * P.nchunk * kGemvBN +
                          ((col + kD / 2) % kGemvBN);
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          const size_t o = static_cast<size_t>(min(i, P.nchunk - 1)) * kGemvBN;
          pre0[i] = p0[o];
          pre1[i] = p1[o];
        }
      }
      // the new key (threads 0..63, pair (t, t + 64)) and value (threads
      // 64..127) of the ring write, which only the last split block stores:
      // loaded by every block, without a branch, so that no path drains the
      // codes' loads before the query is ready
      float prk0[kPre], prk1[kPre];
      {
        const int t = tid & (kD - 1);
        const float* src = t < kD / 2 ? P.pk : P.pv;
        const int c0 = kvh * kD + (t & (kD / 2 - 1)), c1 = c0 + kD / 2;
        const float* p0 = src + static_cast<size_t>(c0 / kGemvBN) * P.nchunk * kGemvBN + (c0 % kGemvBN);
        const float* p1 = src + static_cast<size_t>(c1 / kGemvBN) * P.nchunk * kGemvBN + (c1 % kGemvBN);
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          const size_t o = static_cast<size_t>(min(i, P.nchunk - 1)) * kGemvBN;
          prk0[i] = p0[o];
          prk1[i] = p1[o];
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the codes' (results retire in order)
      fetch_first(ra, t0);
      for (int e = tid; e < G * (kD / 2); e += kThreads) {
        const int hh = e / (kD / 2), dd = e % (kD / 2);
        const int col = (kvh * G + hh) * kD + dd;
        float x0, x1, o0, o1;
        if (e == tid && P.nchunk <= kPre) {  // column_sum2's order: chunk order from 0
          x0 = 0.f;
          x1 = 0.f;
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
        if (writer) {
          P.q16[col] = f2h(o0);
          P.q16[col + kD / 2] = f2h(o1);
        }
      }
      if (writer) {
        const size_t slot = (static_cast<size_t>(kvh) * P.hot_cap + pos % P.hot_cap) * kD;
        float x0 = 0.f, x1 = 0.f;
        if (tid < kD) {  // column_sum2's order: chunk order from 0
          if (P.nchunk <= kPre) {
#pragma unroll
            for (int i = 0; i < kPre; ++i) {
              x0 += i < P.nchunk ? prk0[i] : 0.f;
              x1 += i < P.nchunk ? prk1[i] : 0.f;
            }
          } else {
            const int c0 = kvh * kD + (tid & (kD / 2 - 1));
            column_sum2(tid < kD / 2 ? P.pk : P.pv, c0, c0 + kD / 2, P.nchunk, x0, x1);
          }
        }
        if (tid < kD / 2) {  // key pair (tid, tid + 64), RoPE'd (the factors of query element tid)
          float o0, o1;
          if (P.nchunk <= kPre)
            rope_pair_v(x0, x1, rc0, rc1, rs0, rs1, o0, o1);
          else
            rope_pair(x0, x1, cos_row, sin_row, tid, o0, o1);
          P.k_ring[slot + tid] = f2h(o0);
          P.k_ring[slot + tid + kD / 2] = f2h(o1);
        } else if (tid < kD) {  // value dims (tid - 64, tid): no RoPE
          const int dd = tid - kD / 2;
          P.v_ring[slot + dd] = f2h(x0);
          P.v_ring[slot + dd + kD / 2] = f2h(x1);
        }
      }
      __syncthreads();
      LKV_SPLIT_STAMP(4);
      u32x4 qb = u32x4{0u, 0u, 0u, 0u};
      if (h < G) {
        const float* q = &s_q[h][32 * wave + 8 * g];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          qb[jj] = static_cast<uint32_t>(f2h(q[2 * jj])) | (static_cast<uint32_t>(f2h(q[2 * jj + 1])) << 16);
      }
      rotate_query_hilo_loaded(pik, qb, wave, lane, &s_o[0][0][0], kORow, f);
      __syncthreads();  // s_o is written again by the merge
      LKV_SPLIT_STAMP(5);
    } else if (P.PiK != nullptr) {
      // q_rot on MFMA (rotate_query_hilo), overlapping the first block's
      // loads; s_o is free until the merge.
      float4 pik[8][2];
      load_pik_operand(P.PiK, wave, lane, pik);
      u32x4 qb;
      {
        const uint4 u = *reinterpret_cast<const uint4*>(
            P.q + (static_cast<size_t>(b) * P.Hq + kvh * G + min(h, G - 1)) * kD + 32 * wave + 8 * g);
        qb = h < G ? u32x4{u.x, u.y, u.z, u.w} : u32x4{0u, 0u, 0u, 0u};
      }
      fetch_first(ra, t0);
      LKV_SPLIT_STAMP(4);
      rotate_query_hilo_loaded(pik, qb, wave, lane, &s_o[0][0][0], kORow, f);
      __syncthreads();  // s_o is written again by the merge
      LKV_SPLIT_STAMP(5);
    } else {
      const float4* src = reinterpret_cast<const float4*>(
          P.qrot + (static_cast<size_t>(b) * P.Hq + kvh * G + min(h, G - 1)) * kD + 32 * g);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = src[i];
      fetch_first(ra, t0);
    }
    if constexpr (!PERM) s_lut[tid] = pack2h(c_lo, c_hi);
    const float sl = P.scale_log2;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 f0 = f[2 * kb], f1 = f[2 * kb + 1];
      const float x[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = PERM ? kPermDim[2 * j] : 2 * j, d1 = PERM ? kPermDim[2 * j + 1] : 2 * j + 1;
        v[j] = pack2h(x[d0] * sl, x[d1] * sl);
      }
      qa[kb] = h < G ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int L = min(seq_len, P.max_len);
  const int cold_len = max(0, L - P.hot_cap);
  const int t_end = min(cold_len, t_addr_end);
  if (t_begin >= t_end) {  // uniform over the block: nothing of this split is cold yet
    if (tid < G) {
      rec[tid] = -INFINITY;
      rec[G + tid] = 0.f;
    }
    LKV_SPLIT_STAMP(1);
    LKV_SPLIT_STAMP(2);
    LKV_SPLIT_STAMP(3);
    return;
  }
  LKV_SPLIT_STAMP(1);

  SoftmaxState S;
  S.m = -INFINITY;
  S.l = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) S.o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (!PERM) __syncthreads();  // LUT ready
  // Two register sets in turn: the next block's loads are in flight while
  // the current one is computed, with no register copies between them.
  // (Loading both sets in the prologue measured 29.0 -> 29.5-30.1 us at
  // config 4 and +0.2 % at config 5: the loop is not waiting on the second
  // block's loads.)
  while (t0 < t_end) {
    const int t1 = t0 + kStep;
    if (t1 < t_end) fetch(rb, t1);
    attend<PERM>(ra, t0, t_end, qa, tab, s_lut, lane, S);
    if (t1 >= t_end) break;
    const int t2 = t1 + kStep;
    if (t2 < t_end) fetch(ra, t2);
    attend<PERM>(rb, t1, t_end, qa, tab, s_lut, lane, S);
    t0 = t2;
  }
  LKV_SPLIT_STAMP(2);

  // ---- merge the 4 waves of the block through LDS.  A wave that had no
  // block keeps m = -inf, l = 0, o = 0.
  const float lsum = xgroup_sum(S.l);
  if (g == 0) {
    s_m[wave][h] = S.m;
    s_l[wave][h] = lsum;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float4* dst = reinterpret_cast<float4*>(&s_o[wave][h][32 * g + 8 * i]);
    if constexpr (PERM) {  // dims 0..7 sit in tiles 0, 4, 1, 5, 2, 6, 3, 7
      dst[0] = make_float4(S.o[0][i], S.o[4][i], S.o[1][i], S.o[5][i]);
      dst[1] = make_float4(S.o[2][i], S.o[6][i], S.o[3][i], S.o[7][i]);
    } else {
      dst[0] = make_float4(S.o[0][i], S.o[1][i], S.o[2][i], S.o[3][i]);
      dst[1] = make_float4(S.o[4][i], S.o[5][i], S.o[6][i], S.o[7][i]);
    }
  }
  __syncthreads();
  for (int e = tid; e < G * kD; e += kThreads) {
    const int hh = e / kD, d = e % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][hh]);
    float acc = 0.f, ls = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = fast_exp2(s_m[w][hh] - M);
        acc += wt * s_o[w][hh][d];
        ls += wt * s_l[w][hh];
      }
    }
    rec[rec_acc_off(G) + hh * kD + d] = acc;
    if (d == 0) {
      rec[hh] = M;
      rec[G + hh] = ls;
    }
  }
  LKV_SPLIT_STAMP(3);
}


constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, one L2 each
constexpr int kCombThreads = 512;
constexpr int kCombWaves = kCombThreads / kWave;
constexpr int kMaxSplits = 256;

__device__ __forceinline__ float dot8_f16(const uint4& a, const uint4& b) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s = fmaf(h2f(static_cast<uint16_t>(x[i] & 0xffffu)), h2f(static_cast<uint16_t>(y[i] & 0xffffu)), s);
    s = fmaf(h2f(static_cast<uint16_t>(x[i] >> 16)), h2f(static_cast<uint16_t>(y[i] >> 16)), s);
  }
  return s;
}

// One block per (query head, batch), 512 threads.  Every load is issued up
// front and vectorised where the data is contiguous (the combine is bound by
// load instructions and latency, not bytes):
//   thread (dg = tid % 32, grp = tid / 32): PiV rows 8 grp .. 8 grp + 7 at
//   dims 4 dg .. 4 dg + 3 (float4), and the rotated sums of splits grp, grp +
//   16, ... at the same dims (float4);
//   thread (dh = tid % 16, jg = tid / 16): hot values of slots jg + 32 i
//   (i < 2 NHG) at dims 8 dh .. 8 dh + 7 (16-byte loads);
//   thread (j = tid / 8, part = tid % 8): the hot scores of slots j + 64 q
//   (q < NHG), dims 16 part .. 16 part + 15;  thread s < nsplit: split s's
//   maximum and sum.
// NHG: hot-window slot groups of 64 (hot_cap <= 64 NHG).  Partial sums over
// split groups, slot groups and PiV row groups are joined through LDS in a
// fixed order (for NHG = 1 the same order as any larger NHG on <= 64 slots).
constexpr int kCombSplitGroups = kCombThreads / 32;  // 16
constexpr int kCombSlotGroups = kCombThreads / 16;   // 32
template <int NHG>
__global__ __launch_bounds__(kCombThreads, 4) void tq_attn_combine_kernel(AttnParams P) {  // 2 blocks per CU
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_p[64 * NHG];
  __shared__ float s_red[kCombWaves];
  __shared__ __align__(16) float s_cold[kCombSplitGroups][kD];
  __shared__ __align__(16) float s_hot[kCombSlotGroups][kD];
  __shared__ __align__(16) float s_rot[kD];
  __shared__ float s_hv[kD];

  LKV_COMB_STAMP(0);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  // Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
  // own L2.  The G query heads of one (batch, kv head) read the same hot window
  // and split records, so the linear id is remapped to put them on one XCD:
  // XCD x = p % 8 runs logical blocks x * nb / 8 .. (x + 1) * nb / 8 - 1.
  int hq, b;
  {
    const int nb = static_cast<int>(gridDim.x * gridDim.y), p = static_cast<int>(blockIdx.x + blockIdx.y * gridDim.x);
    const int l = (nb % kXcds == 0) ? (p % kXcds) * (nb / kXcds) + p / kXcds : p;
    hq = l % static_cast<int>(gridDim.x);
    b = l / static_cast<int>(gridDim.x);
  }
  const int G = P.G, kvh = hq / G, hh = hq % G;
  const int ns = P.nsplit;
  const int seq_len = P.indptr ? P.seq_len[b] : *P.seq_len;  // only the masks below depend on it
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  const int RF = rec_floats(G);
  const float* recs = P.partials + bh * ns * RF;
  const size_t hot_base = bh * static_cast<size_t>(P.hot_cap) * kD;
  const int dg = tid & 31, grp = tid >> 5;  // PiV rows / split groups, 4 dims
  const int dh = tid & 15, jg = tid >> 4;   // hot value slot groups, 8 dims

  // ---- A. every load up front, from clamped, always valid addresses (split
  // ns - 1, slot hot_cap - 1), masked after.  The hot window is walked by ring
  // slot: slot j holds a current token exactly when j < hot_len.
  float ms, ls;
  {
    const size_t sr = static_cast<size_t>(min(tid, ns - 1)) * RF;
    const float m_ = recs[sr + hh], l_ = recs[sr + G + hh];
    ms = tid < ns ? m_ : -INFINITY;
    ls = tid < ns ? l_ : 0.f;
  }
  float4 pv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pv[i] = *reinterpret_cast<const float4*>(P.PiV + (8 * grp + i) * kD + 4 * dg);
  uint4 hv[2 * NHG];
#pragma unroll
  for (int i = 0; i < 2 * NHG; ++i) {
    const int jj = min(jg + 32 * i, P.hot_cap - 1);
    hv[i] = *reinterpret_cast<const uint4*>(P.v_hot + hot_base + static_cast<size_t>(jj) * kD + 8 * dh);
  }
  float4 ca = *reinterpret_cast<const float4*>(recs + static_cast<size_t>(min(grp, ns - 1)) * RF + rec_acc_off(G) + hh * kD +
                                              4 * dg);
  // hot score partials: slots j + 64 q, j = tid / 8, dims 16 * (tid % 8) .. +16
  const int j = tid >> 3, part = tid & 7;
  float sdot[NHG];
  {
    const uint4* qp = reinterpret_cast<const uint4*>(P.q + (static_cast<size_t>(b) * P.Hq + hq) * kD + 16 * part);
    const uint4 q0 = qp[0], q1 = qp[1];
    uint4 k0[NHG], k1[NHG];
#pragma unroll
    for (int q = 0; q < NHG; ++q) {
      const int slot = min(j + 64 * q, P.hot_cap - 1);
      const uint4* kp = reinterpret_cast<const uint4*>(P.k_hot + hot_base + static_cast<size_t>(slot) * kD + 16 * part);
      k0[q] = kp[0];
      k1[q] = kp[1];
    }
#pragma unroll
    for (int q = 0; q < NHG; ++q) sdot[q] = dot8_f16(k0[q], q0) + dot8_f16(k1[q], q1);  // masked by `score`
  }
  const int L = min(seq_len, P.max_len);
  const int hot_len = L - max(0, L - P.hot_cap);
  // ---- B. softmax statistics over cold splits and hot tokens
  float score[NHG];
  float smax = -INFINITY;
#pragma unroll
  for (int q = 0; q < NHG; ++q) {
    float d = sdot[q];
    d += dpp_f<0xB1>(d);   // xor 1
    d += dpp_f<0x4E>(d);   // xor 2
    d += dpp_f<0x141>(d);  // the other quad of the 8-lane half row
    score[q] = j + 64 * q < hot_len ? d * P.scale_log2 : -INFINITY;
    smax = fmaxf(smax, score[q]);
  }
  float v = fmaxf(ms, part == 0 ? smax : -INFINITY);
  v = wave_max(v);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kCombWaves; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const float wsp = (tid < ns && ms != -INFINITY) ? fast_exp2(ms - M) : 0.f;
  if (tid < ns) s_w[tid] = wsp;
  float psum = 0.f;
#pragma unroll
  for (int q = 0; q < NHG; ++q) {
    const float pj = j + 64 * q < hot_len ? fast_exp2(score[q] - M) : 0.f;
    if (part == 0) s_p[j + 64 * q] = pj;
    psum += pj;
  }
  float lv = wsp * ls + (part == 0 ? psum : 0.f);
  lv = wave_sum(lv);
  if (lane == 0) s_red[wave] = lv;
  __syncthreads();
  float Lt = 0.f;
#pragma unroll
  for (int w = 0; w < kCombWaves; ++w) Lt += s_red[w];

  // ---- C. partial sums: rotated cold sum of this split group (4 dims), hot
  // value sum of this slot group (8 dims)
  float4 cold = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += kCombSplitGroups) {
    const int sp = s0 + grp;
    if (s0 > 0)
      ca = *reinterpret_cast<const float4*>(recs + static_cast<size_t>(min(sp, ns - 1)) * RF + rec_acc_off(G) + hh * kD +
                                            4 * dg);
    const float w = sp < ns ? s_w[sp] : 0.f;
    if (w != 0.f) {  // an empty split's sums were never written: select, do not multiply
      cold.x = fmaf(w, ca.x, cold.x);
      cold.y = fmaf(w, ca.y, cold.y);
      cold.z = fmaf(w, ca.z, cold.z);
      cold.w = fmaf(w, ca.w, cold.w);
    }
  }
  *reinterpret_cast<float4*>(&s_cold[grp][4 * dg]) = cold;
  float hs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 2 * NHG; ++i) {
    const int jj = jg + 32 * i;
    if (jj < hot_len) {  // an unwritten slot may hold NaN: skipped, never multiplied
      const float p = s_p[jj];
      const uint32_t w4[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hs[2 * e] = fmaf(p, h2f(static_cast<uint16_t>(w4[e] & 0xffffu)), hs[2 * e]);
        hs[2 * e + 1] = fmaf(p, h2f(static_cast<uint16_t>(w4[e] >> 16)), hs[2 * e + 1]);
      }
    }
  }
  *reinterpret_cast<float4*>(&s_hot[jg][8 * dh]) = make_float4(hs[0], hs[1], hs[2], hs[3]);
  *reinterpret_cast<float4*>(&s_hot[jg][8 * dh + 4]) = make_float4(hs[4], hs[5], hs[6], hs[7]);
  __syncthreads();
  if (tid < kD) {
    float c = 0.f, h = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < kCombSplitGroups; ++g2) c += s_cold[g2][tid];
#pragma unroll
    for (int g2 = 0; g2 < kCombSlotGroups; ++g2) h += s_hot[g2][tid];
    s_rot[tid] = c;
    s_hv[tid] = h;
  }
  __syncthreads();

  // ---- D. un-rotate the cold sum: out[d] = sum_k rot[k] PiV[k][d], this
  // thread's 8 rows for its 4 dims, then the 16 row groups in order
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float r = s_rot[8 * grp + i];
    o.x = fmaf(r, pv[i].x, o.x);
    o.y = fmaf(r, pv[i].y, o.y);
    o.z = fmaf(r, pv[i].z, o.z);
    o.w = fmaf(r, pv[i].w, o.w);
  }
  *reinterpret_cast<float4*>(&s_cold[grp][4 * dg]) = o;  // s_cold is free again
  __syncthreads();
  if (tid < kD) {
    float r = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < kCombSplitGroups; ++g2) r += s_cold[g2][tid];
    r += s_hv[tid];
    P.out[(static_cast<size_t>(b) * P.Hq + hq) * kD + tid] = f2h(Lt > 0.f ? r / Lt : 0.f);
  }
  LKV_COMB_STAMP(3);
}

constexpr int kSplitGran = kWaves * kBlk;  // tokens one pass of a block covers

// Split count that gives ~4 blocks per CU (each wave's token loop is a
// latency chain, so more resident waves overlap more of them), at most
// kMaxSplits - 1.
// Tuning knobs, read once.  LKV_ATTN_SPLIT_TARGET=k: aim for k split blocks
// per CU (default: the resident count, kSplitBlocksPerCU).  LKV_ATTN_QROT=kernel:
// lkv_tq_decode_attn rotates the query in its own launch instead of in every
// split block's prologue.
int attn_split_target() {
  static const int k = [] {
    const char* env = getenv("LKV_ATTN_SPLIT_TARGET");
    const int v = env ? atoi(env) : 0;
    return v > 0 && v <= 16 ? v : kSplitBlocksPerCU;
  }();
  return k;
}
// At least 256 cold tokens per split (two passes of a block): at B = 1 the
// target split count would give 128-token splits, and each split block repeats
// the query prologue (q partial sums, RoPE, the rotation with PiK); 256 measured
// 392 vs 384 tok/s at config 5 (512: 383, 1024: 365).  B >= 4 already gets
// longer splits.  LKV_ATTN_MIN_SPLIT_TOKENS=n overrides (0: none).
int64_t attn_min_split_tokens() {
  static const int64_t k = [] {
    const char* env = getenv("LKV_ATTN_MIN_SPLIT_TOKENS");
    const long v = env ? atol(env) : 256;
    return static_cast<int64_t>(v > 0 && v <= (1 << 20) ? v : 0);
  }();
  return k;
}
bool attn_qrot_kernel() {
  static const bool k = [] {
    const char* env = getenv("LKV_ATTN_QROT");
    return env && env[0] == 'k';
  }();
  return k;
}

// q_rot = q @ PiK^T in a launch of its own: one 4-wave block per (kv head, batch).
__global__ __launch_bounds__(kThreads) void qrot_hilo_kernel(const uint16_t* __restrict__ q,
                                                             const float* __restrict__ PiK, float* __restrict__ qrot,
                                                             int Hq, int Hkv) {
  __shared__ __align__(16) float s_part[4 * 16 * kORow];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kvh = blockIdx.x, b = blockIdx.y, G = Hq / Hkv;
  const int h = lane & 15, g = lane >> 4;
  const uint4 u = *reinterpret_cast<const uint4*>(q + (static_cast<size_t>(b) * Hq + kvh * G + min(h, G - 1)) * kD +
                                                  32 * wave + 8 * g);
  const u32x4 qb = h < G ? u32x4{u.x, u.y, u.z, u.w} : u32x4{0u, 0u, 0u, 0u};
  float4 out[8];
  rotate_query_hilo(PiK, qb, wave, lane, s_part, kORow, out);
  if (h < G && wave == 0) {
    float4* dst = reinterpret_cast<float4*>(qrot + (static_cast<size_t>(b) * Hq + kvh * G + h) * kD + 32 * g);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = out[i];
  }
}

int64_t target_splits(int64_t B, int64_t Hkv) {
  const int64_t target = attn_split_target() * static_cast<int64_t>(device_cu_count());
  int64_t ns = (target + B * Hkv - 1) / (B * Hkv);
  if (ns > kMaxSplits - 1) ns = kMaxSplits - 1;
  return ns < 1 ? 1 : ns;
}

}  // namespace

AttnPlan attn_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t hot_cap, int64_t max_split_tokens) {
  AttnPlan p{};
  const int64_t G = Hkv > 0 ? Hq / Hkv : 1;
  const int64_t cold_max = max_len > hot_cap ? max_len - hot_cap : 0;
  int64_t ns_cap = target_splits(B, Hkv);
  int64_t ts = (cold_max + ns_cap - 1) / ns_cap;
  if (ts < attn_min_split_tokens()) ts = attn_min_split_tokens();
  ts = (ts + kSplitGran - 1) / kSplitGran * kSplitGran;
  if (ts < kSplitGran) ts = kSplitGran;
  if (max_split_tokens > 0 && ts > max_split_tokens) ts = max_split_tokens / kSplitGran * kSplitGran;
  int64_t ns = (cold_max + ts - 1) / ts;
  if (ns > ns_cap) ns_cap = ns;
  if (ns < 1) ns = 1;
  p.nsplit = static_cast<int>(ns);
  p.split_tokens = static_cast<int>(ts);
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  p.qrot_off = kTicketBytes;  // keeps the shared workspace layout: ticket area first
  p.part_off = p.qrot_off + al(static_cast<size_t>(B * Hq * kD) * 4);
  // sized for ns_cap so a workspace sized without hot_cap fits every call
  p.total = p.part_off + al(static_cast<size_t>(B * Hkv * ns_cap) * rec_floats(static_cast<int>(G)) * 4);
  return p;
}

int attn_launch(const AttnCall& c, const AttnPlan& pl, hipStream_t st) {
  AttnParams P;
  P.qrot = c.qrot;
  P.q = c.q;
  P.k_codes = c.k_codes;
  P.k_norms = c.k_norms;
  P.v_codes = c.v_codes;
  P.v_norms = c.v_norms;
  P.k_hot = c.k_hot;
  P.v_hot = c.v_hot;
  P.PiV = c.PiV;
  P.PiK = c.PiK;
  P.centroids = c.centroids;
  P.seq_len = c.seq_len;
  P.partials = c.partials;
  P.out = c.out;
  P.scale_log2 = c.scale * kLog2e;
  P.max_len = static_cast<int>(c.max_len);
  P.Hq = static_cast<int>(c.Hq);
  P.Hkv = static_cast<int>(c.Hkv);
  P.G = static_cast<int>(c.Hq / c.Hkv);
  P.cap = static_cast<int>(c.cap);
  P.hot_cap = static_cast<int>(c.hot_cap);
  P.nsplit = pl.nsplit;
  P.split_tokens = pl.split_tokens;
  P.ncent = 1 << c.bits;
  const dim3 grid(static_cast<unsigned>(pl.nsplit), static_cast<unsigned>(c.Hkv), static_cast<unsigned>(c.B));
  const dim3 cgrid(static_cast<unsigned>(c.Hq), static_cast<unsigned>(c.B));
  P.pq = c.pq;
  P.pk = c.pk;
  P.pv = c.pv;
  P.nchunk = c.nchunk;
  P.rope_cos = c.rope_cos;
  P.rope_sin = c.rope_sin;
  P.pos = c.pos;
  P.q16 = c.q16;
  P.k_ring = c.k_ring;
  P.v_ring = c.v_ring;
  P.indptr = c.indptr;
  P.indices = c.indices;
  P.page_shift = c.page_shift;
  P.max_pages = static_cast<int>(c.max_pages);
  P.pool_code_bytes = static_cast<uint32_t>(c.max_pages * c.Hkv * (int64_t(1) << c.page_shift) * tq::row_bytes_for(c.bits));
  P.pool_norm_bytes = static_cast<uint32_t>(c.max_pages * c.Hkv * (int64_t(1) << c.page_shift) * 4);
  if (c.pq != nullptr) {
    P.q = c.q16;  // the combine's hot-window query
    P.k_hot = c.k_ring;
    P.v_hot = c.v_ring;
    // the fewest partial loads ahead of the codes that still cover every chunk
    const bool pre8 = c.nchunk <= 8;
    switch (c.bits) {
      case 1:
        if (pre8)
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 1, 8>), grid, dim3(kThreads), 0, st, P);
        else
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 1, 16>), grid, dim3(kThreads), 0, st, P);
        break;
      case 2:
        if (pre8)
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 2, 8>), grid, dim3(kThreads), 0, st, P);
        else
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 2, 16>), grid, dim3(kThreads), 0, st, P);
        break;
      case 3:
        if (pre8)
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 4, 8>), grid, dim3(kThreads), 0, st, P);
        else
          hipLaunchKernelGGL((tq_attn_split_kernel<true, true, false, 4, 16>), grid, dim3(kThreads), 0, st, P);
        break;
      default:
        if (pre8)
          hipLaunchKernelGGL((tq_attn_split_kernel<false, true, false, 4, 8>), grid, dim3(kThreads), 0, st, P);
        else
          hipLaunchKernelGGL((tq_attn_split_kernel<false, true, false, 4, 16>), grid, dim3(kThreads), 0, st, P);
    }
  } else if (c.indptr != nullptr) {
    switch (c.bits) {
      case 1: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, true, 1>), grid, dim3(kThreads), 0, st, P); break;
      case 2: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, true, 2>), grid, dim3(kThreads), 0, st, P); break;
      case 3: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, true, 4>), grid, dim3(kThreads), 0, st, P); break;
      default: hipLaunchKernelGGL((tq_attn_split_kernel<false, false, true, 4>), grid, dim3(kThreads), 0, st, P);
    }
  } else {
    switch (c.bits) {
      case 1: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, false, 1>), grid, dim3(kThreads), 0, st, P); break;
      case 2: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, false, 2>), grid, dim3(kThreads), 0, st, P); break;
      case 3: hipLaunchKernelGGL((tq_attn_split_kernel<true, false, false, 4>), grid, dim3(kThreads), 0, st, P); break;
      default: hipLaunchKernelGGL((tq_attn_split_kernel<false, false, false, 4>), grid, dim3(kThreads), 0, st, P);
    }
  }
  LKV_LAUNCH_CHECK("tq_decode_attn split");
  if (c.hot_cap <= 64)
    hipLaunchKernelGGL(tq_attn_combine_kernel<1>, cgrid, dim3(kCombThreads), 0, st, P);
  else if (c.hot_cap <= 128)
    hipLaunchKernelGGL(tq_attn_combine_kernel<2>, cgrid, dim3(kCombThreads), 0, st, P);
  else
    hipLaunchKernelGGL(tq_attn_combine_kernel<4>, cgrid, dim3(kCombThreads), 0, st, P);
  LKV_LAUNCH_CHECK("tq_decode_attn combine");
  return LKV_OK;
}

}  // namespace lkv

using namespace lkv;

#ifdef LKV_STAMPS
// Instrumented build only: copy the phase stamps of the last split (which = 0)
// or combine (which = 1) launches to host memory, n <= 8 * 16384 words;
// clear = 1 zeroes them instead.  Not declared in the public header.
extern "C" int lkv_debug_stamps(int which, uint64_t* host, int64_t n, int clear) {
  LKV_REQUIRE(n >= 0 && n <= kStampSlots * kStampBlocks && (clear || host), "debug_stamps: bad buffer");
  hipError_t e;
  if (clear) {
    static uint64_t zeros[kStampSlots * kStampBlocks];
    e = which ? hipMemcpyToSymbol(HIP_SYMBOL(g_comb_stamps), zeros, sizeof(zeros))
              : hipMemcpyToSymbol(HIP_SYMBOL(g_split_stamps), zeros, sizeof(zeros));
  } else {
    e = which ? hipMemcpyFromSymbol(host, HIP_SYMBOL(g_comb_stamps), static_cast<size_t>(n) * 8)
              : hipMemcpyFromSymbol(host, HIP_SYMBOL(g_split_stamps), static_cast<size_t>(n) * 8);
  }
  LKV_REQUIRE(e == hipSuccess, "debug_stamps: %s", hipGetErrorString(e));
  return LKV_OK;
}
#endif

extern "C" size_t lkv_tq_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len < 0) return kTicketBytes;
  // hot_cap only shifts the cold range; the record area is sized for the cap.
  return attn_plan(B, Hq, Hkv, max_len, 0).total;
}

extern "C" int lkv_tq_decode_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                                  const uint8_t* v_codes, const float* v_norms, const void* k_hot,
                                  const void* v_hot, const float* PiK, const float* PiV,
                                  const float* centroids, int bits, const int32_t* seq_len,
                                  int64_t max_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap,
                                  int64_t hot_cap, float scale, void* out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  LKV_REQUIRE(bits >= 1 && bits <= 4, "tq_decode_attn: bits=%d unsupported (1..4 are bit-packed)", bits);
  LKV_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16,
              "tq_decode_attn: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%lld Hkv=%lld)", (long long)Hq,
              (long long)Hkv);
  LKV_REQUIRE(hot_cap >= 1 && hot_cap <= kHotMax, "tq_decode_attn: hot_cap must be 1..%d", kHotMax);
  LKV_REQUIRE(max_len >= 0 && max_len <= cap + hot_cap, "tq_decode_attn: max_len=%lld exceeds cap+hot_cap=%lld",
              (long long)max_len, (long long)(cap + hot_cap));
  LKV_REQUIRE(max_len < (1ll << 31) && cap < (1ll << 31), "tq_decode_attn: length too large");
  if (B == 0) return LKV_OK;
  LKV_REQUIRE(q && k_codes && k_norms && v_codes && v_norms && k_hot && v_hot && PiK && PiV && centroids &&
                  seq_len && out && workspace,
              "tq_decode_attn: null pointer");
  LKV_REQUIRE(aligned16(q) && aligned16(k_codes) && aligned16(v_codes) && aligned16(k_hot) && aligned16(v_hot) &&
                  aligned16(PiK) && aligned16(PiV) && aligned16(out) && aligned16(workspace),
              "tq_decode_attn: q, codes, hot, PiK, PiV, out and workspace must be 16-byte aligned");
  const AttnPlan pl = attn_plan(B, Hq, Hkv, max_len, hot_cap);
  LKV_REQUIRE(workspace_bytes >= pl.total, "tq_decode_attn: workspace of %zu bytes required, got %zu", pl.total,
              workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  AttnCall c{};
  if (attn_qrot_kernel()) {
    float* qr = reinterpret_cast<float*>(ws + pl.qrot_off);
    hipLaunchKernelGGL(qrot_hilo_kernel, dim3(static_cast<unsigned>(Hkv), static_cast<unsigned>(B)), dim3(kThreads), 0,
                       st, static_cast<const uint16_t*>(q), PiK, qr, static_cast<int>(Hq), static_cast<int>(Hkv));
    LKV_LAUNCH_CHECK("tq_decode_attn q rotation");
    c.qrot = qr;
    c.PiK = nullptr;
  } else {
    c.qrot = nullptr;
    c.PiK = PiK;  // the split kernel rotates the query
  }
  c.q = static_cast<const uint16_t*>(q);
  c.k_codes = k_codes;
  c.k_norms = k_norms;
  c.v_codes = v_codes;
  c.v_norms = v_norms;
  c.k_hot = static_cast<const uint16_t*>(k_hot);
  c.v_hot = static_cast<const uint16_t*>(v_hot);
  c.PiV = PiV;
  c.centroids = centroids;
  c.seq_len = seq_len;
  c.partials = reinterpret_cast<float*>(ws + pl.part_off);
  c.out = static_cast<uint16_t*>(out);
  c.scale = scale;
  c.max_len = max_len;
  c.B = B;
  c.Hq = Hq;
  c.Hkv = Hkv;
  c.cap = cap;
  c.hot_cap = hot_cap;
  c.bits = bits;
  return attn_launch(c, pl, st);
}

// ------------------------------------------------------------ paged cold store
namespace {
int page_shift_of(int64_t page_size) {
  for (int sh = 4; sh <= 7; ++sh)
    if (page_size == (int64_t(1) << sh)) return sh;
  return -1;
}
AttnPlan paged_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t hot_cap, int64_t page_size) {
  return attn_plan(B, Hq, Hkv, max_len, hot_cap, int64_t(kMaxPg) * page_size);
}
}  // namespace

extern "C" size_t lkv_tq_paged_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len,
                                                           int64_t page_size) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len < 0 || page_shift_of(page_size) < 0) return kTicketBytes;
  return paged_plan(B, Hq, Hkv, max_len, 0, page_size).total;
}

extern "C" int lkv_tq_paged_decode_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                                        const uint8_t* v_codes, const float* v_norms, const void* k_hot,
                                        const void* v_hot, const float* PiK, const float* PiV, const float* centroids,
                                        int bits, const int32_t* kv_indptr, const int32_t* kv_indices,
                                        const int32_t* seq_lens, int64_t B, int64_t Hq, int64_t Hkv,
                                        int64_t page_size, int64_t max_pages, int64_t max_len, int64_t hot_cap,
                                        float scale, void* out, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  LKV_REQUIRE(bits >= 1 && bits <= 4, "tq_paged_decode_attn: bits=%d unsupported (1..4 are bit-packed)", bits);
  LKV_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16,
              "tq_paged_decode_attn: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%lld Hkv=%lld)", (long long)Hq,
              (long long)Hkv);
  const int shift = page_shift_of(page_size);
  LKV_REQUIRE(shift >= 0, "tq_paged_decode_attn: page_size=%lld must be 16, 32, 64 or 128", (long long)page_size);
  LKV_REQUIRE(hot_cap >= 1 && hot_cap <= kHotMax, "tq_paged_decode_attn: hot_cap must be 1..%d", kHotMax);
  LKV_REQUIRE(max_pages >= 1 && max_pages * Hkv * page_size * tq::row_bytes_for(bits) < (int64_t(1) << 32),
              "tq_paged_decode_attn: max_pages=%lld: the code pool must hold fewer than 2^32 bytes",
              (long long)max_pages);
  LKV_REQUIRE(max_len >= 0 && max_len < (1ll << 31), "tq_paged_decode_attn: bad max_len");
  if (B == 0) return LKV_OK;
  LKV_REQUIRE(q && k_codes && k_norms && v_codes && v_norms && k_hot && v_hot && PiK && PiV && centroids &&
                  kv_indptr && kv_indices && seq_lens && out && workspace,
              "tq_paged_decode_attn: null pointer");
  LKV_REQUIRE(aligned16(q) && aligned16(k_codes) && aligned16(v_codes) && aligned16(k_norms) &&
                  aligned16(v_norms) && aligned16(k_hot) && aligned16(v_hot) && aligned16(PiK) && aligned16(PiV) &&
                  aligned16(out) && aligned16(workspace),
              "tq_paged_decode_attn: q, pools, hot rings, PiK, PiV, out and workspace must be 16-byte aligned");
  const AttnPlan pl = paged_plan(B, Hq, Hkv, max_len, hot_cap, page_size);
  LKV_REQUIRE(pl.nsplit <= kMaxSplits - 1, "tq_paged_decode_attn: max_len=%lld needs %d splits (at most %d)",
              (long long)max_len, pl.nsplit, kMaxSplits - 1);
  LKV_REQUIRE(workspace_bytes >= pl.total, "tq_paged_decode_attn: workspace of %zu bytes required, got %zu",
              pl.total, workspace_bytes);
  AttnCall c{};
  c.qrot = nullptr;
  c.PiK = PiK;
  c.q = static_cast<const uint16_t*>(q);
  c.k_codes = k_codes;
  c.k_norms = k_norms;
  c.v_codes = v_codes;
  c.v_norms = v_norms;
  c.k_hot = static_cast<const uint16_t*>(k_hot);
  c.v_hot = static_cast<const uint16_t*>(v_hot);
  c.PiV = PiV;
  c.centroids = centroids;
  c.seq_len = seq_lens;
  c.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.part_off);
  c.out = static_cast<uint16_t*>(out);
  c.scale = scale;
  c.max_len = max_len;
  c.B = B;
  c.Hq = Hq;
  c.Hkv = Hkv;
  c.cap = 0;
  c.hot_cap = hot_cap;
  c.bits = bits;
  c.indptr = kv_indptr;
  c.indices = kv_indices;
  c.page_shift = shift;
  c.max_pages = max_pages;
  return attn_launch(c, pl, static_cast<hipStream_t>(stream));
}
