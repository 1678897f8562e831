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
//   1. q_rot = q @ PiK^T on fp32 MFMA, one block per (batch, kv head)
//      (the decode step computes it inside its QKV epilogue instead);
//   2. split kernel, grid splits x kv_heads x batch, 4 waves per block, each
//      block owning a contiguous range of cold tokens; each wave walks
//      32-token blocks of it, prefetching the next block's codes and norms
//      while it computes the current one:
//      * scores: v_mfma_f32_16x16x32_f16 with A = rotated query rows (the G
//        heads sharing this kv head, zero padded to 16) and B = 16 tokens x 32
//        dims of centroid values.  A lane loads 16 contiguous code bytes of
//        one token and unpacks them in registers through a 256-entry LDS
//        table that maps one code byte to the fp16 pair (c[lo], c[hi]);
//      * online softmax in the exp2 domain per head;
//      * values: the same MFMA with A = p * n_t (fp16, via a 1 KB LDS tile)
//        and B = 32 tokens x 16 dims of centroid values; a lane loads one code
//        dword (8 dims) of 8 tokens and transposes the fp16 pairs in registers;
//      * the block writes (m, l, acc[G][128]) per head to the workspace;
//   3. combine kernel, one block of 8 waves per (batch, query head): issues
//      every load it needs at once (split maxima and sums, the rotated
//      partial sums, the fp16 hot window and the PiV column slice), then
//      computes the hot scores, merges hot and cold softmax statistics,
//      applies PiV to the cold sum, adds the hot sum, normalises, writes fp16.
#include "kernels.h"
#include "tq_common.h"

namespace lkv {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kBlk = 32;    // tokens per wave step
constexpr int kRowB = 64;   // code bytes per token (4-bit nibbles, dim 128)
constexpr int kHotMax = 64;
constexpr float kLog2e = 1.4426950408889634f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half8 as_half8(const u32x4& v) { return __builtin_bit_cast(half8, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a), as_half8(b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack2h(float lo, float hi) {
  return static_cast<uint32_t>(f2h(lo)) | (static_cast<uint32_t>(f2h(hi)) << 16);
}

// Max / sum across the 16 lanes of a row group (lanes with equal lane/16).
__device__ __forceinline__ float group16_max(float v) { return row16_max(v); }
__device__ __forceinline__ float group16_sum(float v) { return row16_sum(v); }

// 2^x on the hardware exp (v_exp_f32); arguments here are <= 0 and results
// below 2^-126 flush to 0, which only drops contributions < 1e-38 of the max.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
  const float* centroids;   // [2^bits]
  const int32_t* seq_len;
  float* partials;          // [B, Hkv, nsplit, rec]
  uint16_t* out;            // [B, Hq, 128]
  float scale_log2;         // scale * log2(e)
  int max_len, Hq, Hkv, G, cap, hot_cap, nsplit, split_tokens, ncent;
};

__device__ __forceinline__ int rec_floats(int G) { return G * (2 + kD); }

// Code bytes / norms of the two 16-token score tiles and the 8 value tokens
// one lane needs for a 32-token block starting at t0.
struct BlockRegs {
  u32x4 kraw[2];
  float knorm[2];
  uint32_t vdw[8];
  float vnorm[2];
};

// Code bytes / norms of a 32-token block starting at t0, read without any
// condition: tokens at or past t_addr_end read token t_addr_end - 1 (valid
// memory), so every load issues back to back; mask_block zeroes the tokens at
// or past the valid end once it is known.
__device__ __forceinline__ void load_block(BlockRegs& R, int t0, int t_addr_end, int lane, const uint8_t* kc,
                                           const float* kn, const uint8_t* vc, const float* vn) {
  const int g = lane >> 4, w = lane & 15;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tok = min(t0 + 16 * tt + (lane & 15), t_addr_end - 1);
    R.kraw[tt] = *reinterpret_cast<const u32x4*>(kc + static_cast<size_t>(tok) * kRowB + 16 * g);
    R.knorm[tt] = kn[tok];
    R.vnorm[tt] = vn[tok];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int tok = min(t0 + 8 * g + i, t_addr_end - 1);
    R.vdw[i] = *reinterpret_cast<const uint32_t*>(vc + static_cast<size_t>(tok) * kRowB + 4 * w);
  }
}

__device__ __forceinline__ void mask_block(BlockRegs& R, int t0, int t_end, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const bool ok = t0 + 16 * tt + (lane & 15) < t_end;
    R.kraw[tt] = ok ? R.kraw[tt] : u32x4{0u, 0u, 0u, 0u};
    R.knorm[tt] = ok ? R.knorm[tt] : 0.f;
    R.vnorm[tt] = ok ? R.vnorm[tt] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) R.vdw[i] = t0 + 8 * g + i < t_end ? R.vdw[i] : 0u;
}

template <int GMAX>
__global__ __launch_bounds__(kThreads, 4) void tq_attn_split_kernel(AttnParams P) {
  __shared__ uint32_t s_lut[256];
  __shared__ __align__(16) uint16_t s_p[kWaves][16][kBlk];  // p * n_t, fp16, per wave
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  __shared__ __align__(16) float s_o[kWaves][16][kD];  // all 16 MFMA rows: rows >= G hold zeros

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = P.G;
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  float* rec = P.partials + (bh * P.nsplit + split) * rec_floats(G);

  // The split's token range is static; the current length only masks it.
  // So the length load, the wave's first token block, the centroid pairs of
  // the LUT and the rotated query are all in flight before the first wait.
  const int t_begin = split * P.split_tokens;
  const int t_addr_end = min(t_begin + P.split_tokens, P.cap);  // valid memory
  const int seq_len = *P.seq_len;
  const uint8_t* kc = P.k_codes + bh * static_cast<size_t>(P.cap) * kRowB;
  const uint8_t* vc = P.v_codes + bh * static_cast<size_t>(P.cap) * kRowB;
  const float* kn = P.k_norms + bh * static_cast<size_t>(P.cap);
  const float* vn = P.v_norms + bh * static_cast<size_t>(P.cap);
  BlockRegs cur;
  int t0 = t_begin + wave * kBlk;
  if (t_begin < t_addr_end) load_block(cur, t0, t_addr_end, lane, kc, kn, vc, vn);
  float c_lo, c_hi;
  {
    const int cmax = P.ncent - 1;
    c_lo = P.centroids[min(tid & 15, cmax)];
    c_hi = P.centroids[min(tid >> 4, cmax)];
  }
  // A operand of the score MFMA: rotated query x scale*log2(e), head
  // h = lane%16, dims 32*(lane/16) + 8*kb + i for k-block kb.
  const int h = lane & 15, g = lane >> 4;
  u32x4 qa[4];
  {
    // rows h >= G read head G - 1 and are zeroed: unconditional loads
    const float4* src = reinterpret_cast<const float4*>(
        P.qrot + (static_cast<size_t>(b) * P.Hq + kvh * G + min(h, G - 1)) * kD + 32 * g);
    float4 f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = src[i];
    s_lut[tid] = pack2h(c_lo, c_hi);
    const float sl = P.scale_log2;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 f0 = f[2 * kb], f1 = f[2 * kb + 1];
      qa[kb] = h < G ? u32x4{pack2h(f0.x * sl, f0.y * sl), pack2h(f0.z * sl, f0.w * sl), pack2h(f1.x * sl, f1.y * sl),
                             pack2h(f1.z * sl, f1.w * sl)}
                     : u32x4{0u, 0u, 0u, 0u};
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
    return;
  }
  mask_block(cur, t0, t_end, lane);

  float m[4], l[4];
  f32x4 o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // LUT ready
  for (; t0 < t_end; t0 += kWaves * kBlk) {
    const int tn = t0 + kWaves * kBlk;
    BlockRegs nxt;
    if (tn < t_end) {
      load_block(nxt, tn, t_end, lane, kc, kn, vc, vn);
      mask_block(nxt, tn, t_end, lane);
    }
    // ---- scores for tokens t0 .. t0+31 (two 16-token MFMA tiles)
    f32x4 sc[2];
    bool valid[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      valid[tt] = t0 + 16 * tt + (lane & 15) < t_end;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint32_t w = cur.kraw[tt][kb];
        const u32x4 bop = u32x4{s_lut[w & 0xffu], s_lut[(w >> 8) & 0xffu], s_lut[(w >> 16) & 0xffu], s_lut[w >> 24]};
        acc = mfma16x16x32(qa[kb], bop, acc);
      }
      sc[tt] = acc;
    }
    // ---- online softmax (log2 domain); lane holds heads 4g+i, token lane%16
    float p[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s0 = valid[0] ? sc[0][i] * cur.knorm[0] : -INFINITY;
      const float s1 = valid[1] ? sc[1][i] * cur.knorm[1] : -INFINITY;
      const float bmax = group16_max(fmaxf(s0, s1));
      const float mnew = fmaxf(m[i], bmax);
      // Branch-free: while nothing is valid (mnew = -inf) exp2(-inf - 0) = 0
      // keeps l, o and p at 0.
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = fast_exp2(m[i] - mref);
      const float p0 = valid[0] ? fast_exp2(s0 - mref) : 0.f;
      const float p1 = valid[1] ? fast_exp2(s1 - mref) : 0.f;
      l[i] = l[i] * alpha + group16_sum(p0 + p1);
      m[i] = mnew;
#pragma unroll
      for (int t = 0; t < 8; ++t) o[t][i] *= alpha;
      p[0][i] = p0;
      p[1][i] = p1;
    }
    // ---- p * n_t into the per-wave LDS tile [head][token]
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s_p[wave][4 * g + i][16 * tt + (lane & 15)] = f2h(valid[tt] ? p[tt][i] * cur.vnorm[tt] : 0.f);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // ---- P V: A = p*n (head h = lane%16, tokens 8g..8g+7), B = codes
    u32x4 pa = u32x4{0u, 0u, 0u, 0u};
    if (h < G) pa = *reinterpret_cast<const u32x4*>(&s_p[wave][h][8 * g]);
    uint32_t r[8][4];  // r[token i][byte bb] = (c[dim 8w+2bb], c[dim 8w+2bb+1])
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t dw = cur.vdw[i];
      r[i][0] = s_lut[dw & 0xffu];
      r[i][1] = s_lut[(dw >> 8) & 0xffu];
      r[i][2] = s_lut[(dw >> 16) & 0xffu];
      r[i][3] = s_lut[dw >> 24];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // dword pp = (token 2pp, token 2pp+1) of dim 8w + t: low halves of
      // r[..][t/2] for even t, high halves for odd t.
      const int bb = t >> 1;
      u32x4 bop;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t x0 = r[2 * pp][bb], x1 = r[2 * pp + 1][bb];
        bop[pp] = (t & 1) ? ((x0 >> 16) | (x1 & 0xffff0000u)) : ((x0 & 0xffffu) | (x1 << 16));
      }
      o[t] = mfma16x16x32(pa, bop, o[t]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    if (tn < t_end) cur = nxt;
  }

  // ---- merge the 4 waves of the block through LDS
  // Unconditional stores of all 16 rows (no per-row branches); the merge
  // below reads rows < G only.
  if ((lane & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s_m[wave][4 * g + i] = m[i];
      s_l[wave][4 * g + i] = l[i];
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_o[wave][4 * g + i][8 * (lane & 15) + t] = o[t][i];
  __syncthreads();
  for (int e = tid; e < G * kD; e += kThreads) {
    const int hh = e / kD, d = e % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][hh]);
    float acc = 0.f, lsum = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = fast_exp2(s_m[w][hh] - M);
        acc += wt * s_o[w][hh][d];
        lsum += wt * s_l[w][hh];
      }
    }
    rec[2 * G + hh * kD + d] = acc;
    if (d == 0) {
      rec[hh] = M;
      rec[G + hh] = lsum;
    }
  }
}


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

// One block per (query head, batch).  Thread (d = tid % 128, quarter qd =
// tid / 128) owns output dim d for the splits / hot tokens / PiV rows of its
// quarter; the 4 quarters are summed through LDS in a fixed order.
__global__ __launch_bounds__(kCombThreads) void tq_attn_combine_kernel(AttnParams P) {
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_p[kHotMax];
  __shared__ float s_red[kCombWaves];
  __shared__ __align__(16) float s_part[2][4][kD];
  __shared__ float s_rot[kD], s_hv[kD];
  __shared__ float s_o[4][kD];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int hq = blockIdx.x, b = blockIdx.y;
  const int G = P.G, kvh = hq / G, hh = hq % G;
  const int ns = P.nsplit;
  const int seq_len = *P.seq_len;  // only the masks below depend on it
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  const int RF = rec_floats(G);
  const float* recs = P.partials + bh * ns * RF;
  const size_t hot_base = bh * static_cast<size_t>(P.hot_cap) * kD;
  const int d = tid & (kD - 1), qd = tid >> 7;

  // ---- A. every load up front.  The hot window is walked by ring slot:
  // softmax sums do not depend on token order, and slot j holds a current
  // token exactly when j < hot_len (the window is the last hot_len tokens and
  // token t sits in slot t % hot_cap), so no address depends on the length.
  // Loads are unconditional from clamped, always valid addresses (split
  // ns - 1, slot hot_cap - 1) and masked after, so all are in flight together.
  float ms, ls;
  {
    const size_t sr = static_cast<size_t>(min(tid, ns - 1)) * RF;
    const float m_ = recs[sr + hh], l_ = recs[sr + G + hh];
    ms = tid < ns ? m_ : -INFINITY;
    ls = tid < ns ? l_ : 0.f;
  }
  float piv[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) piv[k] = P.PiV[(32 * qd + k) * kD + d];
  uint16_t hv[kHotMax / 4];
#pragma unroll
  for (int i = 0; i < kHotMax / 4; ++i) {
    const int jj = qd + 4 * i;
    hv[i] = P.v_hot[hot_base + static_cast<size_t>(min(jj, P.hot_cap - 1)) * kD + d];
  }
  float ca[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    ca[i] = recs[static_cast<size_t>(min(qd + 4 * i, ns - 1)) * RF + 2 * G + hh * kD + d];

  // hot score partial: slot j = tid / 8, dims 16 * (tid % 8) .. +16
  const int j = tid >> 3, part = tid & 7;
  float sdot = 0.f;
  {
    const int slot = min(j, P.hot_cap - 1);
    const uint4* kp = reinterpret_cast<const uint4*>(P.k_hot + hot_base + static_cast<size_t>(slot) * kD + 16 * part);
    const uint4* qp = reinterpret_cast<const uint4*>(P.q + (static_cast<size_t>(b) * P.Hq + hq) * kD + 16 * part);
    const uint4 k0 = kp[0], k1 = kp[1];
    const uint4 q0 = qp[0], q1 = qp[1];
    sdot = dot8_f16(k0, q0) + dot8_f16(k1, q1);  // slots past hot_len are masked by `score`
  }
  const int L = min(seq_len, P.max_len);
  const int hot_len = L - max(0, L - P.hot_cap);
  const bool hj = j < hot_len;
  // ---- B. softmax statistics over cold splits and hot tokens
  sdot += dpp_f<0xB1>(sdot);   // xor 1
  sdot += dpp_f<0x4E>(sdot);   // xor 2
  sdot += dpp_f<0x141>(sdot);  // the other quad of the 8-lane half row
  const float score = hj ? sdot * P.scale_log2 : -INFINITY;
  float v = fmaxf(ms, part == 0 ? score : -INFINITY);
  v = wave_max(v);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kCombWaves; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const float wsp = (tid < ns && ms != -INFINITY) ? fast_exp2(ms - M) : 0.f;
  const float pj = hj ? fast_exp2(score - M) : 0.f;
  if (tid < ns) s_w[tid] = wsp;
  if (part == 0 && j < kHotMax) s_p[j] = pj;
  float lv = wsp * ls + (part == 0 ? pj : 0.f);
  lv = wave_sum(lv);
  if (lane == 0) s_red[wave] = lv;
  __syncthreads();
  float Lt = 0.f;
#pragma unroll
  for (int w = 0; w < kCombWaves; ++w) Lt += s_red[w];

  // ---- C. weighted sums of this quarter: rotated cold, unrotated hot
  float cold = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int s = qd + 4 * i;
    const float w = s < ns ? s_w[s] : 0.f;
    cold += (w != 0.f) ? w * ca[i] : 0.f;
  }
  for (int s0 = 64; s0 < ns; s0 += 64) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      ca[i] = recs[static_cast<size_t>(min(s0 + qd + 4 * i, ns - 1)) * RF + 2 * G + hh * kD + d];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int s = s0 + qd + 4 * i;
      const float w = s < ns ? s_w[s] : 0.f;
      cold += (w != 0.f) ? w * ca[i] : 0.f;
    }
  }
  float hot = 0.f;
#pragma unroll
  for (int i = 0; i < kHotMax / 4; ++i) {
    const int jj = qd + 4 * i;
    const float t = s_p[jj < hot_len ? jj : 0] * h2f(hv[i]);
    hot += jj < hot_len ? t : 0.f;  // select after the product: an unwritten slot may hold NaN
  }
  s_part[0][qd][d] = cold;
  s_part[1][qd][d] = hot;
  __syncthreads();
  if (tid < kD) {
    s_rot[tid] = ((s_part[0][0][tid] + s_part[0][1][tid]) + s_part[0][2][tid]) + s_part[0][3][tid];
    s_hv[tid] = ((s_part[1][0][tid] + s_part[1][1][tid]) + s_part[1][2][tid]) + s_part[1][3][tid];
  }
  __syncthreads();

  // ---- D. un-rotate the cold sum: out[d] = sum_k rot[k] PiV[k][d]
  float o = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) o = fmaf(s_rot[32 * qd + k], piv[k], o);
  s_o[qd][d] = o;
  __syncthreads();
  if (tid < kD) {
    const float r = (((s_o[0][tid] + s_o[1][tid]) + s_o[2][tid]) + s_o[3][tid]) + s_hv[tid];
    P.out[(static_cast<size_t>(b) * P.Hq + hq) * kD + tid] = f2h(Lt > 0.f ? r / Lt : 0.f);
  }
}

// q_rot = q @ PiK^T for the G query heads of one (kv head, batch): one
// 16-row rotation tile (rows >= G are zero), the arithmetic of tq_rotate.
__global__ __launch_bounds__(tq::kThreads) void qrot_kernel(const uint16_t* __restrict__ q,
                                                            const float* __restrict__ PiK,
                                                            float* __restrict__ qrot, int Hq, int Hkv) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kvh = blockIdx.x, b = blockIdx.y, G = Hq / Hkv;
  float bop[2][32];
  tq::load_pi_operand(PiK, false, wave, lane, bop);
  const int r = lane & 15;
  float a[32];
  if (r < G) {
    tq::load_row_f16(q + (static_cast<size_t>(b) * Hq + kvh * G + r) * kD + 32 * (lane >> 4), a);
  } else {
#pragma unroll
    for (int s = 0; s < 32; ++s) a[s] = 0.f;
  }
  f32x4 acc[2];
  tq::rotate_tile(a, bop, acc);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * (lane >> 4) + i;
      const int dim = 8 * (lane & 15) + 2 * wave + t;
      if (row < G) qrot[(static_cast<size_t>(b) * Hq + kvh * G + row) * kD + dim] = acc[t][i];
    }
}

constexpr int kSplitGran = kWaves * kBlk;  // tokens one pass of a block covers

// Split count that gives ~4 blocks per CU (each wave's token loop is a
// latency chain, so more resident waves overlap more of them), at most
// kMaxSplits - 1.
int64_t target_splits(int64_t B, int64_t Hkv) {
  const int64_t target = 4 * static_cast<int64_t>(device_cu_count());
  int64_t ns = (target + B * Hkv - 1) / (B * Hkv);
  if (ns > kMaxSplits - 1) ns = kMaxSplits - 1;
  return ns < 1 ? 1 : ns;
}

}  // namespace

AttnPlan attn_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_len, int64_t hot_cap) {
  AttnPlan p{};
  const int64_t G = Hkv > 0 ? Hq / Hkv : 1;
  const int64_t cold_max = max_len > hot_cap ? max_len - hot_cap : 0;
  const int64_t ns_cap = target_splits(B, Hkv);
  int64_t ts = (cold_max + ns_cap - 1) / ns_cap;
  ts = (ts + kSplitGran - 1) / kSplitGran * kSplitGran;
  if (ts < kSplitGran) ts = kSplitGran;
  int64_t ns = (cold_max + ts - 1) / ts;
  if (ns < 1) ns = 1;
  p.nsplit = static_cast<int>(ns);
  p.split_tokens = static_cast<int>(ts);
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  p.qrot_off = kTicketBytes;  // keeps the shared workspace layout: ticket area first
  p.part_off = p.qrot_off + al(static_cast<size_t>(B * Hq * kD) * 4);
  // sized for ns_cap so a workspace sized without hot_cap fits every call
  p.total = p.part_off + al(static_cast<size_t>(B * Hkv * ns_cap * G * (2 + kD)) * 4);
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
  if (P.G <= 4)
    hipLaunchKernelGGL((tq_attn_split_kernel<4>), grid, dim3(kThreads), 0, st, P);
  else if (P.G <= 8)
    hipLaunchKernelGGL((tq_attn_split_kernel<8>), grid, dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((tq_attn_split_kernel<16>), grid, dim3(kThreads), 0, st, P);
  LKV_LAUNCH_CHECK("tq_decode_attn split");
  hipLaunchKernelGGL(tq_attn_combine_kernel, cgrid, dim3(kCombThreads), 0, st, P);
  LKV_LAUNCH_CHECK("tq_decode_attn combine");
  return LKV_OK;
}

}  // namespace lkv

using namespace lkv;

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
  LKV_REQUIRE(bits == 3 || bits == 4, "tq_decode_attn: bits=%d unsupported (4-bit nibble layouts only)", bits);
  LKV_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16,
              "tq_decode_attn: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%lld Hkv=%lld)", (long long)Hq,
              (long long)Hkv);
  LKV_REQUIRE(hot_cap >= 1 && hot_cap <= kHotMax, "tq_decode_attn: hot_cap must be 1..64");
  LKV_REQUIRE(max_len >= 0 && max_len <= cap + hot_cap, "tq_decode_attn: max_len=%lld exceeds cap+hot_cap=%lld",
              (long long)max_len, (long long)(cap + hot_cap));
  LKV_REQUIRE(max_len < (1ll << 31) && cap < (1ll << 31), "tq_decode_attn: length too large");
  if (B == 0) return LKV_OK;
  LKV_REQUIRE(q && k_codes && k_norms && v_codes && v_norms && k_hot && v_hot && PiK && PiV && centroids &&
                  seq_len && out && workspace,
              "tq_decode_attn: null pointer");
  LKV_REQUIRE(aligned16(q) && aligned16(k_codes) && aligned16(v_codes) && aligned16(k_hot) && aligned16(v_hot) &&
                  aligned16(PiK) && aligned16(out) && aligned16(workspace),
              "tq_decode_attn: q, codes, hot, PiK, out and workspace must be 16-byte aligned");
  const AttnPlan pl = attn_plan(B, Hq, Hkv, max_len, hot_cap);
  LKV_REQUIRE(workspace_bytes >= pl.total, "tq_decode_attn: workspace of %zu bytes required, got %zu", pl.total,
              workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* qrot = reinterpret_cast<float*>(ws + pl.qrot_off);
  hipLaunchKernelGGL(qrot_kernel, dim3(static_cast<unsigned>(Hkv), static_cast<unsigned>(B)), dim3(tq::kThreads), 0,
                     st, static_cast<const uint16_t*>(q), PiK, qrot, static_cast<int>(Hq), static_cast<int>(Hkv));
  LKV_LAUNCH_CHECK("tq_decode_attn q rotation");
  AttnCall c{};
  c.qrot = qrot;
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
