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
// Launches of lkv_tq_prefill_attn (all on the caller's stream):
//   1. q_rot = q @ PiK^T (fp32), hot rings k @ PiK^T and v @ PiV^T (fp16)
//      with the rotate kernel of lkv_tq_rotate;
//   2. tq_prefill_attn_kernel: grid (query tiles, kv heads, batch), 4 waves.
//      A block owns 128 (query, head) columns: 128 / G consecutive queries x
//      the G heads of one kv head, 32 columns per wave.  It walks the keys in
//      tiles of 32; per tile the block decodes the codes once into LDS --
//      keys as [key][dim] fp16 centroid values, values transposed as
//      [dim][key] -- and every wave runs, on v_mfma_f32_16x16x32_f16,
//      * scores transposed, A = 16 keys x 32 dims from LDS, B = its rotated
//        queries (registers), so a lane holds 8 keys of one column;
//      * the online softmax per lane (key norms, causal mask, exp2 domain,
//        max and sum across the 4 lanes of a column by permlane swaps);
//      * values transposed, A = 16 dims x 32 keys from LDS, B = p * n_t from
//        the lane's own softmax registers.
//      The next tile's codes load while the current one is computed.  Each
//      block writes its normalised rotated rows over its own q_rot rows;
//   3. out = rows @ PiV (fp16) with the rotate kernel.
#include "kernels.h"
#include "tq_attn_common.h"
#include "tq_common.h"

namespace lkv {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kKT = 32;         // keys per tile
constexpr int kCols = 128;      // (query, head) columns per block
constexpr int kRowB = 64;       // code bytes per token (4-bit nibbles)
constexpr int kKRow = kD + 8;   // fp16 row of the decoded key tile (padded)
constexpr int kVRow = kKT + 8;  // fp16 row of the transposed value tile (padded)
constexpr float kLog2e = 1.4426950408889634f;

struct PrefillParams {
  float* rows;             // [B, Hq, S, 128] fp32: q @ PiK^T in, normalised rotated output out
  const uint8_t* k_codes;  // [B, Hkv, cap, 64]
  const float* k_norms;    // [B, Hkv, cap]
  const uint8_t* v_codes;
  const float* v_norms;
  const uint16_t* hk;      // [B, Hkv, hot_cap, 128] fp16: hot keys @ PiK^T (ring slots)
  const uint16_t* hv;      // hot values @ PiV^T
  const float* centroids;  // [2^bits]
  float scale_log2;        // scale * log2(e)
  int S, Hq, Hkv, G, cap, hot_cap, kv_len, cold_len, ncent;
};

// fp16 positions 0..7 of a natural-order group reordered to kPermDim.
__device__ __forceinline__ uint4 perm_group(uint4 a) {
  return uint4{__builtin_amdgcn_perm(a.y, a.x, 0x05040100u), __builtin_amdgcn_perm(a.w, a.z, 0x05040100u),
               __builtin_amdgcn_perm(a.y, a.x, 0x07060302u), __builtin_amdgcn_perm(a.w, a.z, 0x07060302u)};
}

template <bool PERM>
__global__ __launch_bounds__(kThreads, 2) void tq_prefill_attn_kernel(PrefillParams P) {
  __shared__ __align__(16) uint16_t sK[kKT * kKRow];
  __shared__ __align__(16) uint16_t sVt[kD * kVRow];
  __shared__ __align__(16) uint8_t sRaw[2 * kKT * kRowB];  // key codes, then value codes
  __shared__ __align__(16) float sN[2][kKT];                 // key, value norms (1 for hot, 0 past the end)
  __shared__ uint32_t s_lut[256];
  __shared__ uint16_t s_cent[16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h16 = lane & 15, g = lane >> 4;
  const int G = P.G, QT = kCols / G;
  // the latest queries see the most keys: their tiles are dispatched first
  const int qtile = static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x);
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int q0 = qtile * QT;
  const int qpos0 = P.kv_len - P.S;  // position of query 0
  const size_t bh = static_cast<size_t>(b) * P.Hkv + kvh;
  const int cold_len = P.cold_len, kv_len = P.kv_len;

  // ---- centroid tables
  uint32_t tab[4] = {0u, 0u, 0u, 0u};
  if constexpr (PERM) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t c16 = f2h(P.centroids[j]);
      tab[j >> 2] |= (c16 & 0xffu) << (8 * (j & 3));
      tab[2 + (j >> 2)] |= (c16 >> 8) << (8 * (j & 3));
    }
  } else {
    const int cmax = P.ncent - 1;
    s_lut[tid] = pack2h(P.centroids[min(tid & 15, cmax)], P.centroids[min(tid >> 4, cmax)]);
  }
  if (tid < 16) s_cent[tid] = f2h(P.centroids[min(tid, P.ncent - 1)]);

  // ---- query operands: column c = 32 wave + 16 ct + lane % 16 is query
  // q0 + c / G, head c % G; B operand dims 32 kb + 8 (lane / 16) + position.
  int lim[2];  // keys [0, lim) visible to the lane's column (0: no such query)
  u32x4 qa[2][4];
  int wmin = 0x7fffffff;
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int c = 32 * wave + 16 * ct + h16;
    const int qq = q0 + c / G, hh = c % G;
    const bool ok = qq < P.S;
    lim[ct] = ok ? qpos0 + qq + 1 : 0;
    if (ok) wmin = min(wmin, lim[ct]);
    const float* src =
        P.rows + ((static_cast<size_t>(b) * P.Hq + kvh * G + hh) * P.S + min(qq, P.S - 1)) * kD + 8 * g;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const float4 f0 = *reinterpret_cast<const float4*>(src + 32 * kb);
      const float4 f1 = *reinterpret_cast<const float4*>(src + 32 * kb + 4);
      const float x[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = PERM ? kPermDim[2 * j] : 2 * j, d1 = PERM ? kPermDim[2 * j + 1] : 2 * j + 1;
        v[j] = pack2h(x[d0] * P.scale_log2, x[d1] * P.scale_log2);
      }
      qa[ct][kb] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wmin = min(wmin, __shfl_xor(wmin, o));
  wmin = __builtin_amdgcn_readfirstlane(wmin);

  // keys [0, kend) are visible to some column of the block
  const int kend = qpos0 + min(q0 + QT, P.S);
  const int ntile = (kend + kKT - 1) / kKT;

  // ---- staging: thread t loads 16 code bytes of key (t & 127) / 4 of the
  // key (t < 128) or value side; threads < 64 one norm each.
  const int side = tid >> 7, rr = (tid & 127) >> 2, cb = 16 * (tid & 3);
  const uint8_t* codes = (side ? P.v_codes : P.k_codes) + bh * static_cast<size_t>(P.cap) * kRowB;
  const float* norms = ((tid >> 5) & 1 ? P.v_norms : P.k_norms) + bh * static_cast<size_t>(P.cap);
  auto load_raw = [&](int t0) -> uint4 {
    if (cold_len <= 0) return uint4{0u, 0u, 0u, 0u};
    const int tc = min(t0 + rr, cold_len - 1);  // clamped valid row; keys past cold_len are not decoded from it
    return *reinterpret_cast<const uint4*>(codes + static_cast<size_t>(tc) * kRowB + cb);
  };
  auto load_norm = [&](int t0) -> float {
    const int tk = t0 + (tid & 31);
    const float n = cold_len > 0 ? norms[min(tk, cold_len - 1)] : 0.f;
    return tk < cold_len ? n : (tk < kv_len ? 1.f : 0.f);
  };
  uint4 raw = load_raw(0);
  float nrm = tid < 64 ? load_norm(0) : 0.f;

  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[ct][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int it = 0; it < ntile; ++it) {
    const int t0 = it * kKT;
    // ---- stage the tile's codes and norms; then the next tile's loads
    *reinterpret_cast<uint4*>(sRaw + side * kKT * kRowB + rr * kRowB + cb) = raw;
    if (tid < 64) sN[tid >> 5][tid & 31] = nrm;
    __syncthreads();  // also: every wave is done with the previous tile's sK / sVt
    if (it + 1 < ntile) {
      raw = load_raw(t0 + kKT);
      if (tid < 64) nrm = load_norm(t0 + kKT);
    }
    // ---- keys -> sK [key][dim] (kPermDim order within each 8-dim group with PERM)
    {
      const int kk = tid >> 3, part = tid & 7, tk = t0 + kk;
      uint4 o0, o1;
      if (tk < cold_len) {
        const uint2 w = *reinterpret_cast<const uint2*>(sRaw + kk * kRowB + 8 * part);
        uint32_t d0[4], d1[4];
        decode_dw<PERM>(w.x, tab, s_lut, d0);
        decode_dw<PERM>(w.y, tab, s_lut, d1);
        o0 = uint4{d0[0], d0[1], d0[2], d0[3]};
        o1 = uint4{d1[0], d1[1], d1[2], d1[3]};
      } else if (tk < kv_len) {
        const uint4* src = reinterpret_cast<const uint4*>(
            P.hk + (bh * P.hot_cap + static_cast<size_t>(tk % P.hot_cap)) * kD + 16 * part);
        o0 = src[0];
        o1 = src[1];
        if constexpr (PERM) {
          o0 = perm_group(o0);
          o1 = perm_group(o1);
        }
      } else {
        o0 = o1 = uint4{0u, 0u, 0u, 0u};
      }
      *reinterpret_cast<uint4*>(sK + kk * kKRow + 16 * part) = o0;
      *reinterpret_cast<uint4*>(sK + kk * kKRow + 16 * part + 8) = o1;
    }
    // ---- values -> sVt [dim][key]: thread = dims 2j, 2j+1 of keys 8 kg .. 8 kg + 7
    {
      const int j = tid & 63, kg = tid >> 6, tb = t0 + 8 * kg;
      const uint8_t* vr = sRaw + kKT * kRowB + (8 * kg) * kRowB + j;
      uint32_t r0[4], r1[4];  // fp16 pairs (keys 2e, 2e+1) of dim 2j and of dim 2j+1
      if (tb + 8 <= cold_len) {
        const uint32_t wa = vr[0] | (static_cast<uint32_t>(vr[kRowB]) << 8) |
                            (static_cast<uint32_t>(vr[2 * kRowB]) << 16) | (static_cast<uint32_t>(vr[3 * kRowB]) << 24);
        const uint32_t wb = vr[4 * kRowB] | (static_cast<uint32_t>(vr[5 * kRowB]) << 8) |
                            (static_cast<uint32_t>(vr[6 * kRowB]) << 16) | (static_cast<uint32_t>(vr[7 * kRowB]) << 24);
        if constexpr (PERM) {
          // byte k of wa / wb is key k's byte j: low nibble dim 2j, high nibble dim 2j + 1
          uint32_t da[4], db[4];
          decode8(wa, tab, da);
          decode8(wb, tab, db);
          r0[0] = da[0]; r0[1] = da[1]; r0[2] = db[0]; r0[3] = db[1];
          r1[0] = da[2]; r1[1] = da[3]; r1[2] = db[2]; r1[3] = db[3];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w = e < 2 ? wa : wb;
            const uint32_t x0 = s_lut[(w >> (16 * (e & 1))) & 0xffu], x1 = s_lut[(w >> (16 * (e & 1) + 8)) & 0xffu];
            r0[e] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
            r1[e] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t lo2 = 0u, hi2 = 0u;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int tk = tb + 2 * e + k;
            uint32_t lo = 0u, hi = 0u;
            if (tk < cold_len) {
              const uint32_t byte = vr[(2 * e + k) * kRowB];
              lo = s_cent[byte & 15u];
              hi = s_cent[byte >> 4];
            } else if (tk < kv_len) {
              const uint32_t pr = *reinterpret_cast<const uint32_t*>(
                  P.hv + (bh * P.hot_cap + static_cast<size_t>(tk % P.hot_cap)) * kD + 2 * j);
              lo = pr & 0xffffu;
              hi = pr >> 16;
            }
            lo2 |= lo << (16 * k);
            hi2 |= hi << (16 * k);
          }
          r0[e] = lo2;
          r1[e] = hi2;
        }
      }
      *reinterpret_cast<uint4*>(sVt + (2 * j) * kVRow + 8 * kg) = uint4{r0[0], r0[1], r0[2], r0[3]};
      *reinterpret_cast<uint4*>(sVt + (2 * j + 1) * kVRow + 8 * kg) = uint4{r1[0], r1[1], r1[2], r1[3]};
    }
    __syncthreads();

    // ---- scores: S^T tiles [ct][tt] = keys 16 tt .. x columns of ct
    f32x4 sc[2][2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sc[ct][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(sK + (16 * tt + h16) * kKRow + 32 * kb + 8 * g);
        sc[0][tt] = mfma16x16x32(a, qa[0][kb], sc[0][tt]);
        sc[1][tt] = mfma16x16x32(a, qa[1][kb], sc[1][tt]);
      }
    // the lane's keys: t0 + 16 tt + 4 g + i, i.e. slot j = 4 tt + i
    const f32x4 kn0 = *reinterpret_cast<const f32x4*>(&sN[0][4 * g]);
    const f32x4 kn1 = *reinterpret_cast<const f32x4*>(&sN[0][16 + 4 * g]);
    const f32x4 vn0 = *reinterpret_cast<const f32x4*>(&sN[1][4 * g]);
    const f32x4 vn1 = *reinterpret_cast<const f32x4*>(&sN[1][16 + 4 * g]);
    const bool masked = t0 + kKT > wmin;  // wave-uniform
    u32x4 pb[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float s[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = sc[ct][0][i] * kn0[i];
        s[4 + i] = sc[ct][1][i] * kn1[i];
      }
      if (masked) {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          s[jj] = t0 + 16 * (jj >> 2) + 4 * g + (jj & 3) < lim[ct] ? s[jj] : -INFINITY;
      }
      float mx = s[0];
#pragma unroll
      for (int jj = 1; jj < 8; ++jj) mx = vmax(mx, s[jj]);
      mx = xgroup_max(mx);
      const float mn = fmaxf(m[ct], mx);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m[ct] - mu);
      m[ct] = mn;
      float p[8], ps = 0.f;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        p[jj] = fast_exp2(s[jj] - mu);
        ps += p[jj];
      }
      l[ct] = l[ct] * alpha + ps;
      if (wave_ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[ct][dt] = o[ct][dt] * alpha;
      }
      pb[ct] = u32x4{pack2h(p[0] * vn0[0], p[1] * vn0[1]), pack2h(p[2] * vn0[2], p[3] * vn0[3]),
                     pack2h(p[4] * vn1[0], p[5] * vn1[1]), pack2h(p[6] * vn1[2], p[7] * vn1[3])};
    }
    // ---- values: O^T tiles [ct][dt] += V^T (dims 16 dt .., the lane's 8 keys) x P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* row = sVt + (16 * dt + h16) * kVRow;
      const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * g);
      const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * g);
      const u32x4 a = u32x4{lo.x, lo.y, hi.x, hi.y};
      o[0][dt] = mfma16x16x32(a, pb[0], o[0][dt]);
      o[1][dt] = mfma16x16x32(a, pb[1], o[1][dt]);
    }
  }

  // ---- normalise and write the rotated rows over the block's own q_rot rows
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const float L = xgroup_sum(l[ct]);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int c = 32 * wave + 16 * ct + h16;
    const int qq = q0 + c / G, hh = c % G;
    if (qq < P.S) {
      float* dst = P.rows + ((static_cast<size_t>(b) * P.Hq + kvh * G + hh) * P.S + qq) * kD + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(dst + 16 * dt) = o[ct][dt] * inv;
    }
  }
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" size_t lkv_tq_prefill_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                                      int64_t hot_cap) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || S <= 0 || hot_cap <= 0) return 0;
  const size_t rows = static_cast<size_t>(B * Hq * S) * kD * 4;
  const size_t hot = static_cast<size_t>(B * Hkv * hot_cap) * kD * 2;
  return (rows + 255) / 256 * 256 + 2 * ((hot + 255) / 256 * 256);
}

extern "C" int lkv_tq_prefill_attn(const void* q, const uint8_t* k_codes, const float* k_norms,
                                   const uint8_t* v_codes, const float* v_norms, const void* k_hot,
                                   const void* v_hot, const float* PiK, const float* PiV, const float* centroids,
                                   int bits, int64_t kv_len, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                                   int64_t cap, int64_t hot_cap, float scale, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  LKV_REQUIRE(bits == 3 || bits == 4, "tq_prefill_attn: bits=%d unsupported (4-bit nibble layouts only)", bits);
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
  char* ws = static_cast<char*>(workspace);
  const int64_t nrows = B * Hq * S;
  float* rows = reinterpret_cast<float*>(ws);
  uint16_t* hk = reinterpret_cast<uint16_t*>(ws + (static_cast<size_t>(nrows) * kD * 4 + 255) / 256 * 256);
  const size_t hot_bytes = (static_cast<size_t>(B * Hkv * hot_cap) * kD * 2 + 255) / 256 * 256;
  uint16_t* hv = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(hk) + hot_bytes);
  const int64_t cold_len = kv_len > hot_cap ? kv_len - hot_cap : 0;

  if (int e = rotate_rows(q, true, nrows, PiK, 0, rows, false, st)) return e;
  if (kv_len > cold_len) {  // the ring holds hot tokens: rotate every slot (only current ones are read)
    if (int e = rotate_rows(k_hot, true, B * Hkv * hot_cap, PiK, 0, hk, true, st)) return e;
    if (int e = rotate_rows(v_hot, true, B * Hkv * hot_cap, PiV, 0, hv, true, st)) return e;
  }
  PrefillParams P;
  P.rows = rows;
  P.k_codes = k_codes;
  P.k_norms = k_norms;
  P.v_codes = v_codes;
  P.v_norms = v_norms;
  P.hk = hk;
  P.hv = hv;
  P.centroids = centroids;
  P.scale_log2 = scale * kLog2e;
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
  if (bits == 3)
    hipLaunchKernelGGL((tq_prefill_attn_kernel<true>), grid, dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((tq_prefill_attn_kernel<false>), grid, dim3(kThreads), 0, st, P);
  LKV_LAUNCH_CHECK("tq_prefill_attn");
  return rotate_rows(rows, false, nrows, PiV, 1, out, true, st);
}
