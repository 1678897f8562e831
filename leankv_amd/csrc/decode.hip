// Fused B=1 decode step: 8 launches per decoder layer, all state on the device.
//
// The reference decodes through HF generate(): per token, Python walks the
// layers of MistralDecoderLayer (transformers/models/mistral/
// modeling_mistral.py), each TEAL-patched projection launches its own GEMV
// (leankv/teal/patching.py:152-183) and TurboQuantCache.update dequantizes
// the cold store (leankv/turboquant/cache.py:84-189).  Here the same
// arithmetic is regrouped around the GEMVs, which dominate the bytes:
//
//   x (fp16 residual)
//   1. GEMV q|k|v (one launch, 3 segments), prologue x -> RMSNorm(x) * w
//   2. attention split (cold codes), prologue: q|k|v partial sums -> fp16,
//      RoPE, q rotation; new k/v into the hot ring (one block per kv head)
//   3. combine (+ hot window, PiV)
//   4. GEMV o_proj                                5. x += o
//   6. GEMV gate|up (dual), prologue RMSNorm       7. GEMV down, prologue
//      SwiGLU of the gate/up partial sums          8. x += down
//   Per step, before the layers: evict_kernel quantizes, for every layer,
//   the token leaving the hot window.
//   head: GEMV lm_head (prologue final RMSNorm), logits + per-block argmax,
//   final argmax -> tok, pos + 1.
//
// Split-K partial sums are reduced in chunk order by their consumer, so every
// projection equals the standalone lkv_sparse_gemv result for the same chunk
// size.  Rounding follows the fp16 HF modules (see each kernel).
#include "kernels.h"
#include "tq_common.h"

namespace lkv {
namespace {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kMaxG = 8;  // query heads per kv head of the decode step
constexpr int kF16Page = 16;  // tokens per page of the fp16-KV step's pool

struct Plan {
  int64_t Hq, Hkv, G, nq, nkv;                 // q / k,v projection widths
  int64_t sq, sk, sh, sf, svoc;                // column slabs
  int bz_qkv, bz_o, bz_gu, bz_d, bz_lm;
  int nc_qkv, nc_o, nc_gu, nc_d, nc_lm;
  AttnPlan attn;
  int64_t f16_pages;  // pages of the fp16-KV step's pool (kF16Page tokens each)
  size_t off_state, off_pqkv, off_po, off_pgu, off_pd, off_plm, off_q16, off_attn, off_rec, off_cand, off_pt,
      off_prec, prec_bytes, total;
};

size_t al256(size_t v) { return (v + 255) / 256 * 256; }

Plan make_plan(const lkv_decode_dims& d) {
  Plan p{};
  p.Hq = d.n_heads;
  p.Hkv = d.n_kv_heads;
  p.G = d.n_heads / d.n_kv_heads;
  p.nq = d.n_heads * kD;
  p.nkv = d.n_kv_heads * kD;
  p.sq = gemv_slabs(p.nq);
  p.sk = gemv_slabs(p.nkv);
  p.sh = gemv_slabs(d.hidden);
  p.sf = gemv_slabs(d.ffn);
  p.svoc = gemv_slabs(d.vocab);
  p.bz_qkv = gemv_pick_bz(p.sq + 2 * p.sk, d.hidden);
  p.bz_o = gemv_pick_bz(p.sh, p.nq);
  p.bz_gu = gemv_pick_bz(p.sf, d.hidden);
  p.bz_d = gemv_pick_bz(p.sh, d.ffn);
  p.bz_lm = gemv_pick_bz(p.svoc, d.hidden);
  p.nc_qkv = static_cast<int>(gemv_chunks(d.hidden, p.bz_qkv));
  p.nc_o = static_cast<int>(gemv_chunks(p.nq, p.bz_o));
  p.nc_gu = static_cast<int>(gemv_chunks(d.hidden, p.bz_gu));
  p.nc_d = static_cast<int>(gemv_chunks(d.ffn, p.bz_d));
  p.nc_lm = static_cast<int>(gemv_chunks(d.hidden, p.bz_lm));
  p.attn = attn_plan(1, p.Hq, p.Hkv, d.max_len, d.hot_cap);
  size_t o = kTicketBytes;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += al256(bytes);
    return at;
  };
  p.off_state = take(2 * sizeof(int32_t));
  p.off_pqkv = take((gemv_part_floats(p.nq, p.nc_qkv) + 2 * gemv_part_floats(p.nkv, p.nc_qkv)) * 4);
  p.off_po = take(gemv_part_floats(d.hidden, p.nc_o) * 4);
  p.off_pgu = take(2 * gemv_part_floats(d.ffn, p.nc_gu) * 4);
  p.off_pd = take(gemv_part_floats(d.hidden, p.nc_d) * 4);
  p.off_plm = take(gemv_part_floats(d.vocab, p.nc_lm) * 4);
  p.off_q16 = take(static_cast<size_t>(p.nq) * 2);
  p.off_attn = take(static_cast<size_t>(p.nq) * 2);
  p.off_rec = take(p.attn.total - p.attn.part_off);
  p.off_cand = take(static_cast<size_t>(p.svoc) * 8);
  p.f16_pages = (d.max_len + kF16Page - 1) / kF16Page;
  p.off_pt = take(static_cast<size_t>(3 + p.f16_pages) * 4);
  p.prec_bytes = lkv_paged_decode_attn_workspace_bytes(1, d.n_heads, d.n_kv_heads, d.max_len);
  p.off_prec = take(p.prec_bytes);
  p.total = o;
  return p;
}

int check_dims(const lkv_decode_dims* d) {
  LKV_REQUIRE(d != nullptr, "decode: null dims");
  LKV_REQUIRE(d->hidden > 0 && d->hidden % 256 == 0, "decode: hidden=%lld must be a positive multiple of 256",
              (long long)d->hidden);
  LKV_REQUIRE(d->ffn > 0 && d->ffn % 256 == 0, "decode: ffn=%lld must be a positive multiple of 256",
              (long long)d->ffn);
  LKV_REQUIRE(d->vocab > 0 && d->vocab % 8 == 0, "decode: vocab=%lld must be a positive multiple of 8",
              (long long)d->vocab);
  LKV_REQUIRE(d->n_heads > 0 && d->n_kv_heads > 0 && d->n_heads % d->n_kv_heads == 0 &&
                  d->n_heads / d->n_kv_heads <= kMaxG,
              "decode: n_heads=%lld must be a multiple of n_kv_heads=%lld with at most %d query heads per kv head",
              (long long)d->n_heads, (long long)d->n_kv_heads, kMaxG);
  LKV_REQUIRE(d->hot_cap >= 1 && d->hot_cap <= 256, "decode: hot_cap must be 1..256 (the combine walks 256 slots)");
  LKV_REQUIRE(d->max_len >= 1 && d->max_len < (1ll << 30), "decode: max_len=%lld out of range", (long long)d->max_len);
  LKV_REQUIRE(d->cap >= d->max_len - d->hot_cap && d->cap < (1ll << 30),
              "decode: cap=%lld cannot hold max_len - hot_cap = %lld cold tokens", (long long)d->cap,
              (long long)(d->max_len - d->hot_cap));
  LKV_REQUIRE(d->bits >= 1 && d->bits <= 4, "decode: bits=%d unsupported (1..4)", d->bits);
  LKV_REQUIRE(d->bounds && d->centroids && d->rope_cos && d->rope_sin, "decode: null codebook or RoPE table");
  LKV_REQUIRE(aligned16(d->rope_cos) && aligned16(d->rope_sin), "decode: RoPE tables must be 16-byte aligned");
  const int64_t wmax = d->hidden * (d->ffn > d->vocab ? d->ffn : d->vocab);
  LKV_REQUIRE(wmax * 2 < (1ll << 32) && d->hidden * d->n_heads * kD * 2 < (1ll << 32),
              "decode: a weight matrix exceeds the 4 GiB buffer-descriptor range");
  return LKV_OK;
}

int check_ws(const Plan& p, const void* ws, size_t bytes) {
  LKV_REQUIRE(ws && aligned16(ws) && bytes >= p.total, "decode: workspace of %zu bytes (16-byte aligned) required, got %zu",
              p.total, bytes);
  return LKV_OK;
}

// ------------------------------------------------------------------ kernels

// x = embed[tok]; state = {pos, pos + 1} (pos clamped into the tables).
__global__ __launch_bounds__(kThreads) void begin_kernel(const uint16_t* __restrict__ embed,
                                                         const int64_t* __restrict__ tok,
                                                         const int64_t* __restrict__ pos, uint16_t* __restrict__ x,
                                                         int32_t* __restrict__ state, int64_t hidden, int64_t vocab,
                                                         int64_t max_len) {
  int64_t t = *tok;
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;
  if (i < hidden)
    *reinterpret_cast<uint4*>(x + i) = *reinterpret_cast<const uint4*>(embed + t * hidden + i);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    int64_t p = *pos;
    p = p < 0 ? 0 : (p >= max_len ? max_len - 1 : p);
    state[0] = static_cast<int32_t>(p);
    state[1] = static_cast<int32_t>(p + 1);
  }
}

// x[n] = fp16(x[n] + fp16(sum of chunks)): the fp16 residual add of the decoder layer.
__global__ __launch_bounds__(kThreads) void residual_kernel(uint16_t* __restrict__ x, const float* __restrict__ part,
                                                            int N, int nchunk) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  if (n >= N) return;
  // x is loaded with the partials and converted after them: one memory round trip
  const uint16_t xv = x[n];
  const float o = h2f(f2h(column_sum(part, n, nchunk)));
  x[n] = f2h(h2f(xv) + o);
}

// The fp16-KV step's q|k|v epilogue (the dense baseline's cache append): the
// q|k|v partial sums in chunk order, fp16, RoPE at pos for q and k (rope_pair,
// the arithmetic of the TurboQuant split kernel's prologue, so both steps
// produce the same query and key bits), the query to q16, the key and value
// into the token's slot of the fp16 page pool kv [page][K, V][kF16Page][Hkv]
// [128] (token t in page t / kF16Page, slot t % kF16Page), and the page table
// of the one sequence over identity pages: pt = {indptr 0, npages,
// last page length, pages 0 .. npages - 1}.  Items: nq / 2 query dim pairs,
// then nkv / 2 key pairs, then nkv / 2 value pairs.
__global__ __launch_bounds__(kThreads) void f16kv_prep_kernel(const float* __restrict__ pq,
                                                              const float* __restrict__ pk,
                                                              const float* __restrict__ pv, int nchunk,
                                                              const uint16_t* __restrict__ rope_cos,
                                                              const uint16_t* __restrict__ rope_sin,
                                                              const int32_t* __restrict__ state,
                                                              uint16_t* __restrict__ q16, uint16_t* __restrict__ kv,
                                                              int32_t* __restrict__ pt, int nq, int nkv, int Hkv) {
  const int pos = state[0];
  const int e = blockIdx.x * kThreads + threadIdx.x;
  const uint16_t* cos_row = rope_cos + static_cast<size_t>(pos) * kD;
  const uint16_t* sin_row = rope_sin + static_cast<size_t>(pos) * kD;
  const size_t page = pos / kF16Page, slot = pos % kF16Page;
  const size_t row = static_cast<size_t>(Hkv) * kD;  // one token of one page half
  uint16_t* kdst = kv + (page * 2 * kF16Page + slot) * row;
  uint16_t* vdst = kv + ((page * 2 + 1) * kF16Page + slot) * row;
  const int nqp = nq / 2, nkp = nkv / 2;
  if (e < nqp + 2 * nkp) {
    const bool is_q = e < nqp, is_k = !is_q && e < nqp + nkp;
    const int i = is_q ? e : (is_k ? e - nqp : e - nqp - nkp);
    const int col = (i / 64) * kD + i % 64;
    const float* P = is_q ? pq : (is_k ? pk : pv);
    float x0, x1, o0, o1;
    column_sum2(P, col, col + 64, nchunk, x0, x1);
    if (is_q || is_k) {
      rope_pair(x0, x1, cos_row, sin_row, i % 64, o0, o1);
    } else {
      o0 = x0;
      o1 = x1;
    }
    uint16_t* dst = is_q ? q16 : (is_k ? kdst : vdst);
    dst[col] = f2h(o0);
    dst[col + 64] = f2h(o1);
  }
  if (blockIdx.x == 0) {
    const int npages = static_cast<int>(page) + 1;
    if (threadIdx.x == 0) {
      pt[0] = 0;
      pt[1] = npages;
      pt[2] = static_cast<int>(slot) + 1;
    }
    for (int j = threadIdx.x; j < npages; j += kThreads) pt[3 + j] = j;
  }
}

// y = RMSNorm(x) * w for M rows of Z; block (j, m) writes columns
// [256 j, 256 j + 256) of row m after computing the row's rstd itself.
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w, float eps, int Z,
                                                           uint16_t* __restrict__ y) {
  __shared__ float s_wsum[kThreads / kWave];
  const size_t row = static_cast<size_t>(blockIdx.y) * Z;
  const float rstd = rms_rstd(x + row, Z, eps, s_wsum);
  const int z = blockIdx.x * kThreads + threadIdx.x;
  if (z < Z) y[row + z] = f2h(rms_apply(x[row + z], w[z], rstd));
}

// The token leaving the hot window at this step, for up to kEvictLayers
// layers per launch: the layer table travels as kernel arguments.
constexpr int kEvictLayers = 32;
struct EvictLayer {
  const uint16_t* k_hot;
  const uint16_t* v_hot;
  uint8_t* k_codes;
  float* k_norms;
  uint8_t* v_codes;
  float* v_norms;
  const float* PiK;
  const float* PiV;
};
struct EvictArgs {
  const int32_t* state;
  const float* bounds;
  int hot_cap, cap, Hkv;
  EvictLayer L[kEvictLayers];
};

// Grid (groups of 16 kv heads, {key, value}, layers).  At position pos the
// token pos - hot_cap leaves the hot window (cache.py:84-141 flushes the
// oldest hot token once the window exceeds hot_cap): the block takes that
// token of up to 16 kv heads of one layer as the 16 rows of one MFMA tile
// (row r = kv head 16 blockIdx.x + r), normalises, rotates with Pi and buckets
// them (tq_common.h's arithmetic, row by row independent, so the codes equal
// lkv_tq_cache_append's), and their codes and norms go to cold slot
// pos - hot_cap.  Its ring slot, pos % hot_cap, is the one this step's new
// token overwrites, so this kernel runs before the step's first layer; none of
// the step's layer work depends on it until attention, so one launch covers
// every layer.  The block's 64 KB rotation matrix is fetched once for its 16
// heads with coalesced 16-byte loads and staged in LDS for the operand reads.
template <int BITS>
__global__ __launch_bounds__(kThreads) void evict_kernel(EvictArgs A) {
  constexpr int kPiLd = kD + 1;  // padded LDS row
  __shared__ float s_pi[kD * kPiLd];
  __shared__ uint8_t s_codes[tq::kRows * kD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h0 = 16 * blockIdx.x;
  const int nh = min(16, A.Hkv - h0);
  const bool vside = blockIdx.y == 1;
  const EvictLayer& Ly = A.L[blockIdx.z];
  const int pos = A.state[0];
  const int ev = pos - A.hot_cap;
  if (!(pos >= A.hot_cap && ev < A.cap)) return;  // uniform: nothing leaves the window
  const float* Pi = vside ? Ly.PiV : Ly.PiK;
  float4 pr[kD * kD / 4 / kThreads];
#pragma unroll
  for (int i = 0; i < kD * kD / 4 / kThreads; ++i) pr[i] = reinterpret_cast<const float4*>(Pi)[i * kThreads + tid];
  float bd[(1 << BITS) - 1];
#pragma unroll
  for (int i = 0; i < (1 << BITS) - 1; ++i) bd[i] = A.bounds[i];
  const int r = lane & 15, c0 = 32 * (lane >> 4);
  const bool row_ok = r < nh;
  const int slot = pos % A.hot_cap;
  const uint16_t* hot = vside ? Ly.v_hot : Ly.k_hot;
  uint4 hraw[4];  // row r: kv head h0 + r (rows past the heads read head h0 and are zeroed)
  {
    const int hh = h0 + (row_ok ? r : 0);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      hraw[v] = reinterpret_cast<const uint4*>(hot + (static_cast<size_t>(hh) * A.hot_cap + slot) * kD + c0)[v];
  }
#pragma unroll
  for (int i = 0; i < kD * kD / 4 / kThreads; ++i) {
    const int f = i * kThreads + tid;  // float4 index: row f / 32, columns 4 (f % 32) ..
    float* dst = s_pi + (f >> 5) * kPiLd + 4 * (f & 31);
    dst[0] = pr[i].x;
    dst[1] = pr[i].y;
    dst[2] = pr[i].z;
    dst[3] = pr[i].w;
  }
  __syncthreads();
  // tq::load_row_f16's conversion of the preloaded rows; rows past the heads are zero
  float a[32];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t w[4] = {hraw[v].x, hraw[v].y, hraw[v].z, hraw[v].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[8 * v + 2 * i] = row_ok ? h2f(static_cast<uint16_t>(w[i] & 0xffffu)) : 0.f;
      a[8 * v + 2 * i + 1] = row_ok ? h2f(static_cast<uint16_t>(w[i] >> 16)) : 0.f;
    }
  }
  float bop[2][32];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const float* row = s_pi + (8 * (lane & 15) + 2 * wave + t) * kPiLd + c0;
#pragma unroll
    for (int s = 0; s < 32; ++s) bop[t][s] = row[s];
  }
  // cache.py:141 quantizes flush_k.float(): fp32 semantics on the fp16 data.
  const float nrm = tq::normalize_row_f32_if(a, row_ok);
  f32x4 acc[2];
  tq::rotate_tile(a, bop, acc);
  tq::codes_to_lds<BITS>(acc, bd, wave, lane, s_codes);
  if (wave == 0 && lane < nh) (vside ? Ly.v_norms : Ly.k_norms)[static_cast<size_t>(h0 + lane) * A.cap + ev] = nrm;
  __syncthreads();
  const int cap = A.cap;
  tq::pack_store<BITS>(s_codes, vside ? Ly.v_codes : Ly.k_codes, 0, nh, [=](int64_t row) {
    return (static_cast<int64_t>(h0 + row) * cap + ev) * tq::row_bytes_for(BITS);
  });
}


struct Cand {
  float v;
  int i;
};

__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__device__ __forceinline__ void block_argmax(float& v, int& i, Cand* s_c) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) argmax_merge(v, i, __shfl_xor(v, o), __shfl_xor(i, o));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) s_c[wave] = Cand{v, i};
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / kWave; ++w) argmax_merge(v, i, s_c[w].v, s_c[w].i);
  }
}

// logits[n] = fp16(sum of chunks); per-block (max, lowest index of max).
__global__ __launch_bounds__(kThreads) void logits_kernel(const float* __restrict__ part, int vocab, int nchunk,
                                                          uint16_t* __restrict__ logits, Cand* __restrict__ cand) {
  __shared__ Cand s_c[kThreads / kWave];
  const int n = blockIdx.x * kThreads + threadIdx.x;
  float v = -INFINITY;
  int i = n < vocab ? n : 0x7fffffff;
  if (n < vocab) {
    const uint16_t h = f2h(column_sum(part, n, nchunk));
    logits[n] = h;
    v = h2f(h);
  }
  block_argmax(v, i, s_c);
  if (threadIdx.x == 0) cand[blockIdx.x] = Cand{v, i};
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(const Cand* __restrict__ cand, int ncand,
                                                          int64_t* __restrict__ tok, int64_t* __restrict__ pos,
                                                          int64_t* __restrict__ hist, int64_t hist_len) {
  __shared__ Cand s_c[kThreads / kWave];
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int c = threadIdx.x; c < ncand; c += kThreads) argmax_merge(v, i, cand[c].v, cand[c].i);
  block_argmax(v, i, s_c);
  if (threadIdx.x == 0) {
    const int64_t t = i == 0x7fffffff ? 0 : i, p = *pos;
    *tok = t;
    *pos = p + 1;
    if (hist != nullptr && p >= 0 && p < hist_len) hist[p] = t;
  }
}

}  // namespace
}  // namespace lkv

using namespace lkv;

extern "C" int lkv_rmsnorm(const void* x, const void* w, float eps, int64_t M, int64_t Z, void* y, void* stream) {
  LKV_REQUIRE(M >= 0 && Z > 0 && Z % 8 == 0 && Z < (1 << 30), "rmsnorm: Z=%lld must be a positive multiple of 8",
              (long long)Z);
  LKV_REQUIRE(M < 65536, "rmsnorm: M=%lld rows exceeds 65535", (long long)M);
  if (M == 0) return LKV_OK;
  LKV_REQUIRE(x && w && y && aligned16(x), "rmsnorm: null pointer or x not 16-byte aligned");
  const dim3 grid(static_cast<unsigned>((Z + kThreads - 1) / kThreads), static_cast<unsigned>(M));
  hipLaunchKernelGGL(rmsnorm_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), eps, static_cast<int>(Z),
                     static_cast<uint16_t*>(y));
  LKV_LAUNCH_CHECK("rmsnorm");
  return LKV_OK;
}

namespace lkv {
namespace {
// RoPE of B decode rows in place: q [B][Hq][128], k [B][Hkv][128] fp16 at one
// position (cos / sin: that position's 128 fp16 factors).  Thread = one dim
// pair (d, d + 64) of one head: rope_pair_v, the fp16 arithmetic of HF's
// apply_rotary_pos_emb.
__global__ __launch_bounds__(kThreads) void rope_f16_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                            const uint16_t* __restrict__ cos_row,
                                                            const uint16_t* __restrict__ sin_row, int rows_q,
                                                            int rows_k) {
  const int e = blockIdx.x * kThreads + threadIdx.x;  // (row, pair) over the q rows, then the k rows
  const int row = e / (kD / 2), d = e % (kD / 2);
  if (row >= rows_q + rows_k) return;
  uint16_t* x = row < rows_q ? q + static_cast<size_t>(row) * kD : k + static_cast<size_t>(row - rows_q) * kD;
  float o0, o1;
  rope_pair(h2f(x[d]), h2f(x[d + kD / 2]), cos_row, sin_row, d, o0, o1);
  x[d] = f2h(o0);
  x[d + kD / 2] = f2h(o1);
}
}  // namespace
}  // namespace lkv

extern "C" int lkv_rope_f16(void* q, void* k, const void* cos_row, const void* sin_row, int64_t B, int64_t Hq,
                            int64_t Hkv, void* stream) {
  LKV_REQUIRE(B >= 0 && Hq >= 0 && Hkv >= 0 && B * (Hq + Hkv) < (1ll << 24),
              "rope_f16: B=%lld Hq=%lld Hkv=%lld out of range", (long long)B, (long long)Hq, (long long)Hkv);
  const int64_t rows = B * (Hq + Hkv);
  if (rows == 0) return LKV_OK;
  LKV_REQUIRE(cos_row && sin_row && (q || B * Hq == 0) && (k || B * Hkv == 0), "rope_f16: null pointer");
  const unsigned grid = static_cast<unsigned>((rows * (kD / 2) + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(rope_f16_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint16_t*>(q), static_cast<uint16_t*>(k), static_cast<const uint16_t*>(cos_row),
                     static_cast<const uint16_t*>(sin_row), static_cast<int>(B * Hq), static_cast<int>(B * Hkv));
  LKV_LAUNCH_CHECK("rope_f16");
  return LKV_OK;
}

extern "C" size_t lkv_decode_workspace_bytes(const lkv_decode_dims* dims) {
  if (check_dims(dims) != LKV_OK) return 0;
  return make_plan(*dims).total;
}

extern "C" int lkv_decode_workspace_layout(const lkv_decode_dims* dims, lkv_decode_layout* out) {
  if (int e = check_dims(dims)) return e;
  LKV_REQUIRE(out != nullptr, "decode_workspace_layout: null output");
  const Plan p = make_plan(*dims);
  lkv_decode_layout l{};
  l.part_q = p.off_pqkv;
  l.part_k = l.part_q + gemv_part_floats(p.nq, p.nc_qkv) * 4;
  l.part_v = l.part_k + gemv_part_floats(p.nkv, p.nc_qkv) * 4;
  l.part_o = p.off_po;
  l.part_gate = p.off_pgu;
  l.part_up = p.off_pgu + gemv_part_floats(dims->ffn, p.nc_gu) * 4;
  l.part_down = p.off_pd;
  l.part_lm = p.off_plm;
  l.q_rope = p.off_q16;
  l.attn_out = p.off_attn;
  l.chunks_qkv = p.nc_qkv;
  l.chunks_o = p.nc_o;
  l.chunks_gateup = p.nc_gu;
  l.chunks_down = p.nc_d;
  l.chunks_lm = p.nc_lm;
  l.total = p.total;
  *out = l;
  return LKV_OK;
}

extern "C" int lkv_decode_begin(const lkv_decode_dims* dims, const void* embed, const int64_t* tok,
                                const int64_t* pos, void* x, void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_dims(dims)) return e;
  const Plan p = make_plan(*dims);
  if (int e = check_ws(p, workspace, workspace_bytes)) return e;
  LKV_REQUIRE(embed && tok && pos && x && aligned16(embed) && aligned16(x),
              "decode_begin: embed and x must be non-null and 16-byte aligned");
  char* ws = static_cast<char*>(workspace);
  const unsigned grid = static_cast<unsigned>((dims->hidden / 8 + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(begin_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(embed), tok, pos, static_cast<uint16_t*>(x),
                     reinterpret_cast<int32_t*>(ws + p.off_state), dims->hidden, dims->vocab, dims->max_len);
  LKV_LAUNCH_CHECK("decode_begin");
  return LKV_OK;
}

extern "C" int lkv_decode_evict(const lkv_decode_dims* dims, const lkv_decode_layer* layers, int64_t n_layers,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_dims(dims)) return e;
  const lkv_decode_dims& d = *dims;
  const Plan p = make_plan(d);
  if (int e = check_ws(p, workspace, workspace_bytes)) return e;
  LKV_REQUIRE(layers && n_layers >= 0, "decode_evict: null layer table or negative count");
  for (int64_t l = 0; l < n_layers; ++l) {
    const lkv_decode_layer& L = layers[l];
    LKV_REQUIRE(L.k_codes && L.k_norms && L.v_codes && L.v_norms && L.k_hot && L.v_hot && L.PiK && L.PiV,
                "decode_evict: null cache pointer in layer %lld", (long long)l);
    LKV_REQUIRE(aligned16(L.k_codes) && aligned16(L.v_codes) && aligned16(L.k_hot) && aligned16(L.v_hot) &&
                    aligned16(L.PiK) && aligned16(L.PiV),
                "decode_evict: cache buffers and rotations of layer %lld must be 16-byte aligned", (long long)l);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  for (int64_t l0 = 0; l0 < n_layers; l0 += kEvictLayers) {
    const int nl = static_cast<int>(n_layers - l0 < kEvictLayers ? n_layers - l0 : kEvictLayers);
    EvictArgs A{};
    A.state = reinterpret_cast<const int32_t*>(ws + p.off_state);
    A.bounds = d.bounds;
    A.hot_cap = static_cast<int>(d.hot_cap);
    A.cap = static_cast<int>(d.cap);
    A.Hkv = static_cast<int>(p.Hkv);
    for (int i = 0; i < nl; ++i) {
      const lkv_decode_layer& L = layers[l0 + i];
      A.L[i] = EvictLayer{static_cast<const uint16_t*>(L.k_hot), static_cast<const uint16_t*>(L.v_hot),
                          static_cast<uint8_t*>(L.k_codes),      static_cast<float*>(L.k_norms),
                          static_cast<uint8_t*>(L.v_codes),      static_cast<float*>(L.v_norms),
                          L.PiK,                                 L.PiV};
    }
    const dim3 grid(static_cast<unsigned>((p.Hkv + 15) / 16), 2, static_cast<unsigned>(nl));
    switch (d.bits) {
      case 1: hipLaunchKernelGGL((evict_kernel<1>), grid, dim3(kThreads), 0, st, A); break;
      case 2: hipLaunchKernelGGL((evict_kernel<2>), grid, dim3(kThreads), 0, st, A); break;
      case 3: hipLaunchKernelGGL((evict_kernel<3>), grid, dim3(kThreads), 0, st, A); break;
      default: hipLaunchKernelGGL((evict_kernel<4>), grid, dim3(kThreads), 0, st, A);
    }
    LKV_LAUNCH_CHECK("decode_evict");
  }
  return LKV_OK;
}

extern "C" int lkv_tq_cache_evict(const lkv_cache_layer* layers, int64_t n_layers, int64_t R, int64_t hot_cap,
                                  int64_t cap, const float* bounds, int bits, const int32_t* pos, void* stream) {
  LKV_REQUIRE(bits >= 1 && bits <= 4, "tq_cache_evict: bits=%d unsupported (1..4 are bit-packed)", bits);
  LKV_REQUIRE(n_layers >= 0 && R >= 0 && R < (1 << 24) && hot_cap >= 1 && hot_cap < (1 << 30) && cap >= 0 &&
                  cap < (1 << 30),
              "tq_cache_evict: bad sizes layers=%lld R=%lld hot_cap=%lld cap=%lld", (long long)n_layers,
              (long long)R, (long long)hot_cap, (long long)cap);
  if (n_layers == 0 || R == 0) return LKV_OK;
  LKV_REQUIRE(layers && bounds && pos, "tq_cache_evict: null pointer");
  for (int64_t l = 0; l < n_layers; ++l) {
    const lkv_cache_layer& L = layers[l];
    LKV_REQUIRE(L.k_codes && L.k_norms && L.v_codes && L.v_norms && L.k_hot && L.v_hot && L.PiK && L.PiV,
                "tq_cache_evict: null cache pointer in layer %lld", (long long)l);
    LKV_REQUIRE(aligned16(L.k_codes) && aligned16(L.v_codes) && aligned16(L.k_hot) && aligned16(L.v_hot) &&
                    aligned16(L.PiK) && aligned16(L.PiV),
                "tq_cache_evict: cache buffers and rotations of layer %lld must be 16-byte aligned", (long long)l);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int64_t l0 = 0; l0 < n_layers; l0 += kEvictLayers) {
    const int nl = static_cast<int>(n_layers - l0 < kEvictLayers ? n_layers - l0 : kEvictLayers);
    EvictArgs A{};
    A.state = pos;  // state[0]: the position of the token fed this step
    A.bounds = bounds;
    A.hot_cap = static_cast<int>(hot_cap);
    A.cap = static_cast<int>(cap);
    A.Hkv = static_cast<int>(R);  // the kernel's rows: (batch, kv head) pairs
    for (int i = 0; i < nl; ++i) {
      const lkv_cache_layer& L = layers[l0 + i];
      A.L[i] = EvictLayer{static_cast<const uint16_t*>(L.k_hot), static_cast<const uint16_t*>(L.v_hot),
                          static_cast<uint8_t*>(L.k_codes),      static_cast<float*>(L.k_norms),
                          static_cast<uint8_t*>(L.v_codes),      static_cast<float*>(L.v_norms),
                          L.PiK,                                 L.PiV};
    }
    const dim3 grid(static_cast<unsigned>((R + 15) / 16), 2, static_cast<unsigned>(nl));
    switch (bits) {
      case 1: hipLaunchKernelGGL((evict_kernel<1>), grid, dim3(kThreads), 0, st, A); break;
      case 2: hipLaunchKernelGGL((evict_kernel<2>), grid, dim3(kThreads), 0, st, A); break;
      case 3: hipLaunchKernelGGL((evict_kernel<3>), grid, dim3(kThreads), 0, st, A); break;
      default: hipLaunchKernelGGL((evict_kernel<4>), grid, dim3(kThreads), 0, st, A);
    }
    LKV_LAUNCH_CHECK("tq_cache_evict");
  }
  return LKV_OK;
}

namespace lkv {
namespace {

int check_layer_weights(const lkv_decode_layer* L, const void* x) {
  LKV_REQUIRE(L && x && aligned16(x), "decode_layer: null layer or unaligned x");
  LKV_REQUIRE(L->input_norm && L->post_norm && L->wq && L->wk && L->wv && L->wo && L->wg && L->wu && L->wd,
              "decode_layer: null weight");
  LKV_REQUIRE(aligned16(L->wq) && aligned16(L->wk) && aligned16(L->wv) && aligned16(L->wo) && aligned16(L->wg) &&
                  aligned16(L->wu) && aligned16(L->wd),
              "decode_layer: weights must be 16-byte aligned");
  return LKV_OK;
}

// 1. q|k|v: one GEMV launch over three segments, RMSNorm of x in the prologue.
int step_qkv(const Plan& p, const lkv_decode_dims& d, const lkv_decode_layer* L, const uint16_t* x, char* ws,
             hipStream_t st) {
  GemvArgs G{};
  G.x = x;
  G.norm_w = static_cast<const uint16_t*>(L->input_norm);
  G.eps = d.eps;
  G.nseg = 3;
  const void* w[3] = {L->wq, L->wk, L->wv};
  const int64_t n[3] = {p.nq, p.nkv, p.nkv};
  const float t[3] = {L->tq, L->tk, L->tv};
  size_t off = 0;
  int slab = 0;
  for (int s = 0; s < 3; ++s) {
    G.A[s] = static_cast<const uint16_t*>(w[s]);
    G.a_bytes[s] = static_cast<uint32_t>(d.hidden * n[s] * 2);
    G.N[s] = static_cast<int>(n[s]);
    G.t[s] = t[s];
    G.slab0[s] = slab;
    G.part_off[s] = off;
    slab += static_cast<int>(gemv_slabs(n[s]));
    off += gemv_part_floats(n[s], p.nc_qkv);
  }
  G.slab0[3] = slab;
  G.Z = static_cast<int>(d.hidden);
  G.nchunk = p.nc_qkv;
  G.part = reinterpret_cast<float*>(ws + p.off_pqkv);
  return gemv_launch(G, p.bz_qkv, false, kInRmsNorm, slab, st);
}

// 4-8. o_proj on the attention output, residual, gate|up (RMSNorm prologue),
// down (SwiGLU prologue), residual.
int step_tail(const Plan& p, const lkv_decode_dims& d, const lkv_decode_layer* L, uint16_t* xx, char* ws,
              hipStream_t st) {
  const int H = static_cast<int>(d.hidden);
  {
    GemvArgs G{};
    G.x = reinterpret_cast<const uint16_t*>(ws + p.off_attn);
    G.nseg = 1;
    G.A[0] = static_cast<const uint16_t*>(L->wo);
    G.a_bytes[0] = static_cast<uint32_t>(p.nq * d.hidden * 2);
    G.N[0] = H;
    G.t[0] = L->to;
    G.slab0[1] = static_cast<int>(p.sh);
    G.Z = static_cast<int>(p.nq);
    G.nchunk = p.nc_o;
    G.part = reinterpret_cast<float*>(ws + p.off_po);
    if (int e = gemv_launch(G, p.bz_o, false, kInRaw, static_cast<int>(p.sh), st)) return e;
    hipLaunchKernelGGL(residual_kernel, dim3(static_cast<unsigned>(p.sh)), dim3(kThreads), 0, st, xx, G.part, H,
                       p.nc_o);
    LKV_LAUNCH_CHECK("decode residual");
  }
  {
    GemvArgs G{};
    G.x = xx;
    G.norm_w = static_cast<const uint16_t*>(L->post_norm);
    G.eps = d.eps;
    G.nseg = 1;
    G.A[0] = static_cast<const uint16_t*>(L->wg);
    G.A_up = static_cast<const uint16_t*>(L->wu);
    G.a_bytes[0] = static_cast<uint32_t>(d.hidden * d.ffn * 2);
    G.N[0] = static_cast<int>(d.ffn);
    G.t[0] = L->tg;
    G.t_up = L->tu;
    G.slab0[1] = static_cast<int>(p.sf);
    G.Z = H;
    G.nchunk = p.nc_gu;
    G.part = reinterpret_cast<float*>(ws + p.off_pgu);
    G.part_up_off = gemv_part_floats(d.ffn, p.nc_gu);
    if (int e = gemv_launch(G, p.bz_gu, true, kInRmsNorm, static_cast<int>(p.sf), st)) return e;
  }
  {
    GemvArgs G{};
    G.in_part = reinterpret_cast<const float*>(ws + p.off_pgu);
    G.in_nslab = static_cast<int>(p.sf);
    G.in_nchunk = p.nc_gu;
    G.nseg = 1;
    G.A[0] = static_cast<const uint16_t*>(L->wd);
    G.a_bytes[0] = static_cast<uint32_t>(d.ffn * d.hidden * 2);
    G.N[0] = H;
    G.t[0] = L->td;
    G.slab0[1] = static_cast<int>(p.sh);
    G.Z = static_cast<int>(d.ffn);
    G.nchunk = p.nc_d;
    G.part = reinterpret_cast<float*>(ws + p.off_pd);
    if (int e = gemv_launch(G, p.bz_d, false, kInSwiglu, static_cast<int>(p.sh), st)) return e;
    hipLaunchKernelGGL(residual_kernel, dim3(static_cast<unsigned>(p.sh)), dim3(kThreads), 0, st, xx, G.part, H,
                       p.nc_d);
    LKV_LAUNCH_CHECK("decode residual");
  }
  return LKV_OK;
}

// 2-3. attention on the packed cache; the split kernel's prologue sums the
// q|k|v partials, applies RoPE, rotates the query and writes the new token's
// key and value into the ring.
int step_attn(const Plan& p, const lkv_decode_dims& d, const lkv_decode_layer* L, char* ws, hipStream_t st) {
  const int32_t* state = reinterpret_cast<const int32_t*>(ws + p.off_state);
  AttnCall c{};
  c.pq = reinterpret_cast<const float*>(ws + p.off_pqkv);
  c.pk = c.pq + gemv_part_floats(p.nq, p.nc_qkv);
  c.pv = c.pk + gemv_part_floats(p.nkv, p.nc_qkv);
  c.nchunk = p.nc_qkv;
  c.rope_cos = static_cast<const uint16_t*>(d.rope_cos);
  c.rope_sin = static_cast<const uint16_t*>(d.rope_sin);
  c.pos = state;
  c.q16 = reinterpret_cast<uint16_t*>(ws + p.off_q16);
  c.k_ring = static_cast<uint16_t*>(L->k_hot);
  c.v_ring = static_cast<uint16_t*>(L->v_hot);
  c.PiK = L->PiK;
  c.k_codes = static_cast<const uint8_t*>(L->k_codes);
  c.k_norms = static_cast<const float*>(L->k_norms);
  c.v_codes = static_cast<const uint8_t*>(L->v_codes);
  c.v_norms = static_cast<const float*>(L->v_norms);
  c.PiV = L->PiV;
  c.centroids = d.centroids;
  c.seq_len = state + 1;
  c.partials = reinterpret_cast<float*>(ws + p.off_rec);
  c.out = reinterpret_cast<uint16_t*>(ws + p.off_attn);
  c.scale = d.scale;
  c.max_len = d.max_len;
  c.B = 1;
  c.Hq = p.Hq;
  c.Hkv = p.Hkv;
  c.cap = d.cap;
  c.hot_cap = d.hot_cap;
  c.bits = d.bits;
  return attn_launch(c, p.attn, st);
}

}  // namespace
}  // namespace lkv

extern "C" int lkv_decode_layer_step(const lkv_decode_dims* dims, const lkv_decode_layer* L, void* x, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (int e = check_dims(dims)) return e;
  const lkv_decode_dims& d = *dims;
  const Plan p = make_plan(d);
  if (int e = check_ws(p, workspace, workspace_bytes)) return e;
  if (int e = check_layer_weights(L, x)) return e;
  LKV_REQUIRE(L->k_codes && L->k_norms && L->v_codes && L->v_norms && L->k_hot && L->v_hot && L->PiK && L->PiV,
              "decode_layer: null cache pointer");
  LKV_REQUIRE(aligned16(L->k_codes) && aligned16(L->v_codes) && aligned16(L->k_hot) && aligned16(L->v_hot) &&
                  aligned16(L->PiK) && aligned16(L->PiV),
              "decode_layer: cache buffers and rotations must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  uint16_t* xx = static_cast<uint16_t*>(x);
  if (int e = step_qkv(p, d, L, xx, ws, st)) return e;
  // 2-3. attention: the split kernel reduces the q|k|v partials itself (RoPE,
  // query rotation, the new key and value into the ring)
  if (int e = step_attn(p, d, L, ws, st)) return e;
  return step_tail(p, d, L, xx, ws, st);
}

extern "C" int lkv_decode_layer_step_f16kv(const lkv_decode_dims* dims, const lkv_decode_layer* L, void* kv_pool,
                                           void* x, void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_dims(dims)) return e;
  const lkv_decode_dims& d = *dims;
  const Plan p = make_plan(d);
  if (int e = check_ws(p, workspace, workspace_bytes)) return e;
  if (int e = check_layer_weights(L, x)) return e;
  LKV_REQUIRE(kv_pool && aligned16(kv_pool), "decode_layer_f16kv: null or unaligned kv pool");
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  uint16_t* xx = static_cast<uint16_t*>(x);
  if (int e = step_qkv(p, d, L, xx, ws, st)) return e;
  const float* pq = reinterpret_cast<const float*>(ws + p.off_pqkv);
  const float* pk = pq + gemv_part_floats(p.nq, p.nc_qkv);
  const float* pv = pk + gemv_part_floats(p.nkv, p.nc_qkv);
  if (p.Hq / p.Hkv <= 4) {  // one launch pair: the split kernel sums the partials itself
    F16kvStepAttn a{};
    a.pq = pq;
    a.pk = pk;
    a.pv = pv;
    a.nchunk = p.nc_qkv;
    a.rope_cos = static_cast<const uint16_t*>(d.rope_cos);
    a.rope_sin = static_cast<const uint16_t*>(d.rope_sin);
    a.pos = reinterpret_cast<const int32_t*>(ws + p.off_state);
    a.kv = static_cast<uint16_t*>(kv_pool);
    a.Hq = p.Hq;
    a.Hkv = p.Hkv;
    a.page_size = kF16Page;
    a.max_pages = p.f16_pages;
    a.max_len = d.max_len;
    a.scale = d.scale;
    a.out = reinterpret_cast<uint16_t*>(ws + p.off_attn);
    a.records = ws + p.off_prec;
    a.record_bytes = p.prec_bytes;
    if (int e = f16kv_step_attn(a, st)) return e;
    return step_tail(p, d, L, xx, ws, st);
  }
  // more than 4 query heads per kv head: epilogue kernel, then the paged call
  int32_t* pt = reinterpret_cast<int32_t*>(ws + p.off_pt);
  uint16_t* q16 = reinterpret_cast<uint16_t*>(ws + p.off_q16);
  const int items = static_cast<int>(p.nq / 2 + p.nkv);
  hipLaunchKernelGGL(f16kv_prep_kernel, dim3(static_cast<unsigned>((items + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, st, pq, pk, pv, p.nc_qkv, static_cast<const uint16_t*>(d.rope_cos),
                     static_cast<const uint16_t*>(d.rope_sin), reinterpret_cast<const int32_t*>(ws + p.off_state),
                     q16, static_cast<uint16_t*>(kv_pool), pt, static_cast<int>(p.nq), static_cast<int>(p.nkv),
                     static_cast<int>(p.Hkv));
  LKV_LAUNCH_CHECK("decode f16kv prep");
  if (int e = lkv_paged_decode_attn(q16, kv_pool, pt, pt + 3, pt + 2, 1, p.Hq, p.Hkv, kF16Page, p.f16_pages,
                                    d.max_len, d.scale, ws + p.off_attn, ws + p.off_prec, p.prec_bytes, stream))
    return e;
  return step_tail(p, d, L, xx, ws, st);
}

extern "C" int lkv_decode_head(const lkv_decode_dims* dims, const void* final_norm, const void* lm_head, const void* x,
                               void* logits, int64_t* tok, int64_t* pos, int64_t* tok_history,
                               int64_t history_len, void* workspace, size_t workspace_bytes, void* stream) {
  if (int e = check_dims(dims)) return e;
  const lkv_decode_dims& d = *dims;
  const Plan p = make_plan(d);
  if (int e = check_ws(p, workspace, workspace_bytes)) return e;
  LKV_REQUIRE(final_norm && lm_head && x && logits && tok && pos, "decode_head: null pointer");
  LKV_REQUIRE(tok_history != nullptr || history_len == 0, "decode_head: history_len without a history buffer");
  LKV_REQUIRE(aligned16(lm_head) && aligned16(x), "decode_head: lm_head and x must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  GemvArgs G{};
  G.x = static_cast<const uint16_t*>(x);
  G.norm_w = static_cast<const uint16_t*>(final_norm);
  G.eps = d.eps;
  G.nseg = 1;
  G.A[0] = static_cast<const uint16_t*>(lm_head);
  G.a_bytes[0] = static_cast<uint32_t>(d.hidden * d.vocab * 2);
  G.N[0] = static_cast<int>(d.vocab);
  G.t[0] = 0.f;
  G.slab0[1] = static_cast<int>(p.svoc);
  G.Z = static_cast<int>(d.hidden);
  G.nchunk = p.nc_lm;
  G.part = reinterpret_cast<float*>(ws + p.off_plm);
  if (int e = gemv_launch(G, p.bz_lm, false, kInRmsNorm, static_cast<int>(p.svoc), st)) return e;
  Cand* cand = reinterpret_cast<Cand*>(ws + p.off_cand);
  hipLaunchKernelGGL(logits_kernel, dim3(static_cast<unsigned>(p.svoc)), dim3(kThreads), 0, st, G.part,
                     static_cast<int>(d.vocab), p.nc_lm, static_cast<uint16_t*>(logits), cand);
  LKV_LAUNCH_CHECK("decode logits");
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kThreads), 0, st, cand, static_cast<int>(p.svoc), tok, pos,
                     tok_history, history_len);
  LKV_LAUNCH_CHECK("decode argmax");
  return LKV_OK;
}
