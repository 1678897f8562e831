// The decode step's layer tail as one persistent launch (B = 1).
//
// After a layer's attention, the reference runs (HF MistralDecoderLayer,
// transformers/models/mistral/modeling_mistral.py, with every projection a
// TEAL sparse GEMV, leankv/teal/patching.py:152-183):
//   x += o_proj(attn);  x += down(silu(gate(rms(x))) * up(rms(x)));
// and the next layer starts with q|k|v(rms(x)).  Launched one kernel per
// step, each of these GEMVs pays a fixed ~4 us of ramp-up, latency chain and
// drain on MI355X next to 3-20 us of streaming.  Here they run as the work
// items of one grid whose blocks all stay resident, in this order:
//
//   O   (slab, chunk)   o_proj partial sums of the attention output
//   R1  slab            x' = x + sum_chunks(O)                (fp16 residual)
//   GU  (slab, chunk)   gate|up partial sums of RMSNorm(x') * w_post
//   H   slab            h = SwiGLU(sum_chunks(gate), sum_chunks(up))
//   D   (slab, chunk)   down partial sums of h
//   R2  slab            x'' = x' + sum_chunks(D)
//   QKV (slab, chunk)   the next layer's q|k|v partial sums of RMSNorm(x'')
//
// Every item computes exactly what the per-launch step computes (the same
// chunking, gemv_core, chunk-ordered sums and fp16 roundings), so both paths
// give identical bits.  Block b takes items b, b + grid, b + 2 grid, ... in
// that global order; an item only waits on items earlier in the order, and
// all blocks are resident, so every wait ends (each waited-on item is held by
// a running block whose own waits are on still earlier items).  Waits are
// bounded anyway: past kSpinLimit polls the item records an error and goes on.
//
// Hand-off between items runs through tagged words: a 64-bit value holding a
// 32-bit payload (an fp32 partial sum, or two fp16) and a 32-bit tag naming
// the step and layer that wrote it, stored and loaded as relaxed agent-scope
// atomics.  Each such access is single-copy atomic and coherent across the
// XCDs' L2 caches on its own, so a consumer polls the words it needs until
// their tags match and then has the payload: no fence, no flag, no L2-wide
// write-back or invalidate (which cost far more than the launches they would
// save).  The epoch in the workspace state advances once per step
// (lkv_decode_begin), so a word written by an earlier step or layer never
// matches; the workspace starts zeroed (lkv_decode_workspace_init), and tag 0
// is never expected.  Data produced for the next launch (the q|k|v partials,
// the fp16 residual x) is also stored plainly: kernel boundaries order it.
#include "gemv_core.h"
#include "kernels.h"

namespace lkv {
namespace {

constexpr int kNT = kGemvThreads;  // 256 threads per block, every item kind
constexpr int kU = 8;              // rows per lane in flight (the standalone GEMV's)
constexpr int kCP = 2;             // non-temporal weight loads
// Polls before a wait gives up (each poll sleeps ~50 ns and waits one memory
// round trip: about a second in all); every 256 polls a waiting lane also
// checks the error word, so once one wait has given up the others stop too.
constexpr int kSpinLimit = 1 << 20;

__device__ __forceinline__ void tw_store(uint64_t* p, uint32_t payload, uint32_t tag) {
  __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tw_load(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t tw_tag(uint64_t v) { return static_cast<uint32_t>(v >> 32); }

// Words base[k * stride] for k < n (n <= K), polled in two halves so that a
// caller can have several groups in flight: tw_issue loads them once,
// tw_complete re-polls the ones whose tag does not match yet.
template <int K>
struct TwGroup {
  uint64_t v[K];
};
template <int K>
__device__ __forceinline__ void tw_issue(TwGroup<K>& g, const uint64_t* base, size_t stride, int n, uint32_t tag) {
#pragma unroll
  for (int k = 0; k < K; ++k) g.v[k] = k < n ? tw_load(base + k * stride) : static_cast<uint64_t>(tag) << 32;
}
template <int K>
__device__ __forceinline__ void tw_complete(TwGroup<K>& g, const uint64_t* base, size_t stride, int n, uint32_t tag,
                                            int32_t* err) {
  for (int spin = 0;; ++spin) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < K; ++k) ok = ok && tw_tag(g.v[k]) == tag;
    if (ok) break;
    if (spin >= kSpinLimit) {
      __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    if ((spin & 255) == 255 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
    __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k < n && tw_tag(g.v[k]) != tag) g.v[k] = tw_load(base + k * stride);
  }
}

__device__ __forceinline__ uint32_t pack_h2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}
__device__ __forceinline__ uint16_t h_lo(uint32_t w) { return static_cast<uint16_t>(w & 0xffffu); }
__device__ __forceinline__ uint16_t h_hi(uint32_t w) { return static_cast<uint16_t>(w >> 16); }

// rms_rstd (kernels.h) over the tagged fp16 pairs of x: the same loads, the
// same fmaf order per thread, the same wave and block reduction.
// The polled words are kept in s_xw (fp16 pairs of the whole vector) for the
// caller's normalisation, so x is read from memory once.
__device__ __forceinline__ float rms_rstd_tagged(const uint64_t* xt, int Z, float eps, uint32_t tag, float* s_wsum,
                                                 uint32_t* s_xw, int32_t* err) {
  const int tid = threadIdx.x;
  float ss = 0.f;
  for (int z = tid * 8; z < Z; z += kGemvThreads * 8) {
    TwGroup<4> g;
    tw_issue<4>(g, xt + z / 2, 1, 4, tag);
    tw_complete<4>(g, xt + z / 2, 1, 4, tag, err);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = static_cast<uint32_t>(g.v[i]);
      s_xw[z / 2 + i] = w;
      const float a = h2f(h_lo(w));
      const float b = h2f(h_hi(w));
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & (kWave - 1)) == 0) s_wsum[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kGemvThreads / kWave; ++w) tot += s_wsum[w];
  return rsqrtf(tot / static_cast<float>(Z) + eps);
}

template <int BZ>
using Lds1 = GemvLds<kNT, BZ, false, kU>;
template <int BZ>
using Lds2 = GemvLds<kNT, BZ, true, kU>;

union TailLds {
  Lds1<256> s256;
  Lds1<512> s512;
  Lds2<256> d256;
  Lds2<512> d512;
};

// One GEMV item: prologue fills sm.x, gemv_core, the caller stores sums.
// MODE: 0 = fp16 input (plain), 1 = RMSNorm of tagged x, 2 = tagged fp16 pairs (h).
template <int BZ, bool DUAL, int MODE>
__device__ __forceinline__ void tail_gemv(GemvLds<kNT, BZ, DUAL, kU>& sm, uint32_t* s_xw, const TailArgs& A,
                                          const uint16_t* xin, const uint64_t* xtag, uint32_t tag, const uint16_t* norm_w,
                                          const uint16_t* A0, const uint16_t* A1, uint32_t a_bytes, int N, float t0,
                                          float t1, int Z, int z0, int n0, float (&sums)[DUAL ? 2 : 1]) {
  constexpr int E = BZ / kNT;
  const int tid = threadIdx.x;
  if (MODE == 1) {
    const float rstd = rms_rstd_tagged(xtag, Z, A.eps, tag, sm.wsum, s_xw, A.err);  // ends with a barrier
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int z = z0 + e * kNT + tid;
      float v = 0.f;
      if (z < Z) {
        const uint32_t w = s_xw[z / 2];
        v = rms_apply((z & 1) ? h_hi(w) : h_lo(w), norm_w[z], rstd);
      }
      sm.x[e * kNT + tid] = v;
    }
  } else if (MODE == 2) {
    // the E inputs of this thread are words (z0 + tid) / 2 + 128 e
    const int zt = z0 + tid;
    const int n = zt < Z ? min(E, (Z - zt + kNT - 1) / kNT) : 0;
    TwGroup<E> g;
    tw_issue<E>(g, xtag + zt / 2, kNT / 2, n, tag);
    tw_complete<E>(g, xtag + zt / 2, kNT / 2, n, tag, A.err);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t w = static_cast<uint32_t>(g.v[e]);
      sm.x[e * kNT + tid] = e < n ? h2f((zt & 1) ? h_hi(w) : h_lo(w)) : 0.f;
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int z = z0 + e * kNT + tid;
      sm.x[e * kNT + tid] = z < Z ? h2f(xin[z]) : 0.f;
    }
  }
  __syncthreads();
  gemv_core<kNT, BZ, DUAL, kU, kCP>(sm, A0, A1, a_bytes, N, t0, t1, z0, Z, n0, sums);
}

// Residual item: columns n0 .. n0 + 256 of x_out = x_in + fp16(sum of the
// nchunk tagged partials of slab `slab`, in chunk order), one column per
// thread (every chunk polled at once, up to kResChunks per batch); lane pairs
// join their fp16 results into one tagged word.
constexpr int kResChunks = 32;
__device__ __forceinline__ void tail_residual(const TailArgs& A, int slab, const uint64_t* part, int nchunk,
                                              uint32_t part_tag, bool x_in_tagged, uint32_t x_in_tag,
                                              uint32_t x_out_tag, bool plain_out) {
  const int t = threadIdx.x;
  const int n = slab * kGemvBN + t;  // hidden is a multiple of 256: n < hidden
  const uint64_t* p0 = part + static_cast<size_t>(slab) * nchunk * kGemvBN + t;
  // the residual input first: its load overlaps the partials' polls
  uint32_t xw = 0;
  TwGroup<1> gx;
  if (x_in_tagged)
    tw_issue<1>(gx, A.xt + n / 2, 0, 1, x_in_tag);
  else
    xw = *reinterpret_cast<const uint32_t*>(A.x + (n & ~1));
  float s = 0.f;
  for (int c0 = 0; c0 < nchunk; c0 += kResChunks) {
    const int cnt = min(kResChunks, nchunk - c0);
    TwGroup<kResChunks> g;
    tw_issue<kResChunks>(g, p0 + static_cast<size_t>(c0) * kGemvBN, kGemvBN, cnt, part_tag);
    tw_complete<kResChunks>(g, p0 + static_cast<size_t>(c0) * kGemvBN, kGemvBN, cnt, part_tag, A.err);
#pragma unroll
    for (int i = 0; i < kResChunks; ++i)
      if (i < cnt) s += __uint_as_float(static_cast<uint32_t>(g.v[i]));
  }
  if (x_in_tagged) {
    tw_complete<1>(gx, A.xt + n / 2, 0, 1, x_in_tag, A.err);
    xw = static_cast<uint32_t>(gx.v[0]);
  }
  const uint16_t y = f2h(h2f((t & 1) ? h_hi(xw) : h_lo(xw)) + h2f(f2h(s)));
  const uint32_t other = static_cast<uint32_t>(__shfl_xor(static_cast<int>(y), 1));
  if ((t & 1) == 0) {
    const uint32_t yw = pack_h2(y, static_cast<uint16_t>(other));
    tw_store(A.xt + n / 2, yw, x_out_tag);
    if (plain_out) *reinterpret_cast<uint32_t*>(A.x + n) = yw;
  }
}

// SwiGLU item: h for columns n0 .. n0 + 256 of the ffn from the tagged gate
// and up partials (chunk-ordered sums, swiglu_f16), one column per thread.
constexpr int kGuChunks = 16;
__device__ __forceinline__ void tail_swiglu(const TailArgs& A, int slab, uint32_t tag) {
  const int t = threadIdx.x;
  const int n = slab * kGemvBN + t;  // ffn is a multiple of 256
  const int nc = A.nc_gu;
  const size_t mat = static_cast<size_t>(A.sf) * nc * kGemvBN;
  const uint64_t* p0 = A.pgu + static_cast<size_t>(slab) * nc * kGemvBN + t;
  float g = 0.f, u = 0.f;
  for (int c0 = 0; c0 < nc; c0 += kGuChunks) {
    const int cnt = min(kGuChunks, nc - c0);
    const uint64_t* pg = p0 + static_cast<size_t>(c0) * kGemvBN;
    TwGroup<kGuChunks> gg, gu;
    tw_issue<kGuChunks>(gg, pg, kGemvBN, cnt, tag);
    tw_issue<kGuChunks>(gu, pg + mat, kGemvBN, cnt, tag);
    tw_complete<kGuChunks>(gg, pg, kGemvBN, cnt, tag, A.err);
    tw_complete<kGuChunks>(gu, pg + mat, kGemvBN, cnt, tag, A.err);
#pragma unroll
    for (int i = 0; i < kGuChunks; ++i) {
      if (i < cnt) {
        g += __uint_as_float(static_cast<uint32_t>(gg.v[i]));
        u += __uint_as_float(static_cast<uint32_t>(gu.v[i]));
      }
    }
  }
  const uint16_t h = swiglu_f16(g, u);
  const uint32_t other = static_cast<uint32_t>(__shfl_xor(static_cast<int>(h), 1));
  if ((t & 1) == 0) tw_store(A.ph + n / 2, pack_h2(h, static_cast<uint16_t>(other)), tag);
}

__device__ __forceinline__ void store_tagged_sums(uint64_t* part, int slab, int chunk, int nchunk, float v,
                                                  uint32_t tag) {
  if (threadIdx.x < kGemvBN)
    tw_store(part + (static_cast<size_t>(slab) * nchunk + chunk) * kGemvBN + threadIdx.x, __float_as_uint(v), tag);
}

template <int BZ>
__device__ __forceinline__ void item_o(TailLds& U, uint32_t* s_xw, const TailArgs& A, int i, uint32_t tag) {
  const int slab = i % A.sh, chunk = i / A.sh;
  float s[1];
  tail_gemv<BZ, false, 0>(BZ == 256 ? reinterpret_cast<Lds1<BZ>&>(U.s256) : reinterpret_cast<Lds1<BZ>&>(U.s512), s_xw,
                          A,
                          A.attn, nullptr, 0, nullptr, A.wo, nullptr, A.wo_bytes, A.hidden, A.t_o, 0.f, A.nq,
                          chunk * BZ, slab * kGemvBN, s);
  store_tagged_sums(A.po, slab, chunk, A.nc_o, s[0], tag);
}

template <int BZ>
__device__ __forceinline__ void item_gu(TailLds& U, uint32_t* s_xw, const TailArgs& A, int i, uint32_t tag_x,
                                        uint32_t tag) {
  const int slab = i % A.sf, chunk = i / A.sf;
  float s[2];
  tail_gemv<BZ, true, 1>(BZ == 256 ? reinterpret_cast<Lds2<BZ>&>(U.d256) : reinterpret_cast<Lds2<BZ>&>(U.d512), s_xw,
                         A,
                         nullptr, A.xt, tag_x, A.post_norm, A.wg, A.wu, A.wgu_bytes, A.ffn, A.t_g, A.t_u, A.hidden,
                         chunk * BZ, slab * kGemvBN, s);
  store_tagged_sums(A.pgu, slab, chunk, A.nc_gu, s[0], tag);
  store_tagged_sums(A.pgu + static_cast<size_t>(A.sf) * A.nc_gu * kGemvBN, slab, chunk, A.nc_gu, s[1], tag);
}

template <int BZ>
__device__ __forceinline__ void item_d(TailLds& U, uint32_t* s_xw, const TailArgs& A, int i, uint32_t tag) {
  const int slab = i % A.sh, chunk = i / A.sh;
  float s[1];
  tail_gemv<BZ, false, 2>(BZ == 256 ? reinterpret_cast<Lds1<BZ>&>(U.s256) : reinterpret_cast<Lds1<BZ>&>(U.s512), s_xw,
                          A,
                          nullptr, A.ph, tag, nullptr, A.wd, nullptr, A.wd_bytes, A.hidden, A.t_d, 0.f, A.ffn,
                          chunk * BZ, slab * kGemvBN, s);
  store_tagged_sums(A.pd, slab, chunk, A.nc_d, s[0], tag);
}

template <int BZ>
__device__ __forceinline__ void item_qkv(TailLds& U, uint32_t* s_xw, const TailArgs& A, int i, uint32_t tag_x) {
  const int nslab = A.sq + 2 * A.sk;
  const int gslab = i % nslab, chunk = i / nslab;
  const int seg = gslab < A.sq ? 0 : (gslab < A.sq + A.sk ? 1 : 2);
  const int slab = gslab - (seg == 0 ? 0 : (seg == 1 ? A.sq : A.sq + A.sk));
  const uint16_t* W = seg == 0 ? A.wq : (seg == 1 ? A.wk : A.wv);
  const int N = seg == 0 ? A.nq : A.nkv;
  const float t = seg == 0 ? A.tq : (seg == 1 ? A.tk : A.tv);
  float s[1];
  tail_gemv<BZ, false, 1>(BZ == 256 ? reinterpret_cast<Lds1<BZ>&>(U.s256) : reinterpret_cast<Lds1<BZ>&>(U.s512), s_xw,
                          A,
                          nullptr, A.xt, tag_x, A.in_norm, W, nullptr, static_cast<uint32_t>(N) * A.hidden * 2u, N, t,
                          0.f, A.hidden, chunk * BZ, slab * kGemvBN, s);
  if (threadIdx.x < kGemvBN) {
    float* P = A.pqkv + (seg == 0 ? 0 : (seg == 1 ? A.pk_off : A.pv_off)) +
               (static_cast<size_t>(slab) * A.nc_qkv + chunk) * kGemvBN;
    P[threadIdx.x] = s[0];
  }
}

__global__ __launch_bounds__(kNT) void decode_tail_kernel(TailArgs A) {
  __shared__ TailLds U;
  __shared__ uint32_t s_xw[kTailMaxHidden / 2];
  const uint32_t epoch = static_cast<uint32_t>(A.state[2]);
  const uint32_t base = epoch * static_cast<uint32_t>(A.n_layers) + static_cast<uint32_t>(A.layer);
  const uint32_t tag = 2u * base, tag2 = 2u * base + 1u;  // tag2: x after the second residual
  for (int gi = blockIdx.x; gi < A.pre[7]; gi += gridDim.x) {
    if (gi < A.pre[1]) {
      const int i = gi;
      if (A.bz_o == 256) item_o<256>(U, s_xw, A, i, tag); else item_o<512>(U, s_xw, A, i, tag);
    } else if (gi < A.pre[2]) {
      tail_residual(A, gi - A.pre[1], A.po, A.nc_o, tag, false, 0, tag, false);
    } else if (gi < A.pre[3]) {
      const int i = gi - A.pre[2];
      if (A.bz_gu == 256) item_gu<256>(U, s_xw, A, i, tag, tag); else item_gu<512>(U, s_xw, A, i, tag, tag);
    } else if (gi < A.pre[4]) {
      tail_swiglu(A, gi - A.pre[3], tag);
    } else if (gi < A.pre[5]) {
      const int i = gi - A.pre[4];
      if (A.bz_d == 256) item_d<256>(U, s_xw, A, i, tag); else item_d<512>(U, s_xw, A, i, tag);
    } else if (gi < A.pre[6]) {
      tail_residual(A, gi - A.pre[5], A.pd, A.nc_d, tag, true, tag, tag2, true);
    } else {
      const int i = gi - A.pre[6];
      if (A.bz_qkv == 256) item_qkv<256>(U, s_xw, A, i, tag2); else item_qkv<512>(U, s_xw, A, i, tag2);
    }
    __syncthreads();  // LDS is reused by the next item
  }
}

}  // namespace

int tail_blocks_per_cu() {
  static const int k = [] {
    const char* env = getenv("LKV_TAIL_BLOCKS_PER_CU");
    const int v = env ? atoi(env) : 2;
    return v >= 1 && v <= 8 ? v : 2;
  }();
  return k;
}

int tail_launch(const TailArgs& A, hipStream_t st) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_tail_kernel, kNT, 0) != hipSuccess || per_cu < 1) {
    set_error("decode_tail: occupancy query failed");
    return LKV_ERR_HIP;
  }
  const int want = tail_blocks_per_cu();
  const int64_t resident = static_cast<int64_t>(per_cu < want ? per_cu : want) * device_cu_count();
  const int64_t grid = A.pre[7] < resident ? A.pre[7] : resident;
  if (grid <= 0) return LKV_OK;
  hipLaunchKernelGGL(decode_tail_kernel, dim3(static_cast<unsigned>(grid)), dim3(kNT), 0, st, A);
  LKV_LAUNCH_CHECK("decode_tail");
  return LKV_OK;
}

}  // namespace lkv
