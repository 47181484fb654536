// Sliding-window GQA attention for the uTTT blocks on gfx950 (MI355X):
//   * k_rope_append  -- RoPE on q (in place) and k, append rotated k and v to a KV buffer
//   * k_swa_prefill  -- flash-style attention: 64 queries per workgroup, 64-key LDS tiles,
//                       only the key tiles that intersect the window are visited
//   * k_swa_decode   -- one token per request over a ring-buffer KV cache
// Visibility rule (reference model/uttt_layer.py:1028-1037): query at absolute key index p
// sees key j iff 0 <= p - j < window; kv head = h / (n_heads / n_kv_heads).
#include <math.h>

#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {

// ---------------------------------------------------------------------------
// 16x16 MFMA wave tiles (used by attention)
//   fp32: v_mfma_f32_16x16x4f32      (K = 4, lane supplies A[l%16][k0 + l/16])
//   bf16: v_mfma_f32_16x16x32_bf16   (K = 32, lane supplies A[l%16][k0 + 8*(l/16) + 0..7])
//   result: acc[i] = C[4*(l/16) + i][l%16]
// ---------------------------------------------------------------------------
template <typename T> struct Mma16;
template <> struct Mma16<float> {
  static constexpr int kK = 4;
  static constexpr int kPad = 4;  // rows stay 16-byte aligned
  __device__ __forceinline__ static void step(f32x4& acc, const float* a_row, const float* b_row, int k0, int g) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a_row[k0 + g], b_row[k0 + g], acc, 0, 0, 0);
  }
};
template <> struct Mma16<bf16> {
  static constexpr int kK = 32;
  static constexpr int kPad = 8;
  __device__ __forceinline__ static void step(f32x4& acc, const bf16* a_row, const bf16* b_row, int k0, int g) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(a_row + k0 + 8 * g);
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(b_row + k0 + 8 * g);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
};

// acc(16x16) += A(16 x KTOT) B(KTOT x 16); A rows at `a` ([16][lda]), B^T rows at `b` ([16][ldb])
template <typename T, int KTOT>
__device__ __forceinline__ void wave_mma16(f32x4& acc, const T* a, int lda, const T* b, int ldb) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const T* a_row = a + r * lda;
  const T* b_row = b + r * ldb;
#pragma unroll
  for (int k0 = 0; k0 < KTOT; k0 += Mma16<T>::kK) Mma16<T>::step(acc, a_row, b_row, k0, g);
}

// RoPE for one element pair, rounding like the reference's activation-dtype ops:
// out_lo = x_lo*cos - x_hi*sin, out_hi = x_hi*cos + x_lo*sin (model/uttt_layer.py:946-958).
template <typename T>
__device__ __forceinline__ void rope_pair(float x_lo, float x_hi, float c, float s, T& out_lo, T& out_hi) {
#pragma clang fp contract(off)
  const float cr = to_f32(from_f32<T>(c)), sr = to_f32(from_f32<T>(s));
  const float a0 = to_f32(from_f32<T>(x_lo * cr)), b0 = to_f32(from_f32<T>(-x_hi * sr));
  const float a1 = to_f32(from_f32<T>(x_hi * cr)), b1 = to_f32(from_f32<T>(x_lo * sr));
  out_lo = from_f32<T>(a0 + b0);
  out_hi = from_f32<T>(a1 + b1);
}

// ---------------------------------------------------------------------------
// RoPE + KV append: grid (tokens, batch)
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kThreads) k_rope_append(const uttt_rope_append_args a) {
  const int t = blockIdx.x, b = blockIdx.y;
  const int hd = (int)a.head_dim, half = hd / 2;
  const int64_t pos = a.start_pos + t;
  const float* cr = a.cos_table + pos * hd;
  const float* sr = a.sin_table + pos * hd;
  T* q = static_cast<T*>(a.q) + b * a.q_stride_b + t * a.q_stride_t;
  const T* k = static_cast<const T*>(a.k) + b * a.k_stride_b + t * a.k_stride_t;
  const T* v = static_cast<const T*>(a.v) + b * a.v_stride_b + t * a.v_stride_t;
  T* kc = static_cast<T*>(a.k_cache) + b * a.kv_stride_b + (a.kv_offset + t) * a.kv_stride_t;
  T* vc = static_cast<T*>(a.v_cache) + b * a.kv_stride_b + (a.kv_offset + t) * a.kv_stride_t;
  // folded input norm: q, k and v of the token scale by 1 / rms of its input row
  float xs = 1.0f;
  if (a.x != nullptr) {
    __shared__ float red[4];
    const T* xr = static_cast<const T*>(a.x) + b * a.x_stride_b + t * a.x_stride_t;
    float ss = 0.f;
    for (int i = threadIdx.x; i < a.x_dim; i += kThreads) {
      const float xv = to_f32(xr[i]);
      ss += xv * xv;
    }
    xs = 1.0f / sqrtf(block_sum(ss, red) / (float)a.x_dim + a.x_eps);
  }
  const int nq = (int)a.n_heads * half;
  for (int idx = threadIdx.x; idx < nq; idx += kThreads) {
    const int h = idx / half, e = idx - h * half;
    T* qh = q + h * a.q_stride_h;
    T lo, hi;
    rope_pair<T>(xs * to_f32(qh[e]), xs * to_f32(qh[e + half]), cr[e], sr[e], lo, hi);
    qh[e] = lo;
    qh[e + half] = hi;
  }
  const int nk = (int)a.n_kv_heads * half;
  for (int idx = threadIdx.x; idx < nk; idx += kThreads) {
    const int h = idx / half, e = idx - h * half;
    const T* kh = k + h * a.k_stride_h;
    T lo, hi;
    rope_pair<T>(xs * to_f32(kh[e]), xs * to_f32(kh[e + half]), cr[e], sr[e], lo, hi);
    kc[h * a.kv_stride_h + e] = lo;
    kc[h * a.kv_stride_h + e + half] = hi;
  }
  const int nv = (int)a.n_kv_heads * hd;
  for (int idx = threadIdx.x; idx < nv; idx += kThreads) {
    const int h = idx / hd, e = idx - h * hd;
    const T vv = v[h * a.v_stride_h + e];
    vc[h * a.kv_stride_h + e] = a.x != nullptr ? from_f32<T>(xs * to_f32(vv)) : vv;
  }
}

// ---------------------------------------------------------------------------
// Prefill.  grid (q tiles of 64, n_heads, batch * nsplit): the key tiles that intersect a
// q tile's window are divided among `nsplit` workgroups; each wave owns 16 queries.  With
// nsplit > 1 the workgroups write fp32 partials (row max, row sum, unnormalised output)
// and k_swa_prefill_combine merges them.  Q / K rows are staged with 16-byte loads, V is
// transposed in registers to [e][key]; the next key tile is loaded while the current one
// is consumed.
// ---------------------------------------------------------------------------
template <typename T, int HD>
struct AttnStage {
  static constexpr int kVec = 16 / (int)sizeof(T);
  static constexpr int kChunksPerRow = HD / kVec;
  static constexpr int kRowChunks = 64 * kChunksPerRow / kThreads;  // per thread, for a 64-row tile
  static constexpr int kVUnits = 8 * kChunksPerRow;                 // 8 keys x one chunk per unit
  uint4 kr[kRowChunks];
  uint4 vr[8];

  // Branch-free: rows at or past n lie outside the buffer ranges and read as zeros, so the loads
  // carry no condition and the compiler has no reason to wait for them before the current tile's
  // work (a conditional load made it wait for every outstanding load right away).
  __device__ __forceinline__ void load(const T* k, const T* v, int64_t st_k, int64_t st_v, int n) {
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(k, (uint32_t)(max(n, 0) * st_k * (int64_t)sizeof(T)));
    const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(v, (uint32_t)(max(n, 0) * st_v * (int64_t)sizeof(T)));
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kChunksPerRow, c = idx - row * kChunksPerRow;
      kr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rk, (int)((row * st_k + c * kVec) * (int64_t)sizeof(T)), 0, 0));
    }
    if (threadIdx.x < kVUnits) {
      const int kg = threadIdx.x / kChunksPerRow, c = threadIdx.x - kg * kChunksPerRow;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = kg * 8 + i;
        vr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rv, (int)((row * st_v + c * kVec) * (int64_t)sizeof(T)), 0, 0));
      }
    }
  }
  template <int LQ, int LV>
  __device__ __forceinline__ void store(T* ks, T* vt) const {
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kChunksPerRow, c = idx - row * kChunksPerRow;
      *reinterpret_cast<uint4*>(ks + row * LQ + c * kVec) = kr[j];
    }
    if (threadIdx.x < kVUnits) {
      const int kg = threadIdx.x / kChunksPerRow, c = threadIdx.x - kg * kChunksPerRow;
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        T* d = vt + (c * kVec + e) * LV + kg * 8;
        if constexpr (sizeof(T) == 2) {
          bf16x8 o;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(Lanes16<bf16>::get(vr[i], e));
          *reinterpret_cast<bf16x8*>(d) = o;
        } else {
          f32x4 o0, o1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            o0[i] = Lanes16<float>::get(vr[i], e);
            o1[i] = Lanes16<float>::get(vr[i + 4], e);
          }
          *reinterpret_cast<f32x4*>(d) = o0;
          *reinterpret_cast<f32x4*>(d + 4) = o1;
        }
      }
    }
  }
};

struct PrefillPlan {
  int nqt, nsplit, tiles_per_split, q_pad;
};

constexpr int kMaxPrefillSplits = 16;

__host__ __device__ __forceinline__ int prefill_max_tiles(int64_t kv_len, int64_t window) {
  const int64_t span = min(kv_len, window + 63);
  return (int)((span + 63) / 64) + 1;
}

static PrefillPlan prefill_plan(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len, int64_t window) {
  PrefillPlan p;
  p.nqt = (int)((q_len + 63) / 64);
  p.q_pad = p.nqt * 64;
  const int64_t base = (int64_t)p.nqt * heads * batch;
  const int max_tiles = prefill_max_tiles(kv_len, window);
  // about 256 workgroups (one per CU): in the chunk-first prefill the attention shares the GPU
  // with the layer chain, and at config 3 (64 workgroups before the split) 256 measured faster
  // than 128, 192, 320 or 512 workgroups (prefill 552-556 against 554-561 ms on one box)
  int64_t ns = (256 + base - 1) / base;
  if (ns > max_tiles) ns = max_tiles;
  if (ns > kMaxPrefillSplits) ns = kMaxPrefillSplits;
  if (ns < 1) ns = 1;
  p.tiles_per_split = (max_tiles + (int)ns - 1) / (int)ns;
  p.nsplit = (max_tiles + p.tiles_per_split - 1) / p.tiles_per_split;
  return p;
}

// Reductions over the 16 lanes of a DPP row (the lanes that share a query row of a 16 x 16 score
// block): rotations by 8, 4, 2 and 1 within the row leave every lane with the row's result.  They
// run as VALU operations with DPP operands, where cross-lane shuffles (ds_bpermute) would make
// each step an LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kRowRor8 = 0x128, kRowRor4 = 0x124, kRowRor2 = 0x122, kRowRor1 = 0x121;  // DPP row_ror:n
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_row<kRowRor8>(v));
  v = fmaxf(v, dpp_row<kRowRor4>(v));
  v = fmaxf(v, dpp_row<kRowRor2>(v));
  return fmaxf(v, dpp_row<kRowRor1>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_row<kRowRor8>(v);
  v += dpp_row<kRowRor4>(v);
  v += dpp_row<kRowRor2>(v);
  return v + dpp_row<kRowRor1>(v);
}
// e^x for the softmax weights (x <= 0) through the hardware base-2 exponential:
// e^x = 2^(x log2 e); relative error about |x| 2^-23 from the product's rounding, far inside the
// fp32 and bf16 tolerances of the attention output
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

template <typename T, int HD>
__global__ void __launch_bounds__(kThreads) k_swa_prefill(const uttt_swa_prefill_args a, float* part, int nsplit,
                                                          int tiles_per_split, int q_pad, int nqt) {
  constexpr int PAD = Mma16<T>::kPad;
  constexpr int LQ = HD + PAD;   // q/k rows [token][e]
  constexpr int LV = 64 + PAD;   // v^T rows [e][key], p rows [query][key]
  __shared__ __align__(16) T qs[64 * LQ];
  __shared__ __align__(16) T ks[64 * LQ];
  __shared__ __align__(16) T vt[HD * LV];
  __shared__ __align__(16) T ps[64 * LV];
  // the workgroups of one (row, kv head) read the same keys and values: they are placed as the
  // tiles of one row (row_tile), split fastest, then the query heads of the kv head, then q tiles
  const int rep = (int)(a.n_heads / a.n_kv_heads);
  const RowTile rt = row_tile(blockIdx.x, (int)(a.batch * a.n_kv_heads), nqt * rep * nsplit);
  if (!rt.valid) return;
  const int b = rt.b / (int)a.n_kv_heads, kvh = rt.b - b * (int)a.n_kv_heads;
  const int sp = rt.tile % nsplit, qt = rt.tile / (nsplit * rep);
  const int h = kvh * rep + (rt.tile / nsplit) % rep;
  const int q0 = qt * 64;
  const int qn = (int)min((int64_t)64, a.q_len - q0);
  const int64_t p_first = a.q_offset + q0, p_last = a.q_offset + q0 + qn - 1;
  const int64_t lo = max((int64_t)0, p_first - a.window + 1);
  const int64_t hi = min(a.kv_len, p_last + 1);  // exclusive
  const int ntiles = (int)((hi - lo + 63) / 64);
  const int t_begin = sp * tiles_per_split, t_end = min(ntiles, t_begin + tiles_per_split);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  float* pr = part + ((((int64_t)b * a.n_heads + h) * nsplit + sp) * q_pad + q0) * (HD + 2);
  if (t_begin >= t_end) {  // nothing in this split's range (only with nsplit > 1)
    for (int idx = threadIdx.x; idx < 64; idx += kThreads) {
      pr[idx * (HD + 2)] = -INFINITY;
      pr[idx * (HD + 2) + 1] = 0.f;
    }
    return;
  }

  const T* qg = static_cast<const T*>(a.q) + b * a.q_stride_b + h * a.q_stride_h;
  const T* kg = static_cast<const T*>(a.k) + b * a.k_stride_b + kvh * a.k_stride_h;
  const T* vg = static_cast<const T*>(a.v) + b * a.v_stride_b + kvh * a.v_stride_h;
  {
    constexpr int kVec = 16 / (int)sizeof(T), kCpr = HD / kVec;
    for (int idx = threadIdx.x; idx < 64 * kCpr; idx += kThreads) {
      const int r = idx / kCpr, cc = idx - r * kCpr;
      *reinterpret_cast<uint4*>(qs + r * LQ + cc * kVec) =
          r < qn ? *reinterpret_cast<const uint4*>(qg + (q0 + r) * a.q_stride_t + cc * kVec) : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  float m_run[4], l_run[4];
  f32x4 o[HD / 16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < HD / 16; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  AttnStage<T, HD> stg;
  {
    const int64_t kt0 = lo + (int64_t)t_begin * 64;
    stg.load(kg + kt0 * a.k_stride_t, vg + kt0 * a.v_stride_t, a.k_stride_t, a.v_stride_t,
             (int)min((int64_t)64, hi - kt0));
  }
  for (int kt = t_begin; kt < t_end; ++kt) {
    const int64_t kt0 = lo + (int64_t)kt * 64;
    __syncthreads();  // previous tile fully consumed
    stg.template store<LQ, LV>(ks, vt);
    __syncthreads();
    if (kt + 1 < t_end) {
      const int64_t nx = kt0 + 64;
      stg.load(kg + nx * a.k_stride_t, vg + nx * a.v_stride_t, a.k_stride_t, a.v_stride_t,
               (int)min((int64_t)64, hi - nx));
    }

    // S = Q K^T for this wave's 16 queries x 64 keys (4 tiles of 16 keys)
    f32x4 s[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      wave_mma16<T, HD>(s[n], qs + (16 * w) * LQ, LQ, ks + (16 * n) * LQ, LQ);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qi = q0 + 16 * w + 4 * g + i;
      const int64_t p = a.q_offset + qi;
      float mx = -INFINITY;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int64_t key = kt0 + 16 * n + c;
        const bool vis = qi < a.q_len && key < hi && p - key >= 0 && p - key < a.window;
        const float val = vis ? s[n][i] * a.scale : -INFINITY;
        s[n][i] = val;
        mx = fmaxf(mx, val);
      }
      mx = row16_max(mx);
      const float m_new = fmaxf(m_run[i], mx);
      const float corr = m_new == -INFINITY ? 1.f : exp_fast(m_run[i] - m_new);
      float rs = 0.f;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float pv = s[n][i] == -INFINITY ? 0.f : exp_fast(s[n][i] - m_new);
        s[n][i] = pv;
        rs += pv;
      }
      rs = row16_sum(rs);
      l_run[i] = l_run[i] * corr + rs;
      m_run[i] = m_new;
#pragma unroll
      for (int t = 0; t < HD / 16; ++t) o[t][i] *= corr;
#pragma unroll
      for (int n = 0; n < 4; ++n) ps[(16 * w + 4 * g + i) * LV + 16 * n + c] = from_f32<T>(s[n][i]);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < HD / 16; ++t) wave_mma16<T, 64>(o[t], ps + (16 * w) * LV, LV, vt + (16 * t) * LV, LV);
  }

  if (nsplit == 1) {
    T* og = static_cast<T*>(a.out) + b * a.o_stride_b + h * a.o_stride_h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qi = q0 + 16 * w + 4 * g + i;
      if (qi >= a.q_len) continue;
      const float inv = l_run[i] > 0.f ? 1.0f / l_run[i] : 0.f;
#pragma unroll
      for (int t = 0; t < HD / 16; ++t) og[(int64_t)qi * a.o_stride_t + 16 * t + c] = from_f32<T>(o[t][i] * inv);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + 4 * g + i;
      float* row = pr + r * (HD + 2);
      if (c == 0) {
        row[0] = m_run[i];
        row[1] = l_run[i];
      }
#pragma unroll
      for (int t = 0; t < HD / 16; ++t) row[2 + 16 * t + c] = o[t][i];
    }
  }
}

// grid (q_pad * HD / (256 * kCombineEpt), n_heads, batch): kCombineEpt consecutive output
// elements of one query row per thread, their partials read with 8-byte loads; the split
// partials of a row are loaded together (at most kMaxPrefillSplits).  (One element per thread
// took 2048 workgroups at the config-3 chunk shape and 18 us per call beside the layer chain,
// 6.6 us alone.)
constexpr int kCombineEpt = 4;

template <typename T, int HD>
__global__ void __launch_bounds__(kThreads) k_swa_prefill_combine(const uttt_swa_prefill_args a, const float* part,
                                                                  int nsplit, int q_pad) {
  static_assert(HD % kCombineEpt == 0, "a thread's elements lie in one row");
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const int h = blockIdx.y, b = blockIdx.z;
  const int idx = (blockIdx.x * kThreads + threadIdx.x) * kCombineEpt;
  const int qi = idx / HD, e = idx - qi * HD;
  if (qi >= a.q_len) return;
  const float* base = part + (((int64_t)b * a.n_heads + h) * nsplit) * q_pad * (HD + 2) + (int64_t)qi * (HD + 2);
  const int64_t sstride = (int64_t)q_pad * (HD + 2);
  float m[kMaxPrefillSplits], l[kMaxPrefillSplits];
  f32x2 o[kMaxPrefillSplits][2];
#pragma unroll
  for (int s = 0; s < kMaxPrefillSplits; ++s) {
    if (s < nsplit) {
      const float* row = base + s * sstride;  // rows of HD + 2 floats: the output pieces are 8-byte aligned
      m[s] = row[0];
      l[s] = row[1];
      o[s][0] = *reinterpret_cast<const f32x2*>(row + 2 + e);
      o[s][1] = *reinterpret_cast<const f32x2*>(row + 4 + e);
    } else {
      m[s] = -INFINITY;
      l[s] = 0.f;
      o[s][0] = o[s][1] = f32x2{0.f, 0.f};
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxPrefillSplits; ++s) mx = fmaxf(mx, m[s]);
  float num[kCombineEpt] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
  if (mx != -INFINITY) {
#pragma unroll
    for (int s = 0; s < kMaxPrefillSplits; ++s) {
      // a split with no visible key leaves its output partial unwritten: skip it, do not scale it
      if (m[s] != -INFINITY) {
        const float f = expf(m[s] - mx);
        den += l[s] * f;
#pragma unroll
        for (int u = 0; u < kCombineEpt; ++u) num[u] += o[s][u >> 1][u & 1] * f;
      }
    }
  }
  T* og = static_cast<T*>(a.out) + b * a.o_stride_b + h * a.o_stride_h + (int64_t)qi * a.o_stride_t + e;
#pragma unroll
  for (int u = 0; u < kCombineEpt; ++u) og[u] = from_f32<T>(den > 0.f ? num[u] / den : 0.f);
}

// ---------------------------------------------------------------------------
// Decode, split over the window: k_swa_decode_part handles kDecodeKeys ring slots of one
// (request, kv head) and writes softmax partials (max, sum, unnormalised output) per
// query head; k_swa_decode_combine merges the splits.  Lanes cooperate on a key row with
// 16-byte loads (HD/8 lanes per key).
// ---------------------------------------------------------------------------
constexpr int kDecodeKeys = 64;
constexpr int kMaxRep = 8;

__host__ __device__ __forceinline__ int decode_splits(int64_t window) {
  return (int)((window + kDecodeKeys - 1) / kDecodeKeys);
}

template <typename T>
__device__ __forceinline__ void unpack8(float (&dst)[8], const uint4* v) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = Lanes16<bf16>::get(v[0], i);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dst[i] = Lanes16<float>::get(v[0], i);
      dst[i + 4] = Lanes16<float>::get(v[1], i);
    }
  }
}

// grid (n_req, n_kv_heads, splits of KEYS slots), NT threads: softmax partials per split for
// k_swa_decode_combine (the general form: any window, head_dim 64 or 128, up to kMaxRep query
// heads per kv head, bf16 or fp32).
template <typename T, int HD, int NT = kThreads, int KEYS = kDecodeKeys, int REP = kMaxRep>
__global__ void __launch_bounds__(NT) k_swa_decode_part(const uttt_swa_decode_args a, float* part) {
  constexpr int L = HD / 8;                  // lanes per key row (8 elements each)
  constexpr int KPP = NT / L;                // keys per pass
  constexpr int PASSES = KEYS / KPP;         // split form: 2 (HD 64) or 4 (HD 128)
  constexpr int CH = sizeof(T) == 2 ? 1 : 2; // 16-byte chunks per 8 elements
  constexpr int NW = NT / 64;                // waves
  constexpr int KPL = (KEYS + 63) / 64;      // scores per lane in the softmax
  static_assert(PASSES * KPP == KEYS, "the passes must cover the keys");
  __shared__ float qf[REP * HD];
  __shared__ float knew[HD], vnew[HD];
  __shared__ float sc[REP * KEYS];
  __shared__ float wred[NW][REP * HD];
  __shared__ float stat[REP][2];
  const int n = blockIdx.x, kvh = blockIdx.y, sp = blockIdx.z;
  const int rep = (int)(a.n_heads / a.n_kv_heads);
  const int nsplit = gridDim.z;
  const int64_t W = a.window;
  const int64_t pos = a.positions[n];
  if (pos < 0 || (a.cos_table != nullptr && pos >= a.table_len)) return;  // the combine writes NaN
  const int64_t slot = pos % W;
  const int valid = (int)min(pos + 1, W);
  const int j_lo = sp * KEYS, j_hi = min(valid, j_lo + KEYS);
  float* pr = part + (((int64_t)n * a.n_kv_heads + kvh) * nsplit + sp) * rep * (HD + 2);
  if (j_lo >= j_hi) {
    for (int idx = threadIdx.x; idx < rep * (HD + 2); idx += NT) {
      const int e = idx % (HD + 2);
      pr[idx] = e == 0 ? -INFINITY : 0.f;
    }
    return;
  }
  T* kr = static_cast<T*>(a.k_ring) + n * a.ring_stride_n + (int64_t)kvh * W * HD;
  T* vr = static_cast<T*>(a.v_ring) + n * a.ring_stride_n + (int64_t)kvh * W * HD;
  const int sub = threadIdx.x % L, grp = threadIdx.x / L;
  const int e0 = sub * 8;
  // every K / V load of this thread first (the slot being written is read from LDS instead)
  uint4 kraw[PASSES][CH], vraw[PASSES][CH];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int j = j_lo + grp + p * KPP;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool ld = j < j_hi && j != slot;
      kraw[p][c] = ld ? *reinterpret_cast<const uint4*>(kr + (int64_t)j * HD + e0 + c * (8 / CH)) : make_uint4(0u, 0u, 0u, 0u);
      vraw[p][c] = ld ? *reinterpret_cast<const uint4*>(vr + (int64_t)j * HD + e0 + c * (8 / CH)) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  const T* qg = static_cast<const T*>(a.q) + n * a.q_stride_n + (int64_t)kvh * rep * HD;
  const T* kn = static_cast<const T*>(a.k_new) + n * a.kv_new_stride_n + (int64_t)kvh * HD;
  const T* vn = static_cast<const T*>(a.v_new) + n * a.kv_new_stride_n + (int64_t)kvh * HD;
  const bool owns_slot = slot >= j_lo && slot < j_hi;
  constexpr int half = HD / 2;
  // RoPE (activation-dtype rounding as the reference); the split holding the slot writes the ring
  for (int idx = threadIdx.x; idx < (rep + 1) * half; idx += NT) {
    const int r = idx / half, e = idx - r * half;
    const T* src = r < rep ? qg + r * HD : kn;
    T lo = src[e], hi = src[e + half];
    if (a.cos_table != nullptr)
      rope_pair<T>(to_f32(lo), to_f32(hi), a.cos_table[pos * HD + e], a.sin_table[pos * HD + e], lo, hi);
    if (r < rep) {
      qf[r * HD + e] = to_f32(lo);
      qf[r * HD + e + half] = to_f32(hi);
    } else {
      knew[e] = to_f32(lo);
      knew[e + half] = to_f32(hi);
      if (owns_slot) {
        kr[slot * HD + e] = lo;
        kr[slot * HD + e + half] = hi;
      }
    }
  }
  for (int e = threadIdx.x; e < HD; e += NT) {
    const T v = vn[e];
    vnew[e] = to_f32(v);
    if (owns_slot) vr[slot * HD + e] = v;
  }
  __syncthreads();

#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int j = j_lo + grp + p * KPP;
    float kv[8];
    if (j == slot) {
#pragma unroll
      for (int i = 0; i < 8; ++i) kv[i] = knew[e0 + i];
    } else {
      unpack8<T>(kv, kraw[p]);
    }
    float acc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      float s = 0.f;
      if (r < rep) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s += qf[r * HD + e0 + i] * kv[i];
#pragma unroll
        for (int off = 1; off < L; off <<= 1) s += __shfl_xor(s, off, 64);
      }
      acc[r] = s;
    }
    if (sub == 0 && j < j_hi) {
#pragma unroll
      for (int r = 0; r < REP; ++r)
        if (r < rep) sc[r * KEYS + (j - j_lo)] = acc[r] * a.scale;
    }
  }
  __syncthreads();
  const int cnt = j_hi - j_lo;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = wave; r < rep; r += NW) {
    float v0[KPL];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < KPL; ++t) {
      const int jj = lane + 64 * t;
      v0[t] = jj < cnt ? sc[r * KEYS + jj] : -INFINITY;
      mx = fmaxf(mx, v0[t]);
    }
    mx = wave_max(mx);
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < KPL; ++t) {
      const int jj = lane + 64 * t;
      const float p0 = jj < cnt ? expf(v0[t] - mx) : 0.f;
      if (jj < cnt) sc[r * KEYS + jj] = p0;
      psum += p0;
    }
    const float sum = wave_sum(psum);
    if (lane == 0) {
      stat[r][0] = mx;
      stat[r][1] = sum;
    }
  }
  __syncthreads();
  float o[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int i = 0; i < 8; ++i) o[r][i] = 0.f;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int j = j_lo + grp + p * KPP;
    if (j >= j_hi) continue;
    float vv[8];
    if (j == slot) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vv[i] = vnew[e0 + i];
    } else {
      unpack8<T>(vv, vraw[p]);
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      if (r < rep) {
        const float pw = sc[r * KEYS + (j - j_lo)];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[r][i] += pw * vv[i];
      }
    }
  }
  // reduce the key groups of a wave (lanes with equal sub), then across the waves
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    if (r < rep) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int off = L; off < 64; off <<= 1) o[r][i] += __shfl_xor(o[r][i], off, 64);
      }
    }
  }
  if (lane < L) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      if (r < rep) {
#pragma unroll
        for (int i = 0; i < 8; ++i) wred[wave][r * HD + e0 + i] = o[r][i];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rep * HD; idx += NT) {
    const int r = idx / HD, e = idx - r * HD;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) v += wred[q][idx];
    pr[r * (HD + 2) + 2 + e] = v;
    if (e == 0) {
      pr[r * (HD + 2)] = stat[r][0];
      pr[r * (HD + 2) + 1] = stat[r][1];
    }
  }
}

constexpr int kMaxDecodeSplits = 64;
constexpr int kPieceKeys = 128;

template <int CTRL>
__device__ __forceinline__ float dpp_rot(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// max / sum over each 32-lane half of the wave (row rotations within 16 lanes, then across the
// two 16-lane rows of the half)
__device__ __forceinline__ float half_max(float v) {
  v = fmaxf(v, dpp_rot<0x128>(v));
  v = fmaxf(v, dpp_rot<0x124>(v));
  v = fmaxf(v, dpp_rot<0x122>(v));
  v = fmaxf(v, dpp_rot<0x121>(v));
  return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ float half_sum(float v) {
  v += dpp_rot<0x128>(v);
  v += dpp_rot<0x124>(v);
  v += dpp_rot<0x122>(v);
  v += dpp_rot<0x121>(v);
  return v + __shfl_xor(v, 16, 64);
}


// bf16 decode with head_dim 64, windows up to kWindowWaves x kPieceKeys slots and up to 4 query
// heads per kv head: one workgroup per (request, kv head), wave w taking ring slots
// [128 w, 128 w + 128).  A wave's K rows (a row tile: k = head dim along the row) and V rows
// (token slabs: k = slot down the rows) go straight from the ring into LDS (buffer loads with
// the lds bit; slots past the valid ones read as zeros), the slot written this step is replaced
// there by the new (RoPE'd) key and value, and both products run on MFMA with the query heads as
// the rows of a 32-row A operand (rows past the heads zero): S = Q K^T over the wave's 128
// slots, the softmax row statistics over DPP row rotations, P (bf16) = exp(S - max), O = P V.
// The four waves' partials (max, sum, unnormalised O per head) meet in LDS.  LDS: each wave's K
// and V rows (32 KB), the shared query tile (rows 0-31 of a row tile, 4 KB), each wave's P for 64
// slots at a time (4 KB), the partials (4.2 KB): 152 KB, one workgroup per CU.  Measured at the
// config-4 shape: 8.5 us per call, against 12.4 us for the same products split over one-wave
// workgroups whose partials a last workgroup merged through device-coherent stores, a counter
// and loads (4.5 us of round trips), and 14.4 us for that split with 8 lanes per key row and
// cross-lane reductions.
constexpr int kWindowWaves = 4;

__global__ void __launch_bounds__(kWindowWaves * 64) k_swa_decode_window(const uttt_swa_decode_args a) {
  constexpr int HD = 64, KEYS = kPieceKeys, NW = kWindowWaves;
  __shared__ __align__(1024) bf16 kv[NW][4][64 * 64];  // per wave: K slots 0-63, 64-127, V slots 0-63, 64-127
  __shared__ __align__(1024) bf16 qt[32 * 64];          // query rows 0-31 of a row tile
  __shared__ __align__(1024) bf16 pt[NW][32 * 64];      // per wave: P rows 0-31 for 64 slots
  __shared__ float red[NW][4][HD + 2];                  // per wave and head (<= 4): max, sum, O row
  const int n = blockIdx.x, kvh = blockIdx.y;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int rep = (int)(a.n_heads / a.n_kv_heads);
  const int64_t W = a.window;
  const int j_lo = w * KEYS;
  const int span = (int)max((int64_t)0, min(W - j_lo, (int64_t)KEYS));  // ring slots of this wave's piece
  bf16* kr = static_cast<bf16*>(a.k_ring) + n * a.ring_stride_n + (int64_t)kvh * W * HD;
  bf16* vr = static_cast<bf16*>(a.v_ring) + n * a.ring_stride_n + (int64_t)kvh * W * HD;
  // this wave's K / V rows into LDS, issued before the request's position is known (rows past the
  // ring read as zeros; value rows of slots not yet valid are cleared after the loads land)
  const uint32_t k0 = lds_addr(&kv[w][0][0]), v0 = lds_addr(&kv[w][2][0]);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rows = min(max(span - 64 * h, 0), 64);
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kr + (int64_t)(j_lo + 64 * h) * HD, (uint32_t)(rows * HD * 2));
    const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(vr + (int64_t)(j_lo + 64 * h) * HD, (uint32_t)(rows * HD * 2));
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      buffer_load_lds_raw(rk, lds_ptr(k0 + (uint32_t)(h * 8192 + g * 1024)), 16, row_src_off(g, lane, HD), 0, 0, 0);
      buffer_load_lds_raw(rv, lds_ptr(v0 + (uint32_t)(h * 8192 + g * 1024)), 16, slab_src_off(g, lane, HD), 0, 0, 0);
    }
  }
  const int64_t pos = a.positions[n];
  bf16* og = static_cast<bf16*>(a.out) + n * a.o_stride_n + (int64_t)kvh * rep * HD;
  if (pos < 0 || (a.cos_table != nullptr && pos >= a.table_len)) {  // loud NaN output, cache untouched
    for (int idx = threadIdx.x; idx < rep * HD; idx += NW * 64) og[idx] = from_f32<bf16>(NAN);
    wait_vmcnt<0>();  // no LDS write of this workgroup's loads outlives it
    return;
  }
  const int64_t slot = pos % W;
  const int valid = (int)min(pos + 1, W);
  const int cnt = max(0, min(valid, j_lo + KEYS) - j_lo);  // this wave's valid slots
  // rows past the query heads of the query tile are zero (rows 0 .. rep-1 are written below,
  // so no barrier is needed between the two writes)
  if (threadIdx.x >= rep * 8) reinterpret_cast<uint4*>(qt)[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
  // RoPE of the query heads (wave 0 writes them) and of the new key (kept by the wave whose piece
  // holds this step's slot, which writes the ring)
  const bf16* qg = static_cast<const bf16*>(a.q) + n * a.q_stride_n + (int64_t)kvh * rep * HD;
  const bf16* kn = static_cast<const bf16*>(a.k_new) + n * a.kv_new_stride_n + (int64_t)kvh * HD;
  const bf16* vn = static_cast<const bf16*>(a.v_new) + n * a.kv_new_stride_n + (int64_t)kvh * HD;
  const bool owns_slot = slot >= j_lo && slot < j_lo + cnt;
  const int ts = (int)(slot - j_lo);
  constexpr int half = HD / 2;
  bf16 knew[2] = {bf16{}, bf16{}}, vnew_v = bf16{};
  if (w == 0 || owns_slot) {
    const int e = lane & (half - 1);
    const float c = a.cos_table != nullptr ? a.cos_table[pos * HD + e] : 1.f;
    const float sn = a.cos_table != nullptr ? a.sin_table[pos * HD + e] : 0.f;
    for (int r = lane >> 5; r <= rep; r += 2) {  // lanes 0-31 even rows, 32-63 odd rows; row rep: the key
      if (r < rep && w != 0) continue;
      const bf16* src = r < rep ? qg + r * HD : kn;
      bf16 lo = src[e], hi = src[e + half];
      if (a.cos_table != nullptr) rope_pair<bf16>(to_f32(lo), to_f32(hi), c, sn, lo, hi);
      if (r < rep) {
        qt[r * 64 + (((e >> 3) ^ row_swz(r)) << 3) + (e & 7)] = lo;
        qt[r * 64 + ((((e + half) >> 3) ^ row_swz(r)) << 3) + (e & 7)] = hi;
      } else if (owns_slot) {
        knew[0] = lo;
        knew[1] = hi;
      }
    }
    if (owns_slot) vnew_v = vn[lane];
  }
  const bool key_lane = ((rep & 1) == 0) == (lane < 32);  // the half of the wave that took row rep
  wait_vmcnt<0>();  // this wave's K / V rows have landed in LDS
  // value rows of slots not yet valid: zeros (their weights are zero, and 0 x NaN would not be);
  // key rows there are masked out of the scores by selection.  A piece with no valid slot is
  // left out of the merge.
  if (cnt > 0 && cnt < span) {
    for (int i = lane; i < (span - cnt) * 8; i += 64) {
      const int t = cnt + (i >> 3);
      reinterpret_cast<uint4*>(&kv[w][2 + (t >> 6)][(t & 63) * 64])[i & 7] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  if (owns_slot) {  // this step's slot: the new key and value replace what the ring held
    // the ring writes go out after the wait (the vector memory counter counts stores too, so
    // issued earlier they would sit on the wait), and after every load of this piece
    if (key_lane) {
      const int e = lane & (half - 1);
      kr[slot * HD + e] = knew[0];
      kr[slot * HD + e + half] = knew[1];
    }
    vr[slot * HD + lane] = vnew_v;
    const int h = ts >> 6, t = ts & 63;
    bf16* krow = &kv[w][h][t * 64];
    bf16* vrow = &kv[w][2 + h][t * 64];
    if (key_lane) {
      const int e = lane & (half - 1);
      krow[(((e >> 3) ^ row_swz(t)) << 3) + (e & 7)] = knew[0];
      krow[((((e + half) >> 3) ^ row_swz(t)) << 3) + (e & 7)] = knew[1];
    }
    vrow[(((lane >> 3) ^ slab_swz(t)) << 3) + (lane & 7)] = vnew_v;
  }
  __syncthreads();  // the query tile and the replaced slot rows before the fragment reads
  // S = Q K^T over this wave's 128 slots (4 column tiles of 32), k = head dim in 4 steps of 16
  const uint32_t q0 = lds_addr(qt), p0 = lds_addr(&pt[w][0]);
  bf16x8 fq[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) fq[k] = lds_read_bf16x8<0>(row_frag_addr(q0, 0, lane, k));
  f32x16 sacc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    bf16x8 fk[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      fk[k] = lds_read_bf16x8<0>(row_frag_addr(k0 + (uint32_t)((t >> 1) * 8192), 32 * (t & 1), lane, k));
    lds_wait_frags(fq, fk);
    zero(sacc[t]);
#pragma unroll
    for (int k = 0; k < 4; ++k) sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fq[k], fk[k], sacc[t], 0, 0, 0);
  }
  // head r < 4 sits in element r of lanes 0-31 (slot 32 t + lane of tile t); lanes 32-63 hold
  // padding rows and go through the same steps harmlessly.  An empty piece has every slot masked:
  // its weights are zero and its partial is left out of the merge.
  const float scale2 = a.scale * 1.4426950408889634f;  // scores in log2 units
  float mx[4], sum[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = 32 * t + (lane & 31);
      sacc[t][r] = j < cnt ? sacc[t][r] * scale2 : -INFINITY;
      m = fmaxf(m, sacc[t][r]);
    }
    mx[r] = half_max(m);
  }
  f32x16 oacc[2];
  zero(oacc[0]);
  zero(oacc[1]);
#pragma unroll
  for (int r = 0; r < 4; ++r) sum[r] = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // P for slots 64 h .. 64 h + 63, then O += P V over them
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * h + tt;
        const float pf = mx[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sacc[t][r] - mx[r]);
        const bf16 pb = from_f32<bf16>(pf);
        sum[r] += to_f32(pb);
        if (lane < 32 && r < rep) {
          const int c = 32 * tt + lane;
          pt[w][r * 64 + (((c >> 3) ^ row_swz(r)) << 3) + (c & 7)] = pb;
        } else if (lane < 32) {
          const int c = 32 * tt + lane;
          pt[w][r * 64 + (((c >> 3) ^ row_swz(r)) << 3) + (c & 7)] = bf16{};
        }
      }
    }
    if (h == 0) {  // rows 4-31 of P stay zero
#pragma unroll
      for (int i = 0; i < 3; ++i)
        reinterpret_cast<uint4*>(&pt[w][4 * 64])[lane + 64 * i] = make_uint4(0u, 0u, 0u, 0u);
      if (lane < 32) reinterpret_cast<uint4*>(&pt[w][4 * 64])[lane + 192] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();  // the P writes before the fragment reads
    bf16x8 fp[4], fv0[4], fv1[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) fp[k] = lds_read_bf16x8<0>(row_frag_addr(p0, 0, lane, k));
    slab_frags(slab_tr_addr(v0 + (uint32_t)(h * 8192), 0, lane), fv0);
    slab_frags(slab_tr_addr(v0 + (uint32_t)(h * 8192), 32, lane), fv1);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fp[0]), "+v"(fp[1]), "+v"(fp[2]), "+v"(fp[3]), "+v"(fv0[0]), "+v"(fv0[1]), "+v"(fv0[2]),
                   "+v"(fv0[3]), "+v"(fv1[0]), "+v"(fv1[1]), "+v"(fv1[2]), "+v"(fv1[3]));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      oacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp[k], fv0[k], oacc[0], 0, 0, 0);
      oacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp[k], fv1[k], oacc[1], 0, 0, 0);
    }
    __syncthreads();  // every wave's P reads are done before its P tile is rewritten
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) sum[r] = half_sum(sum[r]);
  if (lane < 32) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r < rep) {
        red[w][r][2 + lane] = oacc[0][r];
        red[w][r][2 + 32 + lane] = oacc[1][r];
        if (lane == 0) {
          red[w][r][0] = cnt > 0 ? mx[r] : -INFINITY;  // log2 units
          red[w][r][1] = sum[r];
        }
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rep * HD; idx += NW * 64) {
    const int r = idx / HD, e = idx - r * HD;
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) m = fmaxf(m, red[u][r][0]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      if (red[u][r][0] != -INFINITY) {
        const float f = __builtin_amdgcn_exp2f(red[u][r][0] - m);
        den += red[u][r][1] * f;
        num += red[u][r][2 + e] * f;
      }
    }
    og[idx] = from_f32<bf16>(num / den);
  }
}


// grid (n_req, n_kv_heads): one output element per thread, splits loaded together
template <typename T, int HD>
__global__ void __launch_bounds__(kThreads) k_swa_decode_combine(const uttt_swa_decode_args a, const float* part,
                                                                 int nsplit) {
  const int n = blockIdx.x, kvh = blockIdx.y;
  const int rep = (int)(a.n_heads / a.n_kv_heads);
  const int64_t pos = a.positions[n];
  T* og = static_cast<T*>(a.out) + n * a.o_stride_n + (int64_t)kvh * rep * HD;
  const bool bad = pos < 0 || (a.cos_table != nullptr && pos >= a.table_len);
  const float* pr = part + ((int64_t)n * a.n_kv_heads + kvh) * nsplit * rep * (HD + 2);
  const int used = bad ? 0 : (int)((min(pos + 1, a.window) + kDecodeKeys - 1) / kDecodeKeys);
  for (int idx = threadIdx.x; idx < rep * HD; idx += kThreads) {
    if (bad) {  // position outside the RoPE table: loud NaN output, cache untouched
      og[idx] = from_f32<T>(NAN);
      continue;
    }
    const int r = idx / HD, e = idx - r * HD;
    float m[16], l[16], o[16];
    float mx = -INFINITY, num = 0.f, den = 0.f;
    for (int s0 = 0; s0 < used; s0 += 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int s = s0 + k;
        const float* q = pr + (s * rep + r) * (HD + 2);
        m[k] = s < used ? q[0] : -INFINITY;
        l[k] = s < used ? q[1] : 0.f;
        o[k] = s < used ? q[2 + e] : 0.f;
      }
      float cm = -INFINITY;
#pragma unroll
      for (int k = 0; k < 16; ++k) cm = fmaxf(cm, m[k]);
      const float nm = fmaxf(mx, cm);
      const float scale_old = mx == -INFINITY ? 0.f : expf(mx - nm);
      num *= scale_old;
      den *= scale_old;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (m[k] != -INFINITY) {
          const float f = expf(m[k] - nm);
          den += l[k] * f;
          num += o[k] * f;
        }
      }
      mx = nm;
    }
    og[idx] = from_f32<T>(num / den);
  }
}

template <typename T, int HD>
static void launch_prefill(const uttt_swa_prefill_args& a, const PrefillPlan& p, hipStream_t st) {
  float* part = static_cast<float*>(a.workspace);
  const dim3 grid((unsigned)row_tile_blocks((int)(a.batch * a.n_kv_heads), p.nqt * (int)(a.n_heads / a.n_kv_heads) * p.nsplit));
  hipLaunchKernelGGL((k_swa_prefill<T, HD>), grid, dim3(kThreads), 0, st, a, part, p.nsplit, p.tiles_per_split,
                     p.q_pad, p.nqt);
  if (p.nsplit > 1)
    hipLaunchKernelGGL((k_swa_prefill_combine<T, HD>),
                       dim3((unsigned)((int64_t)p.q_pad * HD / (kThreads * kCombineEpt)), (unsigned)a.n_heads,
                            (unsigned)a.batch),
                       dim3(kThreads), 0, st, a, (const float*)part, p.nsplit, p.q_pad);
}

// k_swa_decode_window's reach: bf16 rings of up to 512 slots, head_dim 64, at most 4 query
// heads per kv head; otherwise the split form and its combine launch
constexpr int kWindowSlots = kWindowWaves * kPieceKeys, kWindowRep = 4;

inline size_t decode_partial_bytes(int64_t n_req, int64_t n_heads, int64_t head_dim, int64_t window) {
  return align_up(sizeof(float) * (size_t)n_req * (size_t)n_heads * (size_t)decode_splits(window) *
                  (size_t)(head_dim + 2));
}

template <typename T, int HD>
static void launch_decode(const uttt_swa_decode_args& a, hipStream_t st) {
  if constexpr (sizeof(T) == 2 && HD == 64) {
    if (a.window <= kWindowSlots && a.n_heads / a.n_kv_heads <= kWindowRep) {
      hipLaunchKernelGGL(k_swa_decode_window, dim3((unsigned)a.n_req, (unsigned)a.n_kv_heads), dim3(kWindowWaves * 64),
                         0, st, a);
      return;
    }
  }
  const int nsplit = decode_splits(a.window);
  float* part = static_cast<float*>(a.workspace);
  hipLaunchKernelGGL((k_swa_decode_part<T, HD>), dim3((unsigned)a.n_req, (unsigned)a.n_kv_heads, (unsigned)nsplit),
                     dim3(kThreads), 0, st, a, part);
  hipLaunchKernelGGL((k_swa_decode_combine<T, HD>), dim3((unsigned)a.n_req, (unsigned)a.n_kv_heads), dim3(kThreads), 0,
                     st, a, (const float*)part, nsplit);
}

}  // namespace uttt

using namespace uttt;

extern "C" int uttt_rope_kv_append(const uttt_rope_append_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->batch >= 1 && a->batch <= 65535 && a->tokens >= 1, "batch/tokens out of range");
  UTTT_REQUIRE(a->head_dim >= 2 && a->head_dim % 2 == 0, "head_dim must be even");
  UTTT_REQUIRE(a->n_heads >= 1 && a->n_kv_heads >= 1, "head counts must be >= 1");
  UTTT_REQUIRE(a->start_pos >= 0 && a->start_pos + a->tokens <= a->table_len,
               "positions [%lld, %lld) exceed the RoPE table (%lld rows)", (long long)a->start_pos,
               (long long)(a->start_pos + a->tokens), (long long)a->table_len);
  UTTT_REQUIRE(a->cos_table && a->sin_table && a->q && a->k && a->v && a->k_cache && a->v_cache,
               "pointers must be non-NULL");
  UTTT_REQUIRE(a->kv_offset >= 0, "kv_offset must be >= 0");
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_F32 || a->act_dtype == UTTT_DTYPE_BF16, "bad act_dtype");
  UTTT_REQUIRE(a->x == nullptr || (a->x_dim >= 1 && a->x_eps > 0.f), "a folded norm needs x_dim >= 1 and x_eps > 0");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)a->tokens, (unsigned)a->batch);
  if (a->act_dtype == UTTT_DTYPE_BF16)
    hipLaunchKernelGGL(k_rope_append<bf16>, grid, dim3(kThreads), 0, st, *a);
  else
    hipLaunchKernelGGL(k_rope_append<float>, grid, dim3(kThreads), 0, st, *a);
  return launch_status("uttt_rope_kv_append");
}

extern "C" size_t uttt_swa_prefill_workspace(int64_t batch, int64_t n_heads, int64_t q_len, int64_t kv_len,
                                             int64_t head_dim, int64_t window) {
  if (batch < 1 || n_heads < 1 || q_len < 1 || kv_len < 1 || window < 1 || head_dim < 1) return 0;
  const PrefillPlan p = prefill_plan(batch, n_heads, q_len, kv_len, window);
  if (p.nsplit == 1) return 16;
  return sizeof(float) * (size_t)p.nsplit * (size_t)batch * (size_t)n_heads * (size_t)p.q_pad * (size_t)(head_dim + 2);
}

extern "C" int uttt_swa_prefill(const uttt_swa_prefill_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->head_dim == 64 || a->head_dim == 128, "head_dim must be 64 or 128 (got %lld)", (long long)a->head_dim);
  UTTT_REQUIRE(a->batch >= 1 && a->n_heads >= 1 && a->n_heads <= 65535, "batch / n_heads out of range");
  UTTT_REQUIRE(a->n_kv_heads >= 1 && a->n_heads % a->n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
  UTTT_REQUIRE(a->q_len >= 1 && a->kv_len >= 1 && a->window >= 1, "q_len, kv_len and window must be >= 1");
  UTTT_REQUIRE(a->q_offset >= 0 && a->q_offset + a->q_len <= a->kv_len,
               "queries must index keys inside [0, kv_len): q_offset %lld + q_len %lld > kv_len %lld",
               (long long)a->q_offset, (long long)a->q_len, (long long)a->kv_len);
  UTTT_REQUIRE(a->q && a->k && a->v && a->out, "pointers must be non-NULL");
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_F32 || a->act_dtype == UTTT_DTYPE_BF16, "bad act_dtype");
  const int64_t vec = a->act_dtype == UTTT_DTYPE_BF16 ? 8 : 4;
  UTTT_REQUIRE(aligned16(a->q) && aligned16(a->k) && aligned16(a->v), "q/k/v must be 16-byte aligned");
  UTTT_REQUIRE(a->q_stride_b % vec == 0 && a->q_stride_h % vec == 0 && a->q_stride_t % vec == 0 &&
               a->k_stride_b % vec == 0 && a->k_stride_h % vec == 0 && a->k_stride_t % vec == 0 &&
               a->v_stride_b % vec == 0 && a->v_stride_h % vec == 0 && a->v_stride_t % vec == 0,
               "q/k/v strides must be multiples of 16 bytes");
  UTTT_REQUIRE(a->k_stride_t >= a->head_dim && a->v_stride_t >= a->head_dim &&
                   a->k_stride_t * 64 * 4 <= 0x7fffffffLL && a->v_stride_t * 64 * 4 <= 0x7fffffffLL,
               "k/v token strides must cover a row and fit a 64-row buffer range");
  const PrefillPlan p = prefill_plan(a->batch, a->n_heads, a->q_len, a->kv_len, a->window);
  UTTT_REQUIRE(a->batch * p.nsplit <= 65535 && a->batch * a->n_heads * p.nqt * p.nsplit + 8LL * a->n_heads <= 0x7fffffffLL,
               "batch too large for the attention grid");
  UTTT_REQUIRE(p.nsplit == 1 || (a->workspace != nullptr &&
                                 a->workspace_bytes >= uttt_swa_prefill_workspace(a->batch, a->n_heads, a->q_len,
                                                                                  a->kv_len, a->head_dim, a->window)),
               "attention workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool b16 = a->act_dtype == UTTT_DTYPE_BF16;
  if (a->head_dim == 64) {
    if (b16) launch_prefill<bf16, 64>(*a, p, st); else launch_prefill<float, 64>(*a, p, st);
  } else {
    if (b16) launch_prefill<bf16, 128>(*a, p, st); else launch_prefill<float, 128>(*a, p, st);
  }
  return launch_status("uttt_swa_prefill");
}

extern "C" size_t uttt_swa_decode_workspace(int64_t n_req, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                            int64_t window) {
  if (n_req < 1 || n_kv_heads < 1 || n_heads < n_kv_heads || window < 1 || head_dim < 1) return 0;
  return decode_partial_bytes(n_req, n_heads, head_dim, window);
}

extern "C" int uttt_swa_decode(const uttt_swa_decode_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->head_dim == 64 || a->head_dim == 128, "head_dim must be 64 or 128 (got %lld)", (long long)a->head_dim);
  UTTT_REQUIRE(a->n_req >= 1 && a->n_req <= 2147483647 && a->n_kv_heads >= 1 && a->n_kv_heads <= 65535 &&
               a->n_heads % a->n_kv_heads == 0, "bad request / head counts");
  UTTT_REQUIRE(a->n_heads / a->n_kv_heads <= kMaxRep, "at most %d query heads per kv head", kMaxRep);
  UTTT_REQUIRE(a->window >= 1 && decode_splits(a->window) <= 65535, "window out of range");
  UTTT_REQUIRE(a->workspace != nullptr &&
               a->workspace_bytes >= uttt_swa_decode_workspace(a->n_req, a->n_heads, a->n_kv_heads, a->head_dim,
                                                               a->window),
               "decode workspace too small");
  UTTT_REQUIRE(aligned16(a->k_ring) && aligned16(a->v_ring) && a->ring_stride_n % 8 == 0,
               "rings must be 16-byte aligned with a 16-byte multiple request stride");
  UTTT_REQUIRE(a->positions && a->q && a->k_new && a->v_new && a->k_ring && a->v_ring && a->out,
               "pointers must be non-NULL");
  UTTT_REQUIRE((a->cos_table == nullptr) == (a->sin_table == nullptr), "cos/sin tables must both be given or both NULL");
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_F32 || a->act_dtype == UTTT_DTYPE_BF16, "bad act_dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool b16 = a->act_dtype == UTTT_DTYPE_BF16;
  if (a->head_dim == 64) {
    if (b16) launch_decode<bf16, 64>(*a, st); else launch_decode<float, 64>(*a, st);
  } else {
    if (b16) launch_decode<bf16, 128>(*a, st); else launch_decode<float, 128>(*a, st);
  }
  return launch_status("uttt_swa_decode");
}
