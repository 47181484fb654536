// The whole chunk loop of one standalone uTTT layer in persistent kernels, for one row with fp32
// activations (d_model 512, d_ff 1024, 16 chunks of 64 tokens), written for
// gfx950 (MI355X).  Replaces the per-chunk fused_chunk_ttt_step calls of uTTTLayer.forward
// (model/uttt_layer.py:1451-1478 around :414-534): every chunk reads its own pre-update state and
// writes the next one.
//
// The fast-weight state stays on chip between the chunks of a launch (up to kSegChunks of them).
// Workgroup w owns the 8 F columns [8 w, 8 w + 8); inside it, wave v owns the features d in
// [v D / 4, (v + 1) D / 4).  Its slice of W_up | W_gate stays in registers, its slices of W_down and
// of the momentum in LDS, each element at the lane that forms its gradient.
// Per chunk (C <= 64 tokens; q and k run through the same pre-update W):
//   1. U | G (64 x 16) for the keys and the queries: every wave over its features, the four
//      partial sums added in LDS; H = SiLU(G) U
//   2. the key path's Z partials (H W_down[cols, :])^T over each wave's features -> workspace; the
//      query path's H and this chunk's W_down[cols, :] saved for the readout;    grid barrier
//   3. one key row per workgroup: Z = sum of the partials, LayerNorm, token loss, dZ (stored for
//      every workgroup);                                                          grid barrier
//   4. per feature tile of 16: dH partial (dZ W_down^T), (dZ^T H)^T; dH summed over the waves,
//      dU, dG; per feature tile: (K^T [dU | dG]); the squared norm of the three;  grid barrier
//   5. clip from the summed norms, S' = beta S - c g, W' = (1 - mean alpha) W + S' in place.
// After each launch the readout of its chunks, out = q + LN(H_q W_down) with the saved operands,
// runs as a batched product over its chunks (launch_saved_readout): its Z partial sums stay off
// the critical path of the update.
// MFMA v_mfma_f32_16x16x4f32 throughout: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and
// holds D[4 (l / 16) + i][l % 16] (checked on the device).  The k index of a step is free: the
// products that contract over features give lane l / 16 the features 4 (l / 16) + i of a tile of 16,
// so that its operand rows are contiguous float4 loads and its gradient elements land where the
// state already sits.  Tiles read transposed (dZ and K with features along lanes) go through a
// 64 x 16 LDS tile per wave.
//
// Grid barriers: data one workgroup hands to others (Z partials, dZ, token losses, norm partials)
// is written and read device-coherently (the sc1 cache policy of agent-scope atomics, here on float4
// buffer accesses), so no cache needs writing back or invalidating: every wave waits for its stores,
// then one thread per workgroup raises a monotone counter and spins on it (bounded: past the bound
// the error flag is set and no later barrier waits) until every workgroup has arrived.  The grid
// never exceeds the CU count (one workgroup per CU), so every workgroup is resident once the CUs are
// free.
#include <algorithm>
#include <mutex>

#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {
namespace {

constexpr int kCols = 8;                   // F columns per workgroup
constexpr int kUgLd = 17;                  // row stride of the per-wave U | G and dH partials in LDS
constexpr int kTLd = 68;                   // row stride of the [16][64] transposed tiles (16-byte rows)
constexpr unsigned kSpinLimit = 1u << 20;  // about a second of polling
constexpr int kCoherent = 16;              // buffer cache policy sc1: device-coherent, as agent-scope atomics

struct ResArgs {
  int T, CS, D, F, c_begin, c_end, normalize;  // chunks [c_begin, c_end) of this launch
  float beta, max_norm, eps;
  const float* q; const float* k; const float* v; const float* eta; const float* alpha; const float* mask;
  const float* w[3]; const float* s[3];
  const float* ln_w; const float* ln_b;
  float* out;
  float* surprise;    // (chunks,)
  unsigned char* ws;  // workspace, laid out as WsLayout
  unsigned* error_word;  // optional: set to 1 on a barrier timeout, never cleared here
};

constexpr int kSegChunks = 16;  // chunks per launch: bounds the saved readout operands
constexpr int kReadoutSplits = 4;  // F splits of the readout's Z partial sums

// Workspace: barrier counter and flag, the six state output pointers (stored by the init kernel and
// read back at the end, so that they do not occupy scalar registers for the whole kernel), token
// losses, gradient-norm partials, dZ, the key path's Z partials, then per chunk of a launch the
// saved query H (64 x F) and W_down (F x D) for the readout, and the readout's Z partials.  The
// offsets depend only on D and the workgroup count nw = F / 8, so the kernel derives every pointer
// from the one base.
struct WsLayout {
  static constexpr size_t kCounter = 0, kFlag = 4, kOutPtrs = 64, kLoss = 256, kNorms = 512;
  static constexpr size_t kDz = kNorms + 4 * 1024;  // room for 1024 norm partials
  static constexpr size_t dz_bytes(int64_t D) { return 4 * 64 * (size_t)D; }
  static constexpr size_t part(int64_t D) { return kDz + dz_bytes(D); }
  static constexpr size_t hq(int64_t D, int64_t nw) { return part(D) + 4 * (size_t)nw * 64 * D; }
  static constexpr size_t wds(int64_t D, int64_t nw) { return hq(D, nw) + 4 * (size_t)kSegChunks * 64 * 8 * nw; }
  static constexpr size_t zp(int64_t D, int64_t nw) { return wds(D, nw) + 4 * (size_t)kSegChunks * 8 * nw * D; }
  static constexpr size_t total(int64_t D, int64_t nw) {
    return zp(D, nw) + 4 * (size_t)kReadoutSplits * kSegChunks * 64 * D;
  }
};

__device__ __forceinline__ unsigned* ws_counter(const ResArgs& a) { return reinterpret_cast<unsigned*>(a.ws + WsLayout::kCounter); }
__device__ __forceinline__ unsigned* ws_flag(const ResArgs& a) { return reinterpret_cast<unsigned*>(a.ws + WsLayout::kFlag); }
__device__ __forceinline__ float* ws_loss(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::kLoss); }
__device__ __forceinline__ float* ws_norms(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::kNorms); }
__device__ __forceinline__ float* ws_dz(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::kDz); }
template <int D>
__device__ __forceinline__ float* ws_part(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::part(D)); }
template <int D>
__device__ __forceinline__ float* ws_hq(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::hq(D, gridDim.x)); }
template <int D>
__device__ __forceinline__ float* ws_wds(const ResArgs& a) { return reinterpret_cast<float*>(a.ws + WsLayout::wds(D, gridDim.x)); }

__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 ld4_coherent(__amdgpu_buffer_rsrc_t rs, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kCoherent));
}
__device__ __forceinline__ void st4_coherent(__amdgpu_buffer_rsrc_t rs, int off, f32x4 v) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, off, 0, kCoherent);
}

// Every workgroup arrives, then waits until all have arrived for the `round`-th time.
__device__ void grid_barrier(const ResArgs& a, unsigned round) {
  wait_vmcnt<0>();  // this wave's device-coherent stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(ws_counter(a), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned target = round * gridDim.x;
    if (__hip_atomic_load(ws_flag(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
      unsigned spins = 0;
      while (__hip_atomic_load(ws_counter(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(2);
        if (++spins > kSpinLimit) {
          __hip_atomic_store(ws_flag(a), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (a.error_word != nullptr) __hip_atomic_store(a.error_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
  }
  __syncthreads();
}

struct OutPtrs {
  float* p[6];  // W_up, W_gate, W_down, S_up, S_gate, S_down
};

// Before each launch of k_resident_update: the barrier counter restarts; the error flag is set by
// the first launch of a call only (flag_mode 1: cleared, 2: raised, as if a barrier had timed out,
// with the error word; 0: kept), so that it reports a timeout in any of the call's launches.
__global__ void __launch_bounds__(kThreads) k_resident_init(unsigned char* ws, const OutPtrs outs, int flag_mode,
                                                            unsigned* error_word) {
  if (threadIdx.x == 0) {
    *reinterpret_cast<unsigned*>(ws + WsLayout::kCounter) = 0u;
    if (flag_mode != 0) *reinterpret_cast<unsigned*>(ws + WsLayout::kFlag) = flag_mode == 2 ? 1u : 0u;
    if (flag_mode == 2 && error_word != nullptr) *error_word = 1u;
  }
  if (threadIdx.x < 6) reinterpret_cast<float**>(ws + WsLayout::kOutPtrs)[threadIdx.x] = outs.p[threadIdx.x];
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Order one wave's LDS writes before its later reads (and reads before later writes) of its own
// tile: a wave's LDS instructions execute in order, so only the compiler must not move them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// rows 16 r + col (r < 4) of a (rows, D) matrix at features d0 + 4 kq .. + 3; rows at or past
// `valid` read as zero.  Buffer loads (the range check of the descriptor supplies the zeros), so
// there is no branch around a load and the compiler can count loads still in flight.
// AUX: the cache policy (kCoherent for data other workgroups of the launch wrote).
template <int AUX = 0>
__device__ __forceinline__ void load_rows(const float* x, int D, int d0, int valid, int col, int kq, f32x4 (&v)[4]) {
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(x, (uint32_t)valid * (uint32_t)D * 4u);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int off = ((16 * r + col) * D + d0 + 4 * kq) * 4;
    v[r] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, AUX));
  }
}

// the 64 x 16 tile held by load_rows (row 16 r + col, feature 4 kq + i) into a wave's LDS tile,
// transposed: [feature][row]
__device__ __forceinline__ void put_tile_t(float* tile, int col, int kq, const f32x4 (&v)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[(4 * kq + i) * kTLd + 16 * r + col] = v[r][i];
}

// sum over the 64 tokens of A[m][t] B[t][n] with A^T and B^T rows in LDS ([m][t] and [n][t], 16-byte
// aligned rows of kTLd floats): lane (col, kq) takes tokens 16 kq .. 16 kq + 15 as its k steps, read
// as float4 from A^T row col and B^T row brow.  b_on false: B's row for this lane is zero.
__device__ __forceinline__ f32x4 mfma_tokens(const float* at, const float* bt, int brow, bool b_on, int col,
                                             int kq) {
  f32x4 acc = zero4();
  const f32x4* ar = reinterpret_cast<const f32x4*>(at + col * kTLd + 16 * kq);
  const f32x4* br = reinterpret_cast<const f32x4*>(bt + brow * kTLd + 16 * kq);
  f32x4 av[4], bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    av[j] = ar[j];
    bv[j] = b_on ? br[j] : zero4();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = mfma4(av[j][q], bv[j][q], acc);
  return acc;
}

// Z of one key row from the partials of every workgroup (fixed order), then LayerNorm, the token
// loss and dZ.  Threads th < D / 4 hold features 4 th .. + 3.
template <int D>
__device__ void ln_row(const ResArgs& a, int t, int t0, int C, float* comb, float* red) {
  constexpr int kF4 = D / 4;             // float4 per row
  constexpr int kGroups = kThreads / kF4;  // partial subsets summed side by side
  constexpr int kFlight = 32;            // loads in flight per thread
  const int nw = gridDim.x;
  const int g = threadIdx.x / kF4, f4 = threadIdx.x % kF4;
  // partials of workgroups u >= nw lie past the descriptor's range and read as zero (the whole
  // offset is in the vector operand, which the range check covers)
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(ws_part<D>(a), (uint32_t)nw * 64u * (uint32_t)D * 4u);
  const int base = (t * D + 4 * f4) * 4;
  constexpr int kUStride = 64 * D * 4;  // bytes between the partials of consecutive workgroups
  f32x4 z = zero4();
  for (int u0 = g; u0 < nw; u0 += kFlight * kGroups) {
    f32x4 v[kFlight];
#pragma unroll
    for (int j = 0; j < kFlight; ++j) {
      const int u = u0 + j * kGroups;
      v[j] = ld4_coherent(rs, base + u * kUStride);
    }
#pragma unroll
    for (int j = 0; j < kFlight; ++j) z += v[j];
  }
  if constexpr (kGroups > 1) {
    *reinterpret_cast<f32x4*>(comb + g * D + 4 * f4) = z;
    __syncthreads();
    if (g == 0) {
#pragma unroll
      for (int gg = 1; gg < kGroups; ++gg) z += *reinterpret_cast<const f32x4*>(comb + gg * D + 4 * f4);
    }
  }
  const bool mine = threadIdx.x < kF4;
  const float inv_d = 1.0f / (float)D;
  const float inv_scale = a.normalize ? inv_d : 1.0f;
  const float mean = block_sum(mine ? (z[0] + z[1]) + (z[2] + z[3]) : 0.f, red) * inv_d;
  f32x4 cz = z - mean;
  const float var = block_sum(mine ? (cz[0] * cz[0] + cz[1] * cz[1]) + (cz[2] * cz[2] + cz[3] * cz[3]) : 0.f, red) * inv_d;
  const float rstd = 1.0f / sqrtf(var + a.eps);
  const int tg = t0 + t;
  const int d = 4 * f4;
  f32x4 lw = zero4(), lb = zero4();
  if (mine) {
    lw = *reinterpret_cast<const f32x4*>(a.ln_w + d);
    lb = *reinterpret_cast<const f32x4*>(a.ln_b + d);
  }
  f32x4 zh = zero4(), e = zero4();
  float se = 0.f;
  if (mine) {
    const f32x4 kk = *reinterpret_cast<const f32x4*>(a.k + (int64_t)tg * D + d);
    const f32x4 vv = *reinterpret_cast<const f32x4*>(a.v + (int64_t)tg * D + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      zh[i] = cz[i] * rstd;
      e[i] = (kk[i] + (zh[i] * lw[i] + lb[i])) - vv[i];
    }
    se = (e[0] * e[0] + e[1] * e[1]) + (e[2] * e[2] + e[3] * e[3]);
  }
  float sums[2] = {se, (a.mask != nullptr && threadIdx.x < C) ? a.mask[t0 + threadIdx.x] : 0.f};
  block_sums<2>(sums, red);
  const float token_loss = 0.5f * sums[0] * inv_scale;
  const float eta_t = a.eta[tg];
  float weight, m_t = 1.f;
  if (a.mask != nullptr) {
    m_t = a.mask[tg];
    weight = (eta_t * m_t) / fmaxf(sums[1], 1.0f);
  } else {
    weight = eta_t * (1.0f / (float)C);
  }
  const float coef = weight * inv_scale;
  float s3 = 0.f, s4 = 0.f;
  if (mine) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = coef * e[i] * lw[i];  // dZ_hat
      s3 += e[i];
      s4 += e[i] * zh[i];
    }
  }
  float moments[2] = {s3, s4};
  block_sums<2>(moments, red);
  const float m1 = moments[0] * inv_d, m2 = moments[1] * inv_d;
  if (mine) {
    f32x4 dz;
#pragma unroll
    for (int i = 0; i < 4; ++i) dz[i] = rstd * (e[i] - m1 - zh[i] * m2);
    st4_coherent(buffer_rsrc(ws_dz(a), 64u * D * 4u), (t * D + d) * 4, dz);
  }
  if (threadIdx.x == 0) st_agent(ws_loss(a) + t, a.mask != nullptr ? token_loss * m_t : token_loss);
}

template <int ND>
__global__ void __launch_bounds__(kThreads, 1) k_resident_update(const ResArgs a) {
  constexpr int D = ND * 64;
  constexpr int DW = D / 4;      // features per wave: ND tiles of 16
  constexpr int WDLD = D + 4;    // W_down row stride in LDS (spreads the 8 rows over banks)
  __shared__ __align__(16) float wdn[kCols * WDLD];  // W_down [c][d]
  __shared__ float part_lds[4 * 2 * 64 * kUgLd];      // per-wave U | G partials [v][p][t][c]; dH partials; row sums
  __shared__ __align__(16) float hs[2][64 * kCols];   // H of the keys / queries [t][c]
  __shared__ float uk[64 * kCols], gk[64 * kCols];    // U, G of the keys
  __shared__ __align__(16) float hkt[kCols * kTLd];   // H^T of the keys [c][t]
  __shared__ __align__(16) float dugt[16 * kTLd];     // [dU | dG]^T [c][t]
  __shared__ __align__(16) float tiles[4][16 * kTLd]; // per-wave transposed tile [feature][t]
  // momentum, element (m, i) of a lane (see below) at [(wave ND + m) 64 + lane] (S_up | S_gate) and
  // [(wave ND + m) 32 + 8 kq + col] (S_down, lanes col < 8) as float4
  __shared__ f32x4 s_ug_lds[4 * ND * 64], s_dn_lds[4 * ND * 32];
  __shared__ float red[16];
  const int w = blockIdx.x, f0 = w * kCols;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kq = lane >> 4;  // MFMA column / k index of this lane
  const int dbase = wave * DW;
  float* tile = tiles[wave];

  // ---- the state slices.  Element (m, i) of a lane: feature d = dbase + 16 m + 4 kq + i, column col
  // (W_up / S_up for col < 8, W_gate / S_gate for col >= 8; S_down row col for col < 8).  W_up | W_gate
  // in registers, the momentum in LDS.
  f32x4* const s_ug = s_ug_lds + wave * ND * 64 + lane;              // element m at s_ug[64 m]
  f32x4* const s_dn = s_dn_lds + wave * ND * 32 + 8 * kq + (col & 7);  // element m at s_dn[32 m]
  float w_ug[ND][4];
#pragma unroll
  for (int m = 0; m < ND; ++m) {
    f32x4 su, sd;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dbase + 16 * m + 4 * kq + i;
      const int64_t off = (int64_t)d * a.F + f0 + (col & 7);
      w_ug[m][i] = col < kCols ? a.w[0][off] : a.w[1][off];
      su[i] = col < kCols ? a.s[0][off] : a.s[1][off];
      sd[i] = col < kCols ? a.s[2][(int64_t)(f0 + col) * D + d] : 0.f;
    }
    s_ug[64 * m] = su;
    if (col < kCols) s_dn[32 * m] = sd;
  }
  for (int i = threadIdx.x; i < kCols * D; i += kThreads) {
    const int c = i / D, d = i % D;
    wdn[c * WDLD + d] = a.w[2][(int64_t)(f0 + c) * D + d];
  }
  __syncthreads();
  unsigned round = 0;
  // step 1 keeps three feature tiles of key and query rows in flight; the first two of a chunk are
  // issued at the end of the previous chunk
  f32x4 xb[3][2][4];
  {
    const int tb = a.c_begin * a.CS, C0 = min(a.CS, a.T - tb);
    load_rows(a.k + (int64_t)tb * D, D, dbase, C0, col, kq, xb[0][0]);
    load_rows(a.q + (int64_t)tb * D, D, dbase, C0, col, kq, xb[0][1]);
    if (ND > 1) {
      load_rows(a.k + (int64_t)tb * D, D, dbase + 16, C0, col, kq, xb[1][0]);
      load_rows(a.q + (int64_t)tb * D, D, dbase + 16, C0, col, kq, xb[1][1]);
    }
  }

  for (int c = a.c_begin; c < a.c_end; ++c) {
    const int t0 = c * a.CS, C = min(a.CS, a.T - t0);
    const float* xk = a.k + (int64_t)t0 * D;
    const float* xq = a.q + (int64_t)t0 * D;
    // ---------------- 1. U | G partials over this wave's features, both paths
    {
      f32x4 acc[2][4];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[p][r] = zero4();
#pragma unroll
      for (int m = 0; m < ND; ++m) {
        if (m + 2 < ND) {
          load_rows(xk, D, dbase + 16 * (m + 2), C, col, kq, xb[(m + 2) % 3][0]);
          load_rows(xq, D, dbase + 16 * (m + 2), C, col, kq, xb[(m + 2) % 3][1]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[p][r] = mfma4(xb[m % 3][p][r][i], w_ug[m][i], acc[p][r]);
      }
      // acc[p][r][j] = partial U | G of token 16 r + 4 kq + j, column col
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            part_lds[((wave * 2 + p) * 64 + 16 * r + 4 * kq + j) * kUgLd + col] = acc[p][r][j];
    }
    __syncthreads();
    // U | G summed over the waves (in wave order), H = SiLU(G) U
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = threadIdx.x + j * kThreads;  // (p, t, c): 2 x 64 x 8
      const int p = e >> 9, t = (e >> 3) & 63, cc = e & 7;
      float u = 0.f, g = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float* row = part_lds + ((v * 2 + p) * 64 + t) * kUgLd;
        u += row[cc];
        g += row[cc + kCols];
      }
      const float h = (g * sigmoidf_acc(g)) * u;
      hs[p][t * kCols + cc] = h;
      if (p == 0) {
        uk[t * kCols + cc] = u;
        gk[t * kCols + cc] = g;
        hkt[cc * kTLd + t] = h;
      }
    }
    __syncthreads();
    // ---------------- 2. the key path's Z^T partials over this wave's features:
    // (W_down[cols, d])^T H^T; the query path's H and this chunk's W_down[cols, :] are saved for the
    // readout, which runs after the launch
    {
      const __amdgpu_buffer_rsrc_t pw = buffer_rsrc(ws_part<D>(a) + (int64_t)w * 64 * D, 64u * D * 4u);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * r + col;
        const float h0 = hs[0][t * kCols + kq], h1 = hs[0][t * kCols + 4 + kq];
#pragma unroll
        for (int n = 0; n < ND; ++n) {
          const int d = dbase + 16 * n + col;
          f32x4 z = mfma4(wdn[kq * WDLD + d], h0, zero4());
          z = mfma4(wdn[(4 + kq) * WDLD + d], h1, z);
          // z[j] = Z partial of token t, feature dbase + 16 n + 4 kq + j
          if (t < C) st4_coherent(pw, (t * D + dbase + 16 * n + 4 * kq) * 4, z);
        }
      }
      const int slot = c - a.c_begin;
      if (threadIdx.x < 128) {  // H of the queries: rows t, columns f0 .. f0 + 7
        const int t = threadIdx.x >> 1, half = threadIdx.x & 1;
        *reinterpret_cast<f32x4*>(ws_hq<D>(a) + ((int64_t)slot * 64 + t) * a.F + f0 + 4 * half) =
            *reinterpret_cast<const f32x4*>(&hs[1][t * kCols + 4 * half]);
      }
      float* wsave = ws_wds<D>(a) + ((int64_t)slot * a.F + f0) * D;  // this chunk's W_down rows f0 .. f0 + 7
#pragma unroll
      for (int j = 0; j < 2 * D / kThreads; ++j) {
        const int e = threadIdx.x + j * kThreads;  // float4 index over 8 x D / 4
        const int cc = e / (D / 4), d4 = e % (D / 4);
        *reinterpret_cast<f32x4*>(wsave + (int64_t)cc * D + 4 * d4) =
            *reinterpret_cast<const f32x4*>(&wdn[cc * WDLD + 4 * d4]);
      }
    }
    grid_barrier(a, ++round);
    // ---------------- 3. key rows: Z, LayerNorm, loss and dZ
    for (int t = w; t < C; t += gridDim.x) {
      ln_row<D>(a, t, t0, C, part_lds, red);
      __syncthreads();  // part_lds and red are reused by the next row
    }
    grid_barrier(a, ++round);
    // ---------------- 4. gradients over this wave's features
    f32x4 g_ug[ND], g_dn[ND];
    float sq = 0.f;
    {
      const float* dzp = ws_dz(a);
      f32x4 dh[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) dh[r] = zero4();
      f32x4 zb[4][4];  // four feature tiles of dZ rows in flight
#pragma unroll
      for (int m = 0; m < 3 && m < ND; ++m) load_rows<kCoherent>(dzp, D, dbase + 16 * m, C, col, kq, zb[m]);
      // warm this XCD's L2 with a slice of the next chunk's key and query rows (workgroup w runs on
      // XCD w mod 8; a wrong guess only costs the warm-up): 16 KB per workgroup
      f32x4 warm[4];
      {
        const int tn = t0 + a.CS, Cn = c + 1 < a.c_end ? min(a.CS, a.T - tn) : 0;
        const uint32_t kbytes = (uint32_t)Cn * D * 4u;
        const int piece = (w >> 3) * 16384;  // byte offset in [K rows | Q rows] of the next chunk
        const bool in_k = piece < 64 * D * 4;
        const __amdgpu_buffer_rsrc_t rw =
            buffer_rsrc(in_k ? a.k + (int64_t)tn * D : a.q + (int64_t)tn * D, kbytes);
        const int off = (in_k ? piece : piece - 64 * D * 4) + threadIdx.x * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          warm[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off + j * 4096, 0, 0));
      }
      if (w == 0 && threadIdx.x < 64) {  // the chunk's surprise: masked token losses / valid tokens
        const int l = threadIdx.x;
        float num = l < C ? ld_agent(ws_loss(a) + l) : 0.f;
        float den = l < C ? (a.mask != nullptr ? a.mask[t0 + l] : 1.f) : 0.f;
        num = wave_sum(num);
        den = wave_sum(den);
        if (l == 0) a.surprise[c] = a.mask != nullptr ? num / fmaxf(den, 1.f) : num / den;
      }
#pragma unroll
      for (int m = 0; m < ND; ++m) {
        if (m + 3 < ND) load_rows<kCoherent>(dzp, D, dbase + 16 * (m + 3), C, col, kq, zb[(m + 3) % 4]);
        const f32x4 (&z)[4] = zb[m % 4];
        // dH partial [t][c] += dZ[t][d] W_down[c][d] over this tile's features
        const f32x4 wv = *reinterpret_cast<const f32x4*>(&wdn[(col & 7) * WDLD + dbase + 16 * m + 4 * kq]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float b = col < kCols ? wv[i] : 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) dh[r] = mfma4(z[r][i], b, dh[r]);
        }
        put_tile_t(tile, col, kq, z);
        wave_lds_sync();
        // gradient of W_down[c][d] for this tile's features: sum_t dZ[t][d] H[t][c]
        const f32x4 gd = mfma_tokens(tile, hkt, col & 7, col < kCols, col, kq);
        g_dn[m] = gd;
        if (col < kCols) sq += (gd[0] * gd[0] + gd[1] * gd[1]) + (gd[2] * gd[2] + gd[3] * gd[3]);
        wave_lds_sync();
      }
      // the first key tiles of the W_up | W_gate gradient, in flight during the dH sum
      f32x4 kb[3][4];
      load_rows(xk, D, dbase, C, col, kq, kb[0]);
      if (ND > 1) load_rows(xk, D, dbase + 16, C, col, kq, kb[1]);
      // dH summed over the waves; dU, dG
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) part_lds[(wave * 64 + 16 * r + 4 * kq + j) * kUgLd + col] = dh[r][j];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int e = threadIdx.x + j * kThreads;  // (t, c): 64 x 8
        const int t = e >> 3, cc = e & 7;
        float dhs = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) dhs += part_lds[(v * 64 + t) * kUgLd + cc];
        const float u = uk[t * kCols + cc], g = gk[t * kCols + cc];
        const float sg = sigmoidf_acc(g);
        dugt[cc * kTLd + t] = dhs * (g * sg);
        dugt[(kCols + cc) * kTLd + t] = dhs * u * (sg * (1.0f + g * (1.0f - sg)));
      }
      __syncthreads();
      // gradient of W_up | W_gate: sum_t K[t][d] [dU | dG][t][c]
#pragma unroll
      for (int m = 0; m < ND; ++m) {
        if (m + 2 < ND) load_rows(xk, D, dbase + 16 * (m + 2), C, col, kq, kb[(m + 2) % 3]);
        put_tile_t(tile, col, kq, kb[m % 3]);
        wave_lds_sync();
        const f32x4 gu = mfma_tokens(tile, dugt, col, true, col, kq);
        g_ug[m] = gu;
        sq += (gu[0] * gu[0] + gu[1] * gu[1]) + (gu[2] * gu[2] + gu[3] * gu[3]);
        wave_lds_sync();
      }
      // the warm-up loads have long completed; consume them so that they are kept
      asm volatile("" ::"v"(warm[0]), "v"(warm[1]), "v"(warm[2]), "v"(warm[3]));
      const float total = block_sum(sq, red);
      if (threadIdx.x == 0) st_agent(ws_norms(a) + w, total);
    }
    // this chunk's alpha and mask values, read while the barrier waits
    const float alpha_t = threadIdx.x < C ? a.alpha[t0 + threadIdx.x] : 0.f;
    const float mask_t = (a.mask != nullptr && threadIdx.x < C) ? a.mask[t0 + threadIdx.x] : 0.f;
    grid_barrier(a, ++round);
    // ---------------- 5. clip, momentum, decay, in place
    {
      float n2 = 0.f;
      for (int i = threadIdx.x; i < (int)gridDim.x; i += kThreads) n2 += ld_agent(ws_norms(a) + i);
      n2 = block_sum(n2, red);
      float asum = 0.f, msum = 0.f, any = 0.f;
      if (threadIdx.x < C) {
        if (a.mask != nullptr) {
          asum = alpha_t * mask_t;
          msum = mask_t;
          any = mask_t != 0.f ? 1.f : 0.f;
        } else {
          asum = alpha_t;
        }
      }
      float sums[3] = {asum, msum, any};
      block_sums<3>(sums, red);
      const float abar = a.mask != nullptr ? sums[0] / fmaxf(sums[1], 1.f) : sums[0] / (float)C;
      const float clip = a.max_norm > 0.f ? fminf(a.max_norm * (1.0f / sqrtf(n2 + 1e-8f)), 1.0f) : 1.0f;
      const float decay = 1.0f - abar;
      const bool active = a.mask == nullptr || sums[2] > 0.f;
      if (active) {
#pragma unroll
        for (int m = 0; m < ND; ++m) {
          f32x4 su = s_ug[64 * m], sd = col < kCols ? s_dn[32 * m] : zero4();
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            {
#pragma clang fp contract(off)
              const float step = g_ug[m][i] * clip;
              const float s_new = a.beta * su[i] - step;
              w_ug[m][i] = decay * w_ug[m][i] + s_new;
              su[i] = s_new;
            }
            if (col < kCols) {
#pragma clang fp contract(off)
              float* wd = &wdn[col * WDLD + dbase + 16 * m + 4 * kq + i];
              const float step = g_dn[m][i] * clip;
              const float s_new = a.beta * sd[i] - step;
              *wd = decay * *wd + s_new;
              sd[i] = s_new;
            }
          }
          s_ug[64 * m] = su;
          if (col < kCols) s_dn[32 * m] = sd;
        }
      }
      if (c + 1 < a.c_end) {  // the next chunk's first two feature tiles
        const int tn = t0 + a.CS, Cn = min(a.CS, a.T - tn);
        load_rows(a.k + (int64_t)tn * D, D, dbase, Cn, col, kq, xb[0][0]);
        load_rows(a.q + (int64_t)tn * D, D, dbase, Cn, col, kq, xb[0][1]);
        if (ND > 1) {
          load_rows(a.k + (int64_t)tn * D, D, dbase + 16, Cn, col, kq, xb[1][0]);
          load_rows(a.q + (int64_t)tn * D, D, dbase + 16, Cn, col, kq, xb[1][1]);
        }
      }
      __syncthreads();  // W_down updated in LDS before the next chunk reads it
    }
  }
  // ---- the final state.  The lane index is re-derived through an empty asm statement so that the
  // compiler recomputes these addresses here instead of keeping the ones of the initial loads live
  // (in registers, or spilled) through the chunk loop.
  // A barrier of this call that waited past its bound (every workgroup that passed a timed-out
  // barrier sees the flag by now) leaves the results invalid: they are made loud instead, NaN in
  // the state, the surprise of this launch's chunks and, through the saved query H, their readout.
  const bool timed_out = __hip_atomic_load(ws_flag(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
  const float nan = __builtin_nanf("");
  float* const* outs = reinterpret_cast<float* const*>(a.ws + WsLayout::kOutPtrs);
  int lane_f = threadIdx.x & 63;
  asm volatile("" : "+v"(lane_f));
  const int col_f = lane_f & 15, kq_f = lane_f >> 4;
#pragma unroll
  for (int m = 0; m < ND; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dbase + 16 * m + 4 * kq_f + i;
      const int64_t off = (int64_t)d * a.F + f0 + (col_f & 7);
      outs[col_f < kCols ? 0 : 1][off] = timed_out ? nan : w_ug[m][i];
      outs[col_f < kCols ? 3 : 4][off] = timed_out ? nan : s_ug_lds[(wave * ND + m) * 64 + lane_f][i];
      if (col_f < kCols)
        outs[5][(int64_t)(f0 + col_f) * D + d] = timed_out ? nan : s_dn_lds[(wave * ND + m) * 32 + 8 * kq_f + col_f][i];
    }
  for (int i = threadIdx.x; i < kCols * D; i += kThreads) {
    const int c = i / D, d = i % D;
    outs[2][(int64_t)(f0 + c) * D + d] = timed_out ? nan : wdn[c * WDLD + d];
  }
  if (timed_out) {
    const int nseg = a.c_end - a.c_begin;  // this workgroup's 8 columns of each chunk's saved query H
    const f32x4 nan4{nan, nan, nan, nan};
    for (int i = threadIdx.x; i < nseg * 64 * 2; i += kThreads) {
      const int slot = i >> 7, t = (i >> 1) & 63, half = i & 1;
      *reinterpret_cast<f32x4*>(ws_hq<D>(a) + ((int64_t)slot * 64 + t) * a.F + f0 + 4 * half) = nan4;
    }
    if (w == 0)
      for (int c = a.c_begin + threadIdx.x; c < a.c_end; c += kThreads) a.surprise[c] = nan;
  }
}

std::mutex cu_mutex;
int cu_count[64] = {};

// CUs of the current device (cached per device)
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(cu_mutex);
  if (cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cu_count[dev] = n;
  }
  return cu_count[dev];
}

int check_resident(int64_t batch, int64_t d_model, int64_t d_ff) {
  UTTT_REQUIRE(batch == 1, "the resident update takes one row (got batch %lld)", (long long)batch);
  UTTT_REQUIRE(d_model == 128 || d_model == 256 || d_model == 512,
               "the resident update takes d_model 128, 256 or 512 (got %lld)", (long long)d_model);
  UTTT_REQUIRE(d_ff >= 64 && d_ff % 64 == 0, "d_ff must be a positive multiple of 64 (got %lld)", (long long)d_ff);
  const int cus = device_cus();
  UTTT_REQUIRE(cus > 0, "cannot read the device's CU count");
  UTTT_REQUIRE(d_ff / kCols <= cus, "the resident update needs d_ff / %d = %lld workgroups, more than the %d CUs",
               kCols, (long long)(d_ff / kCols), cus);
  return UTTT_OK;
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_layer_update_resident_supported(int64_t batch, int64_t d_model, int64_t d_ff) {
  if (check_resident(batch, d_model, d_ff) != UTTT_OK) return 0;
  return 1;
}

extern "C" size_t uttt_layer_update_resident_workspace(int64_t d_model, int64_t d_ff) {
  if (d_model < 64 || d_ff < kCols) return 0;
  return WsLayout::total(d_model, d_ff / kCols);
}

extern "C" size_t uttt_layer_update_resident_flag_offset(int64_t d_model, int64_t d_ff) {
  if (d_model < 64 || d_ff < kCols) return 0;
  return WsLayout::kFlag;
}

extern "C" int uttt_layer_update_resident(const uttt_layer_update_args* a, void* workspace, size_t workspace_bytes,
                                          uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  int rc = check_resident(a->batch, a->d_model, a->d_ff);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->tokens >= 1 && a->tokens <= (1 << 24), "tokens must be in [1, 2^24] (got %lld)", (long long)a->tokens);
  UTTT_REQUIRE(a->chunk_size >= 1 && a->chunk_size <= 64, "chunk_size must be in [1, 64] (got %lld)",
               (long long)a->chunk_size);
  UTTT_REQUIRE(a->q && a->k && a->v && a->eta && a->alpha, "q/k/v/eta/alpha must be non-NULL");
  UTTT_REQUIRE(a->w_up && a->w_gate && a->w_down && a->s_up && a->s_gate && a->s_down, "state pointers must be non-NULL");
  UTTT_REQUIRE(a->w_up_out && a->w_gate_out && a->w_down_out && a->s_up_out && a->s_gate_out && a->s_down_out,
               "output state pointers must be non-NULL");
  UTTT_REQUIRE(a->ln_weight && a->ln_bias && a->out && a->surprise, "ln_weight/ln_bias/out/surprise must be non-NULL");
  UTTT_REQUIRE(aligned16(a->q) && aligned16(a->k) && aligned16(a->v) && aligned16(a->out) && aligned16(a->ln_weight) &&
                   aligned16(a->ln_bias),
               "q/k/v/out/ln_weight/ln_bias must be 16-byte aligned");
  const size_t need = WsLayout::total(a->d_model, a->d_ff / kCols);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small: need %zu bytes, got %zu", need,
               workspace_bytes);
  UTTT_REQUIRE(a->d_ff / kCols <= 1024, "d_ff / %d must be at most 1024", kCols);
  ResArgs r{};
  r.T = (int)a->tokens;
  r.CS = (int)a->chunk_size;
  r.D = (int)a->d_model;
  r.F = (int)a->d_ff;
  r.normalize = a->normalize_by_dim;
  r.beta = a->momentum_beta;
  r.max_norm = a->max_inner_grad_norm;
  r.eps = a->eps;
  r.q = a->q; r.k = a->k; r.v = a->v;
  r.eta = a->eta; r.alpha = a->alpha; r.mask = a->token_mask;
  r.w[0] = a->w_up; r.w[1] = a->w_gate; r.w[2] = a->w_down;
  r.s[0] = a->s_up; r.s[1] = a->s_gate; r.s[2] = a->s_down;
  r.ln_w = a->ln_weight; r.ln_b = a->ln_bias;
  r.out = a->out;
  r.surprise = a->surprise;
  r.ws = static_cast<unsigned char*>(workspace);
  r.error_word = a->error_word;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const OutPtrs outs{{a->w_up_out, a->w_gate_out, a->w_down_out, a->s_up_out, a->s_gate_out, a->s_down_out}};
  const int D = r.D, F = r.F, CS = r.CS, T = r.T;
  const int nw = F / kCols;
  const int nchunks = (T + CS - 1) / CS;
  float* hq = reinterpret_cast<float*>(r.ws + WsLayout::hq(D, nw));
  float* wds = reinterpret_cast<float*>(r.ws + WsLayout::wds(D, nw));
  float* zp = reinterpret_cast<float*>(r.ws + WsLayout::zp(D, nw));
  const dim3 grid((unsigned)nw), blk(kThreads);
  // launches of up to kSegChunks chunks, each followed by the readout of its chunks
  for (int c0 = 0; c0 < nchunks; c0 += kSegChunks) {
    const int c1 = std::min(nchunks, c0 + kSegChunks);
    r.c_begin = c0;
    r.c_end = c1;
    if (c0 > 0) {  // the state the previous launch left
      for (int m = 0; m < 3; ++m) {
        r.w[m] = outs.p[m];
        r.s[m] = outs.p[3 + m];
      }
    }
    hipLaunchKernelGGL(k_resident_init, dim3(1), dim3(kThreads), 0, st, r.ws, outs,
                       c0 == 0 ? (a->force_timeout ? 2 : 1) : 0, a->error_word);
    switch (D) {
      case 128: hipLaunchKernelGGL(k_resident_update<2>, grid, blk, 0, st, r); break;
      case 256: hipLaunchKernelGGL(k_resident_update<4>, grid, blk, 0, st, r); break;
      default: hipLaunchKernelGGL(k_resident_update<8>, grid, blk, 0, st, r); break;
    }
    const int nseg = c1 - c0;
    const int nfull = (c1 == nchunks && T % CS != 0) ? nseg - 1 : nseg;  // chunks of CS tokens
    const int64_t tb = (int64_t)c0 * CS;
    if (nfull > 0)
      launch_saved_readout(nfull, CS, D, F, kReadoutSplits, hq, wds, (int64_t)F * D, zp, a->q + tb * D,
                           (int64_t)CS * D, a->ln_weight, a->ln_bias, a->eps, a->out + tb * D, (int64_t)CS * D, st);
    if (nfull < nseg) {  // the last chunk, shorter than CS
      const int64_t tl = (int64_t)(c0 + nfull) * CS;
      launch_saved_readout(1, (int)(T - tl), D, F, kReadoutSplits, hq + (int64_t)nfull * 64 * F,
                           wds + (int64_t)nfull * F * D, 0, zp, a->q + tl * D, 0, a->ln_weight, a->ln_bias, a->eps,
                           a->out + tl * D, 0, st);
    }
  }
  return launch_status("uttt_layer_update_resident");
}
