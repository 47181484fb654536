// One chunk's fast-weight updates for all L layers of the chunk-first shared schedule,
// written for gfx950 (MI355X).
//
// In the reference schedule (model/uttt_model.py:453-608) every layer of a chunk reads the
// chunk-start snapshot (W_s, S_s) for its readout and layer l's update is applied to the
// cursor left by layers 0..l-1 (model/uttt_layer.py:414-534 per layer).  Because every
// readout reads the snapshot, all L layers' keys, values, eta and alpha are known before the
// first update, and the L chained updates can be carried out without materialising the
// intermediate states.  Per row, with g_j = (K_j^T dU_j, K_j^T dG_j, H_j^T dZ_j) the
// gradient of layer j, clip c_j, decay d_j = 1 - mean(alpha_j) and momentum beta:
//
//   S_{l+1} = beta S_l - c_l g_l,   W_{l+1} = d_l W_l + S_{l+1}     (rows without tokens: no-op)
//   =>  W_l = a_l W_s + b_l S_s + sum_{j<l} gam_{l,j} g_j,   S_l = e_l S_s + sum_{j<l} sig_{l,j} g_j
//   e' = beta e, sig'_j = beta sig_j, sig'_l = -c_l, a' = d a, b' = d b + e', gam'_j = d gam_j + sig'_j
//
// so layer l's forward pass through W_l needs only products with the snapshot plus small
// products with earlier layers' activations:
//   U_l = a K_l W_up,s + b K_l S_up,s + sum_j gam_{l,j} (K_l K_j^T) dU_j          (G alike)
//   Z_l = H_l (a W_down,s + b S_down,s) + sum_j gam_{l,j} (H_l H_j^T) dZ_j
//   dH_l = dZ_l (a W_down,s + b S_down,s)^T + sum_j gam_{l,j} (dZ_l dZ_j^T) H_j
//   |g_l|^2 = <K_l K_l^T, dU_l dU_l^T + dG_l dG_l^T> + <H_l H_l^T, dZ_l dZ_l^T>
// and the state is written once, at the end of the chunk.  The (K W_s, K S_s) products of
// all layers form one GEMM with L*64 rows, so W_up/W_gate/S_up/S_gate are read once per
// chunk instead of once per layer, and W/S are written once per chunk instead of once per
// layer.
//
// Launch sequence (one stream), layers in groups (single layers while one launch's state read is
// small, else kPqGroup layers with the last kPqTail layers alone; pq_group_size):
// at the stage of a group's last layer, pq (K_l W_s, K_l S_s for the group's layers) and the
// key Gram rows of the group, then per layer l of the group: up (layer l - 1's clip / decay /
// recurrence step, then U, G, H) -> H-gram -> down (Z partials) -> k_ln_grad (dZ, loss) ->
// dZ-gram -> back (dU, dG, norm partials); stage 0 first initialises the coefficient table;
// stage L: the last layer's recurrence step (coef) and apply (final W, S and their bf16
// copies).  Stage l reads only layers <= l, so a caller can run it as soon as layer l's keys
// and values exist.
#include <algorithm>

#include "update_ln.h"
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {

namespace {

constexpr int KT = 64;
constexpr int kMaxChain = UTTT_MAX_CHAIN;
constexpr int kCoefStride = 4 + 2 * kMaxChain;  // a, b, e, #updating layers, gam[], sig[]
constexpr int kGam = 4, kSig = 4 + kMaxChain;
constexpr int kPqGroup = 4;  // layers per workgroup in the P/Q GEMM

template <typename T> constexpr int lds_ld() { return KT + Mma<T>::kPad; }

struct LayerPtrs {
  const void* p[kMaxChain];
};

// Per-layer activations: row b, token t of layer l at ptr[l] + b * row_stride + t * tok_stride.
struct Acts {
  LayerPtrs k, v, eta, alpha;
  int64_t kv_rs, kv_ts;     // k / v strides (elements)
  int64_t ea_rs, ea_ts;     // eta / alpha strides
};

template <typename T>
__device__ __forceinline__ const T* layer_row(const LayerPtrs& lp, int l, int b, int64_t rs) {
  return static_cast<const T*>(lp.p[l]) + (int64_t)b * rs;
}

// Store N (4 or 8) consecutive values to LDS as T with one vector write (dst aligned to N * sizeof(T)).
template <typename T, int N>
__device__ __forceinline__ void store_vec(T* dst, const float* v) {
  if constexpr (sizeof(T) == 2) {
    typedef bf16 vec_t __attribute__((ext_vector_type(N)));
    vec_t o;
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = from_f32<bf16>(v[i]);
    *reinterpret_cast<vec_t*>(dst) = o;
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) *reinterpret_cast<f32x4*>(dst + i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
  }
}

// dst[row][k] = scale * (register-staged fp32 64 x 64 tile), converted to T
template <typename T>
__device__ __forceinline__ void store_scaled(const RowStage<float, 64>& st, T* dst, int ldd, float scale) {
#pragma unroll
  for (int j = 0; j < RowStage<float, 64>::kN; ++j) {
    const int idx = threadIdx.x + j * kThreads;
    const int row = idx >> 4, c = idx & 15;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = scale * Lanes16<float>::get(st.r[j], q);
    store_vec<T, 4>(dst + row * ldd + c * 4, v);
  }
}

// Register-staged KT x 64 tile (KT source rows) of ca * X + cb * Y, source type S (fp32
// masters or their bf16 copies), transposed to [col][k].  One unit: 8 rows x 16 bytes.
template <typename S>
struct CombColStage {
  static constexpr int kVec = Lanes16<S>::kVec;
  static constexpr int kColGroups = 64 / kVec;
  static constexpr int kUnits = (KT / 8) * kColGroups;  // 128 (fp32) or 64 (bf16)
  uint4 rx[8], ry[8];
  __device__ __forceinline__ void load(const S* x, const S* y, int64_t ld, bool with_y) {
    if (threadIdx.x >= kUnits) return;
    const int kg = threadIdx.x / kColGroups, cg = threadIdx.x % kColGroups;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t off = (int64_t)(kg * 8 + i) * ld + cg * kVec;
      rx[i] = *reinterpret_cast<const uint4*>(x + off);
      ry[i] = with_y ? *reinterpret_cast<const uint4*>(y + off) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  template <typename T>
  __device__ __forceinline__ void store(T* dst, int ldd, float ca, float cb) const {
    if (threadIdx.x >= kUnits) return;
    const int kg = threadIdx.x / kColGroups, cg = threadIdx.x % kColGroups;
#pragma unroll
    for (int v = 0; v < kVec; ++v) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = ca * Lanes16<S>::get(rx[i], v) + cb * Lanes16<S>::get(ry[i], v);
      store_vec<T, 8>(dst + (cg * kVec + v) * ldd + kg * 8, o);
    }
  }
};

// Register-staged 64 x KT tile of ca * X + cb * Y (row-major source of type S), LDS [row][k].
template <typename S>
struct CombRowStage {
  static constexpr int kVec = Lanes16<S>::kVec;
  static constexpr int kPerRow = KT / kVec;
  static constexpr int kN = 64 * kPerRow / kThreads;  // 4 (fp32) or 2 (bf16)
  uint4 rx[kN], ry[kN];
  __device__ __forceinline__ void load(const S* x, const S* y, int64_t ld, bool with_y) {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kPerRow, c = idx % kPerRow;
      const int64_t off = (int64_t)row * ld + c * kVec;
      rx[j] = *reinterpret_cast<const uint4*>(x + off);
      ry[j] = with_y ? *reinterpret_cast<const uint4*>(y + off) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  template <typename T>
  __device__ __forceinline__ void store(T* dst, int ldd, float ca, float cb) const {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kPerRow, c = idx % kPerRow;
      float o[kVec];
#pragma unroll
      for (int v = 0; v < kVec; ++v) o[v] = ca * Lanes16<S>::get(rx[j], v) + cb * Lanes16<S>::get(ry[j], v);
      store_vec<T, kVec>(dst + row * ldd + c * kVec, o);
    }
  }
};

// ---------------------------------------------------------------------------
// 0. coefficient tables: a = e = 1, everything else 0 (a fill kernel, safe in graphs)
// ---------------------------------------------------------------------------
// The coefficient table of layer 0 (a = e = 1, the rest 0), and the Gram counters cleared (every
// Gram launch leaves them zero; this covers a fresh workspace).
__global__ void __launch_bounds__(kThreads) k_chain_init(float* coef, int n, unsigned* counters, int ncounters) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < ncounters) counters[i] = 0u;
  if (i >= n) return;
  const int slot = i % kCoefStride;
  coef[i] = (slot == 0 || slot == 2) ? 1.f : 0.f;
}

// ---------------------------------------------------------------------------
// 1. P/Q: pq[m][l][b] = K_l X_m for X = (W_up, S_up, W_gate, S_gate) of the snapshot,
//    G layers per workgroup sharing each staged X tile (G = 4: one layer per wave).
// ---------------------------------------------------------------------------
struct PqArgs {
  int B, L, C, D, F;
  int l_begin, l_count;  // layers of this launch
  Acts acts;
  const void* x[4];  // fp32 state or its bf16 copies
  void* pq;  // (4, L, B, 64, F) act dtype
  int s_only;  // products with S_up and S_gate only (m = 1, 3): the caller gave the W products
};

template <typename T, typename WT, int G>
__global__ void __launch_bounds__(kThreads, 2) k_chain_pq(const PqArgs a) {
  constexpr int LD = lds_ld<T>();
  __shared__ __align__(16) T bs[64 * LD];
  __shared__ __align__(16) T as[G * 64 * LD];
  const int nlg = (a.l_count + G - 1) / G;
  const int nm = a.s_only ? 2 : 4;  // matrices of this launch (the launch grid holds nm * F / 64 tiles per row)
  const RowTile rt = row_tile(blockIdx.x, a.B, nm * (a.F / 64) * nlg);
  if (!rt.valid) return;
  // tile = (m, F tile, layer group) with the layer groups that share an X tile adjacent
  const int mi = rt.tile / (nlg * (a.F / 64));
  const int b = rt.b, lg = rt.tile % nlg, ft = (rt.tile / nlg) % (a.F / 64), m = a.s_only ? 2 * mi + 1 : mi;
  const int f0 = ft * 64, l0 = a.l_begin + lg * G;
  const int nl = min(G, a.l_begin + a.l_count - l0);
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const WT* xs = static_cast<const WT*>(a.x[m]) + (int64_t)b * a.D * a.F + f0;
  const T* kr[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    kr[g] = layer_row<T>(a.acts.k, g < nl ? l0 + g : l0, b, a.acts.kv_rs);

  ColStage<WT, KT> xst;
  RowStage<T, KT> kst[G];
  xst.load(xs, a.F, KT, threadIdx.x);
#pragma unroll
  for (int g = 0; g < G; ++g)
    if (g < nl) kst[g].load(kr[g], a.acts.kv_ts, a.C);
  f32x16 acc[G < 4 ? 4 : G];  // G == 4: the four 32 x 32 quadrants of this wave's layer
#pragma unroll
  for (int g = 0; g < (G < 4 ? 4 : G); ++g) zero(acc[g]);
  for (int d0 = 0; d0 < a.D; d0 += KT) {
    xst.template store<T>(bs, LD);
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g < nl) kst[g].template store<T>(as + g * 64 * LD, LD);
    __syncthreads();
    if (d0 + KT < a.D) {
      xst.load(xs + (int64_t)(d0 + KT) * a.F, a.F, KT, threadIdx.x);
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (g < nl) kst[g].load(kr[g] + d0 + KT, a.acts.kv_ts, a.C);
    }
    if constexpr (G == kThreads / 64) {
      // one layer per wave, its whole 64 x 64 tile: the X fragments are read once per wave
      if (w < nl) wave_mma64<T, KT>(acc, as + w * 64 * LD, LD, bs, LD);
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (g < nl) wave_mma<T, KT>(acc[g], as + g * 64 * LD + wr * LD, LD, bs + wc * LD, LD);
    }
    __syncthreads();
  }
  if constexpr (G == kThreads / 64) {
    if (w >= nl) return;
    T* out = static_cast<T*>(a.pq) + (((int64_t)m * a.L + l0 + w) * a.B + b) * 64 * a.F + f0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row0 = (q >> 1) * 32, col = (q & 1) * 32 + acc_col();
#pragma unroll
      for (int i = 0; i < 16; ++i) out[(int64_t)(row0 + acc_row(i)) * a.F + col] = from_f32<T>(acc[q][i]);
    }
  } else {
    const int col = f0 + wc + acc_col();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g >= nl) continue;
      T* out = static_cast<T*>(a.pq) + (((int64_t)m * a.L + l0 + g) * a.B + b) * 64 * a.F;
#pragma unroll
      for (int i = 0; i < 16; ++i) out[(int64_t)(wr + acc_row(i)) * a.F + col] = from_f32<T>(acc[g][i]);
    }
  }
}

// bf16 activations and copies, one layer: the key rows and the X tiles go straight into LDS
// through a ring of kPqSlots d steps of 64 (X rows d hold 64 f columns: transposing reads); the
// products accumulate over d in the same order as the readout's key products.
constexpr int kPqSlots = 3;

constexpr int kPqRing = kPqSlots * 2 * 8192;  // bytes of LDS: kPqSlots steps of key rows and an X tile

// workgroup `bid` of the snapshot products (ring: kPqRing bytes of LDS, 1 KB aligned)
__device__ __forceinline__ void pq_lds_tile(const PqArgs& a, int bid, char* ring) {
  constexpr int kSlot = 2 * 8192;  // key rows, X tile
  constexpr int PER = 4;           // 16 row groups per step over 4 waves
  const int nF = a.F / 64, nm = a.s_only ? 2 : 4;
  const RowTile rt = row_tile(bid, a.B, nm * nF);
  if (!rt.valid) return;
  const int mi = rt.tile / nF, ft = rt.tile - mi * nF, b = rt.b;
  const int m = a.s_only ? 2 * mi + 1 : mi, f0 = ft * 64, l = a.l_begin;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const bf16* kr = layer_row<bf16>(a.acts.k, l, b, a.acts.kv_rs);
  const bf16* xs = static_cast<const bf16*>(a.x[m]) + (int64_t)b * a.D * a.F + f0;
  const int kts = (int)a.acts.kv_ts;
  int voff[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + 4 * i;  // groups 0..7: key rows, 8..15: X rows
    voff[i] = g < 8 ? row_src_off(g & 7, lane, kts) : slab_src_off(g & 7, lane, a.F);
  }
  const uint32_t ring0 = lds_addr(ring);
  const int nsteps = a.D / 64;
  const bool nt = stream_nt(a.B, a.D, a.F);  // the streamed state copies: non-temporal
  auto issue = [&](int step) {  // key rows past C are out of the buffer range: zeros
    const int d0 = step * 64;
    const uint32_t base = ring0 + (uint32_t)((step % kPqSlots) * kSlot);
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kr + d0, (uint32_t)(a.C * kts * 2));
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(xs + (int64_t)d0 * a.F, (uint32_t)(64 * a.F * 2));
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int g = w + 4 * i;
      buffer_load_lds16(g >= 8 && nt, g < 8 ? rk : rx, lds_ptr(base + (uint32_t)(g * 1024)), voff[i]);
    }
  };
  for (int j = 0; j < min(nsteps, kPqSlots - 1); ++j) issue(j);
  uint32_t ta[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) ta[k] = row_frag_addr(ring0, wr, lane, k);
  const uint32_t tx = slab_tr_addr(ring0 + 8192u, wc, lane);
  f32x16 acc;
  zero(acc);
  for (int step = 0; step < nsteps; ++step) {
    wait_steps<PER, kPqSlots - 2>(min(nsteps - 1, step + kPqSlots - 2) - step);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the last step's slot is free
    if (step + kPqSlots - 1 < nsteps) issue(step + kPqSlots - 1);
    const uint32_t so = (uint32_t)((step % kPqSlots) * kSlot);
    bf16x8 fa[4], fx[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) fa[k] = lds_read_bf16x8<0>(ta[k] + so);
    slab_frags(tx + so, fx);
    lds_wait_frags(fa, fx);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fx[k], acc, 0, 0, 0);
  }
  bf16* out = static_cast<bf16*>(a.pq) + (((int64_t)m * a.L + l) * a.B + b) * 64 * a.F + f0;
  const int col = wc + acc_col();
#pragma unroll
  for (int i = 0; i < 16; ++i) out[(int64_t)(wr + acc_row(i)) * a.F + col] = from_f32<bf16>(acc[i]);
}

__global__ void __launch_bounds__(kThreads) k_chain_pq_lds(const PqArgs a) {
  __shared__ __align__(1024) char ring[kPqRing];
  pq_lds_tile(a, blockIdx.x, ring);
}

// ---------------------------------------------------------------------------
// 2. Gram blocks G[l][j] = X_l X_j^T over the feature dimension for the layers l in
//    [layer, layer_end) and every j <= l, operands loaded straight from global memory (rows
//    >= C are 0).
// ---------------------------------------------------------------------------
struct GramArgs {
  int B, L, C, kd, LL, layer, layer_end;
  int64_t rs, ts;  // row / token strides of X (elements)
  LayerPtrs x;
  float* out;      // row b's block row l at out + (b * out_rows + out_r0 + l * out_lstep) * LL
  int out_rows, out_r0, out_lstep;
  // bf16 path: the feature range is split over `splits` workgroups per block; their partial
  // blocks (4096 floats each) go to `part` and the last of them, counted in `counters` (one per
  // row and block of the launch, zero before the launch and left zero), sums them into `out`
  float* part;
  unsigned* counters;
  int splits;
  // optional (bf16 path): block (l, j) also written as bf16(gamma_j * G) to scaled at the same
  // place (row b's rows at scaled + b * out_rows * LL), gamma_j = coef[b * kCoefStride + kGam + j]:
  // the back pass's correction operand, rounded as that pass rounded it from the fp32 block
  bf16* scaled;
  const float* coef;
};

// 32 x 32 quadrant tiles of the block rows [l0, l1): row l has 4 (l + 1) of them
__host__ __device__ inline int gram_tiles(int l0, int l1) { return 2 * (l1 * (l1 + 1) - l0 * (l0 + 1)); }

// One 32 x 32 quadrant per workgroup; the kGramWaves waves take an equal share of the
// feature range (in steps of 16) each and their partial sums meet in LDS.
constexpr int kGramWaves = 8;

template <typename T>
__global__ void __launch_bounds__(kGramWaves * 64) k_chain_gram(const GramArgs a) {
  __shared__ float part[(kGramWaves - 1) * 16 * 64];
  const RowTile rt = row_tile(blockIdx.x, a.B, gram_tiles(a.layer, a.layer_end));
  if (!rt.valid) return;
  int l = a.layer, rem = rt.tile;
  while (rem >= 4 * (l + 1)) {  // at most layer_end - layer steps
    rem -= 4 * (l + 1);
    ++l;
  }
  const int q = rem & 3;  // 32 x 32 quadrant of the 64 x 64 block
  const int j = rem >> 2, b = rt.b;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int ti = (q >> 1) * 32 + r, tj = (q & 1) * 32 + r;
  const int nk = a.kd / 16, kb = 16 * (nk * wave / kGramWaves), ke = 16 * (nk * (wave + 1) / kGramWaves);
  const T* xa = layer_row<T>(a.x, l, b, a.rs) + (int64_t)ti * a.ts;
  const T* xb = layer_row<T>(a.x, j, b, a.rs) + (int64_t)tj * a.ts;
  const bool va = ti < a.C, vb = tj < a.C;
  f32x16 acc;
  zero(acc);
  if constexpr (sizeof(T) == 2) {
    for (int k0 = kb; k0 < ke; k0 += 128) {  // the range is a multiple of 16; 8 steps of 16 in flight
      uint4 ra[8], rb[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const bool in = k0 + u * 16 < ke;
        ra[u] = va && in ? *reinterpret_cast<const uint4*>(xa + k0 + u * 16 + h * 8) : make_uint4(0u, 0u, 0u, 0u);
        rb[u] = vb && in ? *reinterpret_cast<const uint4*>(xb + k0 + u * 16 + h * 8) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8*>(&ra[u]),
                                                      *reinterpret_cast<const bf16x8*>(&rb[u]), acc, 0, 0, 0);
    }
  } else {
    for (int k0 = kb; k0 < ke; k0 += 32) {  // 4 groups of 8 (each lane 4 consecutive k)
      f32x4 av[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool in = k0 + u * 8 < ke;
        av[u] = va && in ? *reinterpret_cast<const f32x4*>(xa + k0 + u * 8 + h * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
        bv[u] = vb && in ? *reinterpret_cast<const f32x4*>(xb + k0 + u * 8 + h * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u][e], bv[u][e], acc, 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) part[((wave - 1) * 16 + i) * 64 + lane] = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;
  float* out = a.out + ((int64_t)b * a.out_rows + a.out_r0 + l * a.out_lstep) * a.LL;
  const int c = j * 64 + (q & 1) * 32 + r;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float v = acc[i];
#pragma unroll
    for (int u = 0; u < kGramWaves - 1; ++u) v += part[(u * 16 + i) * 64 + lane];
    const int row = (q >> 1) * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
    out[(int64_t)row * a.LL + c] = v;
  }
}

// bf16 activations: one workgroup per 64 x 64 block (b, l, j) and slice of kGramSplitSteps 64-wide
// feature steps.  Four waves, one 32 x 32 quadrant each, stream coalesced 64-wide row tiles of X_l
// and X_j straight into LDS through a ring of kGramSlots steps.  With one slice the block is written
// directly; otherwise every workgroup stores its partial block with device-coherent stores, waits
// for them to complete and raises the block's counter, and the workgroup that completes the count
// reads the partials back with device-coherent loads (no cache write-back or invalidate between
// XCDs), sums them in slice order (deterministic) and returns the counter to zero.
constexpr int kGramSlots = 3;
// 1024-feature slices: in the chunk-first prefill the chain shares the GPU with the forward
// pass, and fewer, longer Gram workgroups measured faster there than 512- or 256-feature slices
constexpr int kGramSplitSteps = 16;

__host__ __device__ inline int gram_blocks(int l0, int l1) { return (l1 * (l1 + 1) - l0 * (l0 + 1)) / 2; }
__host__ __device__ inline int gram_splits(int kd) { return (kd / 64 + kGramSplitSteps - 1) / kGramSplitSteps; }

constexpr int kGramRing = kGramSlots * 16384;  // bytes of LDS: kGramSlots steps of X_l and X_j rows

// workgroup `bid` of the Gram blocks (ring: kGramRing bytes of LDS; last: an LDS int)
__device__ __forceinline__ void gram_lds_tile(const GramArgs& a, int bid, char* ring, int& last) {
  constexpr int kSlot = 16384;  // X_l rows, X_j rows (64 x 64 bf16 each)
  constexpr int PER = 4;        // 16 row groups per step over 4 waves
  const int nblk = gram_blocks(a.layer, a.layer_end);
  const RowTile rt = row_tile(bid, a.B, nblk * a.splits);
  if (!rt.valid) return;
  const int blk = rt.tile / a.splits, sp = rt.tile % a.splits;
  int l = a.layer, j = blk;
  while (j >= l + 1) {  // at most layer_end - layer steps
    j -= l + 1;
    ++l;
  }
  const int b = rt.b;
  const int q = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = a.kd / 64;
  const int s_begin = sp * kGramSplitSteps, mine = min(n, s_begin + kGramSplitSteps) - s_begin;
  const bf16* xa = layer_row<bf16>(a.x, l, b, a.rs);
  const bf16* xb = layer_row<bf16>(a.x, j, b, a.rs);
  const int ts = (int)a.ts;
  int voff[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) voff[i] = row_src_off((q + 4 * i) & 7, lane, ts);
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int t) {  // step t of this slice; rows past C are out of the buffer range: zeros
    const int k0 = (s_begin + t) * 64;
    const uint32_t base = ring0 + (uint32_t)((t % kGramSlots) * kSlot);
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(xa + k0, (uint32_t)(a.C * ts * 2));
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(xb + k0, (uint32_t)(a.C * ts * 2));
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int g = q + 4 * i;  // groups 0..7: X_l rows, 8..15: X_j rows
      buffer_load_lds_raw(g < 8 ? ra : rb, lds_ptr(base + (uint32_t)(g * 1024)), 16, voff[i], 0, 0, 0);
    }
  };
  for (int t = 0; t < min(mine, kGramSlots - 1); ++t) issue(t);
  uint32_t ta[4], tb[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ta[k] = row_frag_addr(ring0, (q >> 1) * 32, lane, k);
    tb[k] = row_frag_addr(ring0 + 8192u, (q & 1) * 32, lane, k);
  }
  f32x16 acc;
  zero(acc);
  for (int t = 0; t < mine; ++t) {
    wait_steps<PER, kGramSlots - 2>(min(mine - 1, t + kGramSlots - 2) - t);
    __builtin_amdgcn_s_barrier();
    if (t + kGramSlots - 1 < mine) issue(t + kGramSlots - 1);
    const uint32_t so = (uint32_t)((t % kGramSlots) * kSlot);
    bf16x8 fa[4], fb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      fa[k] = lds_read_bf16x8<0>(ta[k] + so);
      fb[k] = lds_read_bf16x8<0>(tb[k] + so);
    }
    lds_wait_frags(fa, fb);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fb[k], acc, 0, 0, 0);
  }
  const int64_t out_off = ((int64_t)b * a.out_rows + a.out_r0 + l * a.out_lstep) * a.LL;
  float* out = a.out + out_off;
  const int c = j * 64 + (q & 1) * 32 + acc_col();
  auto write = [&](const float (&v)[16]) {
    const float gj = a.scaled != nullptr ? a.coef[(int64_t)b * kCoefStride + kGam + j] : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t o = (int64_t)((q >> 1) * 32 + acc_row(i)) * a.LL + c;
      out[o] = v[i];
      if (a.scaled != nullptr) a.scaled[out_off + o] = static_cast<bf16>(gj * v[i]);
    }
  };
  if (a.splits == 1) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = acc[i];
    write(v);
    return;
  }
  const int64_t blk_id = (int64_t)b * nblk + blk;
  float* mine_part = a.part + (blk_id * a.splits + sp) * 4096;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    __hip_atomic_store(mine_part + (q * 16 + i) * 64 + lane, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(a.counters + blk_id, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == (unsigned)(a.splits - 1);
  }
  __syncthreads();
  if (!last) return;
  const float* parts = a.part + blk_id * a.splits * 4096;
  float sum[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) sum[i] = 0.f;
  for (int u = 0; u < a.splits; ++u) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i] = __hip_atomic_load(parts + (int64_t)u * 4096 + (q * 16 + i) * 64 + lane, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int i = 0; i < 16; ++i) sum[i] += v[i];
  }
  write(sum);
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + blk_id, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void __launch_bounds__(kThreads) k_chain_gram_lds(const GramArgs a) {
  __shared__ __align__(1024) char ring[kGramRing];
  __shared__ int last;
  gram_lds_tile(a, blockIdx.x, ring, last);
}

// Part 1 of a single-layer stage in one launch: the snapshot products' workgroups (the first
// npq ids), then the key Gram row's (both read only layer l's keys and the chunk-start state, so
// they need no order between them); one launch instead of two per layer.
static_assert(sizeof(PqArgs) + sizeof(GramArgs) + 16 <= 4096, "the fused launch's arguments fit the kernarg segment");

__global__ void __launch_bounds__(kThreads) k_chain_keys_lds(const PqArgs pa, const GramArgs ga, int npq) {
  __shared__ __align__(1024) char ring[kPqRing > kGramRing ? kPqRing : kGramRing];
  __shared__ int last;
  if ((int)blockIdx.x < npq)
    pq_lds_tile(pa, blockIdx.x, ring);
  else
    gram_lds_tile(ga, (int)blockIdx.x - npq, ring, last);
}

// ---------------------------------------------------------------------------
// 3a. Per row: |g_l|^2, clip, decay, active flag, surprise; advance the recurrences.
// ---------------------------------------------------------------------------
struct CoefArgs {
  int B, C, LL, l, nF;
  float beta, max_norm, min_row_surprise;
  const float* npart;
  const float* hh;
  const float* zz;
  Acts acts;
  const float* mask;
  int64_t mask_rs;
  const float* loss;  // (B, 64)
  const float* src;   // coefficient table before layer l (B, kCoefStride)
  float* dst;         // coefficient table after layer l
  float* surprise;    // (L,)
  float* row_loss;    // optional (L, B, 2)
};

// Layer l's clip, decay and active flag for row b, and the coefficient table after layer l,
// left in `out` (LDS, kCoefStride floats).  All 256 threads call it.  With `publish` the
// table goes to a.dst and the layer's surprise outputs are written.
template <typename T>
__device__ void advance_coef(const CoefArgs& a, int b, float* out, float* red, bool publish) {
  __shared__ float sc[3];
  const float* src = a.src + (int64_t)b * kCoefStride;
  for (int i = threadIdx.x; i < kCoefStride; i += kThreads) out[i] = src[i];
  float n2 = 0.f;
  for (int i = threadIdx.x; i < a.nF; i += kThreads) n2 += a.npart[(int64_t)b * a.nF + i];
  const float* hh = a.hh + (int64_t)b * 64 * a.LL + a.l * 64;
  const float* zz = a.zz + (int64_t)b * 64 * a.LL + a.l * 64;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    const int64_t off = (int64_t)(idx >> 6) * a.LL + (idx & 63);
    n2 += hh[off] * zz[off];
  }
  const int t = threadIdx.x;
  const T* al = layer_row<T>(a.acts.alpha, a.l, b, a.acts.ea_rs);
  float mt = 0.f, at = 0.f;
  if (t < a.C) {
    mt = a.mask != nullptr ? a.mask[(int64_t)b * a.mask_rs + t] : 1.f;
    at = to_f32(al[(int64_t)t * a.acts.ea_ts]);
  }
  const float lt = t < 64 ? a.loss[b * 64 + t] : 0.f;
  __shared__ float red5[20];
  float sums[5] = {n2, at * mt, mt, mt != 0.f ? 1.f : 0.f, lt};
  block_sums<5>(sums, red5);
  n2 = sums[0];
  const float asum = sums[1], msum = sums[2], any = sums[3], lsum = sums[4];
  if (threadIdx.x == 0) {
    const float denom = a.mask != nullptr ? fmaxf(msum, 1.f) : (float)a.C;
    const float row_mean = lsum / fmaxf(a.mask != nullptr ? msum : (float)a.C, 1.f);
    const bool gated_off = a.min_row_surprise > 0.f && row_mean < a.min_row_surprise;
    const bool active = (a.mask == nullptr || any > 0.f) && !gated_off;
    sc[0] = a.max_norm > 0.f ? fminf(a.max_norm * (1.0f / sqrtf(n2 + 1e-8f)), 1.0f) : 1.0f;
    sc[1] = 1.0f - asum / denom;
    sc[2] = active ? 1.f : 0.f;
    if (publish && a.row_loss != nullptr) {
      a.row_loss[((int64_t)a.l * a.B + b) * 2] = lsum;
      a.row_loss[((int64_t)a.l * a.B + b) * 2 + 1] = a.mask != nullptr ? msum : (float)a.C;
    }
  }
  if (publish && b == 0 && threadIdx.x >= 192) {
    // batch-global surprise of this layer: masked token losses over all rows / valid tokens
    const int lane = threadIdx.x - 192;
    float num = 0.f, den = 0.f;
    for (int i = lane; i < a.B * 64; i += 64) {
      const int bb = i >> 6, tt = i & 63;
      num += a.loss[i];
      if (tt < a.C) den += a.mask != nullptr ? a.mask[(int64_t)bb * a.mask_rs + tt] : 1.f;
    }
    num = wave_sum(num);
    den = wave_sum(den);
    if (lane == 0) a.surprise[a.l] = a.mask != nullptr ? num / fmaxf(den, 1.f) : num / den;
  }
  __syncthreads();
  if (sc[2] != 0.f) {  // without tokens, or gated off, the layer leaves the row unchanged
    const float c = sc[0], d = sc[1];
    const int j = threadIdx.x;
    const float e_new = a.beta * src[2];
    if (j <= a.l) {
      const float s_new = j < a.l ? a.beta * src[kSig + j] : -c;
      out[kSig + j] = s_new;
      out[kGam + j] = d * src[kGam + j] + s_new;
    }
    if (threadIdx.x == 0) {
      out[0] = d * src[0];
      out[1] = d * src[1] + e_new;
      out[2] = e_new;
      out[3] = src[3] + 1.f;
    }
  }
  __syncthreads();
  if (publish) {
    float* dst = a.dst + (int64_t)b * kCoefStride;
    for (int i = threadIdx.x; i < kCoefStride; i += kThreads) dst[i] = out[i];
  }
}

// The last layer's recurrence step (every other layer's runs inside the next k_chain_up).
template <typename T>
__global__ void __launch_bounds__(kThreads) k_chain_coef(const CoefArgs a) {
  __shared__ float red[4];
  __shared__ float out[kCoefStride];
  advance_coef<T>(a, blockIdx.x, out, red, true);
}

// ---------------------------------------------------------------------------
// 3. Layer l forward through W_l: U, G (fp32, kept for the backward), H (act dtype)
// ---------------------------------------------------------------------------
struct UpArgs {
  int B, L, C, D, F, LL, l;
  CoefArgs prev;      // layer l - 1's recurrence step (l > 0): its table -> the table of layer l
  const float* coef;  // table of layer l when l == 0
  const void* pq;
  const float* kk;  // (B, LL, LL)
  const void* du_all;
  const void* dg_all;  // (L, B, 64, F)
  float* u_cur;
  float* g_cur;  // (B, 64, F)
  void* h_all;
};

template <typename T>
__global__ void __launch_bounds__(kThreads) k_chain_up(const UpArgs a) {
  constexpr int LD = lds_ld<T>();
  __shared__ __align__(16) T as[2][64 * LD];
  __shared__ __align__(16) T bu[2][64 * LD];
  __shared__ __align__(16) T bg[2][64 * LD];
  __shared__ float cf[kCoefStride];
  __shared__ float red[4];
  const RowTile rt = row_tile(blockIdx.x, a.B, a.F / 64);
  if (!rt.valid) return;
  const int ft = rt.tile, b = rt.b, f0 = ft * 64;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  // loads that do not depend on the coefficients go out first: this tile's snapshot products
  // and the first correction tiles, so their latency overlaps the recurrence step below
  const int64_t plane = (int64_t)a.L * a.B * 64 * a.F;
  const T* pl = static_cast<const T*>(a.pq) + ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
  const int col = wc + acc_col();
  T pw_u[16], pw_g[16], ps_u[16], ps_g[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
    pw_u[i] = pl[off];
    ps_u[i] = pl[plane + off];
    pw_g[i] = pl[2 * plane + off];
    ps_g[i] = pl[3 * plane + off];
  }
  constexpr int U = ColStage<T, 64>::kUnits;
  const bool up_half = threadIdx.x < U;
  const int unit = up_half ? (int)threadIdx.x : min((int)threadIdx.x - U, U);
  const T* dsrc = static_cast<const T*>(up_half ? a.du_all : a.dg_all) + (int64_t)b * 64 * a.F + f0;
  const int64_t lstride = (int64_t)a.B * 64 * a.F;
  const float* kk = a.kk + ((int64_t)b * a.LL + a.l * 64) * a.LL;
  RowStage<float, 64> kst;
  ColStage<T, 64> st;
  if (a.l > 0) {
    kst.load(kk, a.LL, 64);
    st.load(dsrc, a.F, 64, unit);
    // the previous layer's recurrence step: every F tile of the row derives the same table,
    // the first one publishes it (and that layer's surprise) for the layer's later kernels
    advance_coef<T>(a.prev, b, cf, red, ft == 0);
  } else {
    for (int i = threadIdx.x; i < kCoefStride; i += kThreads) cf[i] = a.coef[(int64_t)b * kCoefStride + i];
    __syncthreads();
  }
  const float ca = cf[0], cb = cf[1];
  float pu[16], pg[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pu[i] = ca * to_f32(pw_u[i]) + cb * to_f32(ps_u[i]);
    pg[i] = ca * to_f32(pw_g[i]) + cb * to_f32(ps_g[i]);
  }
  f32x16 au, ag;
  zero(au);
  zero(ag);
  for (int j = 0; j < a.l; ++j) {
    const int buf = j & 1;
    store_scaled<T>(kst, as[buf], LD, cf[kGam + j]);
    st.template store<T>(up_half ? bu[buf] : bg[buf], LD);
    __syncthreads();
    if (j + 1 < a.l) {
      kst.load(kk + (j + 1) * 64, a.LL, 64);
      st.load(dsrc + (j + 1) * lstride, a.F, 64, unit);
    }
    wave_mma<T, 64>(au, as[buf] + wr * LD, LD, bu[buf] + wc * LD, LD);
    wave_mma<T, 64>(ag, as[buf] + wr * LD, LD, bg[buf] + wc * LD, LD);
  }
  const int64_t lane_base = (int64_t)b * 64 * a.F + f0;
  T* h = static_cast<T*>(a.h_all) + ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
    const float u = pu[i] + au[i];
    const float g = pg[i] + ag[i];
    a.u_cur[lane_base + off] = u;
    a.g_cur[lane_base + off] = g;
    h[off] = from_f32<T>((g * sigmoidf_acc(g)) * u);
  }
}

// bf16 activations: the correction loop's operands go straight into LDS -- per layer j < l the
// key Gram block K_l K_j^T (fp32, 16 KB; scaled by gam_j and rounded to bf16 as the A fragments
// are read) and the du_j, dg_j slabs (8 KB each, transposing reads) -- through a ring of
// kUpSlots slots: one workgroup per CU, loads run up to three layers ahead.
constexpr int kUpSlots = 4;
constexpr int kUpSlotBytes = 16384 + 2 * 8192;

// Key Gram block in LDS: 64 rows of 64 fp32 (256 bytes); 16-byte piece p of row r sits in slot
// p ^ (r & 15), so the 16 rows one read instruction serves per cycle hit distinct banks.  One
// load instruction covers a row group of 4 rows.
__device__ __forceinline__ int gram_src_off(int rg, int lane, int ld) {
  const int r = 4 * rg + (lane >> 4);
  return (r * ld + ((lane & 15) ^ (r & 15)) * 4) * 4;
}


__global__ void __launch_bounds__(kThreads, 1) k_chain_up_lds(const UpArgs a) {
  __shared__ __align__(1024) char ring[kUpSlots * kUpSlotBytes];
  __shared__ float cf[kCoefStride];
  __shared__ float red[4];
  const RowTile rt = row_tile(blockIdx.x, a.B, a.F / 64);
  if (!rt.valid) return;
  const int ft = rt.tile, b = rt.b, f0 = ft * 64;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  // loads that do not depend on the coefficients go out first: this tile's snapshot products
  // and the first correction layers, so their latency overlaps the recurrence step below
  const int64_t plane = (int64_t)a.L * a.B * 64 * a.F;
  const bf16* pl = static_cast<const bf16*>(a.pq) + ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
  const int col = wc + acc_col();
  bf16 pw_u[16], pw_g[16], ps_u[16], ps_g[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
    pw_u[i] = pl[off];
    ps_u[i] = pl[plane + off];
    pw_g[i] = pl[2 * plane + off];
    ps_g[i] = pl[3 * plane + off];
  }
  const int64_t lstride = (int64_t)a.B * 64 * a.F;
  const bf16* du0 = static_cast<const bf16*>(a.du_all) + (int64_t)b * 64 * a.F + f0;
  const bf16* dg0 = static_cast<const bf16*>(a.dg_all) + (int64_t)b * 64 * a.F + f0;
  const float* kk0 = a.kk + ((int64_t)b * a.LL + a.l * 64) * a.LL;  // layer j's block at + 64 j
  int kk_off[4], d_off[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) kk_off[i] = gram_src_off(w + 4 * i, lane, a.LL);
#pragma unroll
  for (int i = 0; i < 2; ++i) d_off[i] = slab_src_off(w + 4 * i, lane, a.F);
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int j) {  // 8 loads per wave
    const uint32_t base = ring0 + (uint32_t)((j % kUpSlots) * kUpSlotBytes);
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(kk0 + 64 * j, (uint32_t)(64 * a.LL * 4));
    const __amdgpu_buffer_rsrc_t ur = buffer_rsrc(du0 + j * lstride, (uint32_t)(64 * a.F * 2));
    const __amdgpu_buffer_rsrc_t gr = buffer_rsrc(dg0 + j * lstride, (uint32_t)(64 * a.F * 2));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      buffer_load_lds_raw(kr, lds_ptr(base + (uint32_t)((w + 4 * i) * 1024)), 16, kk_off[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      buffer_load_lds_raw(ur, lds_ptr(base + 16384u + (uint32_t)((w + 4 * i) * 1024)), 16, d_off[i], 0, 0, 0);
      buffer_load_lds_raw(gr, lds_ptr(base + 24576u + (uint32_t)((w + 4 * i) * 1024)), 16, d_off[i], 0, 0, 0);
    }
  };
  for (int j = 0; j < min(a.l, kUpSlots - 1); ++j) issue(j);
  if (a.l > 0) {
    // the previous layer's recurrence step: every F tile of the row derives the same table,
    // the first one publishes it (and that layer's surprise) for the layer's later kernels
    advance_coef<bf16>(a.prev, b, cf, red, ft == 0);
  } else {
    for (int i = threadIdx.x; i < kCoefStride; i += kThreads) cf[i] = a.coef[(int64_t)b * kCoefStride + i];
    __syncthreads();
  }
  // A fragments (k step s): row i = wr + lane % 32, fp32 pieces 4 s + 2 h and + 1 (h = lane / 32)
  const int ia = wr + (lane & 31), ha = lane >> 5;
  uint32_t aaddr[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) aaddr[q] = ring0 + (uint32_t)(ia * 256 + (((2 * q + 2 * ha - (q & 1)) ^ (ia & 15)) * 16));
  const uint32_t tu = slab_tr_addr(ring0 + 16384u, wc, lane), tg = slab_tr_addr(ring0 + 24576u, wc, lane);
  const uint32_t cf_gam = lds_addr(cf) + 4u * kGam;
  f32x16 au, ag;
  zero(au);
  zero(ag);
  for (int j = 0; j < a.l; ++j) {
    // this wave's loads of layer j are done once those of the later issued layers remain
    wait_steps<8, kUpSlots - 2>(min(a.l - 1, j + kUpSlots - 2) - j);
    __builtin_amdgcn_s_barrier();  // every wave's loads of layer j landed; layer j - 1's slot is free
    if (j + kUpSlots - 1 < a.l) issue(j + kUpSlots - 1);
    const uint32_t so = (uint32_t)((j % kUpSlots) * kUpSlotBytes);
    bf16x8 fu[4], fg[4];
    slab_frags(tu + so, fu);
    slab_frags(tg + so, fg);
    f32x4 kv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) kv[q] = lds_read_b128(aaddr[q] + so);
    float gj = lds_read_b32(cf_gam + 4u * (uint32_t)j);
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fu[0]), "+v"(fu[1]), "+v"(fu[2]), "+v"(fu[3]), "+v"(fg[0]), "+v"(fg[1]), "+v"(fg[2]),
                   "+v"(fg[3]), "+v"(kv[0]), "+v"(kv[1]), "+v"(kv[2]), "+v"(kv[3]), "+v"(kv[4]), "+v"(kv[5]),
                   "+v"(kv[6]), "+v"(kv[7]), "+v"(gj));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      bf16x8 fa;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        fa[e] = static_cast<bf16>(gj * kv[2 * k][e]);
        fa[4 + e] = static_cast<bf16>(gj * kv[2 * k + 1][e]);
      }
      au = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fu[k], au, 0, 0, 0);
      ag = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fg[k], ag, 0, 0, 0);
    }
  }
  const float ca = cf[0], cb = cf[1];
  const int64_t lane_base = (int64_t)b * 64 * a.F + f0;
  bf16* h = static_cast<bf16*>(a.h_all) + ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
    const float u = (ca * to_f32(pw_u[i]) + cb * to_f32(ps_u[i])) + au[i];
    const float g = (ca * to_f32(pw_g[i]) + cb * to_f32(ps_g[i])) + ag[i];
    a.u_cur[lane_base + off] = u;
    a.g_cur[lane_base + off] = g;
    h[off] = from_f32<bf16>((g * sigmoidf_acc(g)) * u);
  }
}

// ---------------------------------------------------------------------------
// 4. Z partials: splits < nsplit take H_l (a W_down,s + b S_down,s) over an F range;
//    split nsplit (l > 0) takes sum_j gam_j (H_l H_j^T) dZ_j.
// ---------------------------------------------------------------------------
struct DownArgs {
  int B, L, C, D, F, LL, l, nsplit;
  const float* coef;
  const void* h_all;
  const void* wd;
  const void* sd;  // (B, F, D): fp32 state or its bf16 copies
  const float* hh;  // (B, 64, LL): H_l H_j^T
  const bf16* hhb;  // (B, 64, LL): bf16(gamma_j H_l H_j^T), the bf16 pass's correction operand
  const void* dz_all;  // (L, B, 64, D)
  float* zp;           // (nsplit + correction splits, B, 64, D)
};

// layers j per correction split (3 measured faster in the prefills than 1, 2 or 4)
constexpr int kCorrPerSplit = 3;

template <typename T, typename WT>
__global__ void __launch_bounds__(kThreads) k_chain_down(const DownArgs a) {
  constexpr int LD = lds_ld<T>();
  __shared__ __align__(16) T hs[2][64 * LD];
  __shared__ __align__(16) T ws[2][64 * LD];
  const int nsp = a.nsplit + (a.l + kCorrPerSplit - 1) / kCorrPerSplit;
  const RowTile rt = row_tile(blockIdx.x, a.B, (a.D / 64) * nsp);
  if (!rt.valid) return;
  const int dt = rt.tile % (a.D / 64), split = rt.tile / (a.D / 64), b = rt.b, d0 = dt * 64;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const float* cf = a.coef + (int64_t)b * kCoefStride;
  f32x16 acc;
  zero(acc);
  if (split < a.nsplit) {
    const float ca = cf[0], cb = cf[1];
    const bool with_s = cb != 0.f;
    const int nF = a.F / 64;
    const int f_begin = (nF * split / a.nsplit) * 64, f_end = (nF * (split + 1) / a.nsplit) * 64;
    const T* h = static_cast<const T*>(a.h_all) + ((int64_t)a.l * a.B + b) * 64 * a.F;
    const int64_t mat = (int64_t)a.F * a.D;
    const WT* wd = static_cast<const WT*>(a.wd) + b * mat + d0;
    const WT* sd = static_cast<const WT*>(a.sd) + b * mat + d0;
    RowStage<T, KT> hst;
    CombColStage<WT> wst;
    if (f_begin < f_end) {
      hst.load(h + f_begin, a.F, 64);
      wst.load(wd + (int64_t)f_begin * a.D, sd + (int64_t)f_begin * a.D, a.D, with_s);
    }
    int buf = 0;
    for (int f0 = f_begin; f0 < f_end; f0 += KT, buf ^= 1) {
      hst.template store<T>(hs[buf], LD);
      wst.template store<T>(ws[buf], LD, ca, cb);
      __syncthreads();
      if (f0 + KT < f_end) {
        hst.load(h + f0 + KT, a.F, 64);
        wst.load(wd + (int64_t)(f0 + KT) * a.D, sd + (int64_t)(f0 + KT) * a.D, a.D, with_s);
      }
      wave_mma<T, KT>(acc, hs[buf] + wr * LD, LD, ws[buf] + wc * LD, LD);
    }
  } else {
    const int j_begin = (split - a.nsplit) * kCorrPerSplit;
    const int j_end = min(a.l, j_begin + kCorrPerSplit);
    const T* dsrc = static_cast<const T*>(a.dz_all) + (int64_t)b * 64 * a.D + d0;
    const int64_t lstride = (int64_t)a.B * 64 * a.D;
    const float* hh = a.hh + (int64_t)b * 64 * a.LL;
    RowStage<float, 64> hst;
    ColStage<T, 64> st;
    if (j_begin < j_end) {
      hst.load(hh + j_begin * 64, a.LL, 64);
      st.load(dsrc + j_begin * lstride, a.D, 64, threadIdx.x);
    }
    for (int j = j_begin; j < j_end; ++j) {
      const int buf = (j - j_begin) & 1;
      store_scaled<T>(hst, hs[buf], LD, cf[kGam + j]);
      st.template store<T>(ws[buf], LD);
      __syncthreads();
      if (j + 1 < j_end) {
        hst.load(hh + (j + 1) * 64, a.LL, 64);
        st.load(dsrc + (j + 1) * lstride, a.D, 64, threadIdx.x);
      }
      wave_mma<T, 64>(acc, hs[buf] + wr * LD, LD, ws[buf] + wc * LD, LD);
    }
  }
  float* zp = a.zp + (((int64_t)split * a.B + b) * 64) * a.D + d0;
  const int col = wc + acc_col();
#pragma unroll
  for (int i = 0; i < 16; ++i) zp[(int64_t)(wr + acc_row(i)) * a.D + col] = acc[i];
}


// bf16 activations and copies: a main split streams H_l rows (k = f) with the W_down and S_down
// tiles of its F range (rows f hold 64 d columns: transposing reads), a correction split the H
// Gram blocks gamma_j H_l H_j^T (bf16, scaled and rounded by the Gram launch: row tiles read as
// is) with the dZ_j slabs, straight into LDS through a ring of kDownSlots steps.  H (a W_d + b S_d) is formed as a H W_d + b H S_d.
constexpr int kDownSlots = 3;

__global__ void __launch_bounds__(kThreads) k_chain_down_lds(const DownArgs a) {
  constexpr int kSlot = 24576;  // H, W_d, S_d tiles; or the Gram block (16 KB) and the dZ slab
  constexpr int PER = 6;        // 24 row groups per step over 4 waves
  __shared__ __align__(1024) char ring[kDownSlots * kSlot];
  const int nsp = a.nsplit + (a.l + kCorrPerSplit - 1) / kCorrPerSplit;
  const RowTile rt = row_tile(blockIdx.x, a.B, (a.D / 64) * nsp);
  if (!rt.valid) return;
  const int dt = rt.tile % (a.D / 64), split = rt.tile / (a.D / 64), b = rt.b, d0 = dt * 64;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const __attribute__((address_space(4))) float* cf =
      (const __attribute__((address_space(4))) float*)(uintptr_t)(a.coef + (int64_t)b * kCoefStride);
  const bool main_split = split < a.nsplit;
  const float ca = cf[0], cb = cf[1];
  const bool with_s = cb != 0.f;
  // main split: F steps [s0, s1); correction split: layers [s0, s1)
  int s0, s1;
  if (main_split) {
    const int nF = a.F / 64;
    s0 = nF * split / a.nsplit;
    s1 = nF * (split + 1) / a.nsplit;
  } else {
    s0 = (split - a.nsplit) * kCorrPerSplit;
    s1 = min(a.l, s0 + kCorrPerSplit);
  }
  const int nst = s1 - s0;
  const bf16* h = static_cast<const bf16*>(a.h_all) + ((int64_t)a.l * a.B + b) * 64 * a.F;
  const int64_t mat = (int64_t)a.F * a.D;
  const bf16* wd = static_cast<const bf16*>(a.wd) + b * mat + d0;
  const bf16* sd = static_cast<const bf16*>(a.sd) + b * mat + d0;
  const bf16* dsrc = static_cast<const bf16*>(a.dz_all) + (int64_t)b * 64 * a.D + d0;
  const int64_t lstride = (int64_t)a.B * 64 * a.D;
  const bf16* hhb = a.hhb + (int64_t)b * 64 * a.LL;  // layer j's block at + 64 j
  int voff[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + 4 * i;  // main: 0..7 H rows, 8..15 W_d rows, 16..23 S_d rows (8 rows each);
                              // correction: 0..7 Gram rows, 8..15 nothing (no range: they keep
                              // the per-step count), 16..23 dZ rows
    voff[i] = main_split ? (g < 8 ? row_src_off(g & 7, lane, a.F) : slab_src_off(g & 7, lane, a.D))
                         : (g < 8 ? row_src_off(g, lane, a.LL) : (g < 16 ? 0 : slab_src_off(g & 7, lane, a.D)));
  }
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int t) {
    const uint32_t slot = ring0 + (uint32_t)((t % kDownSlots) * kSlot);
    if (main_split) {
      const int f0 = (s0 + t) * 64;
      const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(h + f0, (uint32_t)(64 * a.F * 2));
      const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wd + (int64_t)f0 * a.D, (uint32_t)(64 * a.D * 2));
      // without S the S loads have no range: they move no data and keep the per-step count
      const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sd + (int64_t)f0 * a.D, with_s ? (uint32_t)(64 * a.D * 2) : 0u);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int g = w + 4 * i;
        buffer_load_lds_raw(g < 8 ? rh : (g < 16 ? rw : rs), lds_ptr(slot + (uint32_t)(g * 1024)), 16, voff[i], 0,
                            0, 0);
      }
    } else {
      const int j = s0 + t;
      const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(hhb + 64 * j, (uint32_t)(64 * a.LL * 2));
      const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(dsrc + j * lstride, (uint32_t)(64 * a.D * 2));
      const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(hhb, 0u);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int g = w + 4 * i;
        buffer_load_lds_raw(g < 8 ? rg : (g < 16 ? rn : rz), lds_ptr(slot + (uint32_t)(g * 1024)), 16, voff[i], 0, 0,
                            0);
      }
    }
  };
  for (int t = 0; t < min(nst, kDownSlots - 1); ++t) issue(t);
  uint32_t th[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) th[k] = row_frag_addr(ring0, wr, lane, k);  // H rows, or the Gram rows
  const uint32_t tw = slab_tr_addr(ring0 + 8192u, wc, lane), ts = slab_tr_addr(ring0 + 16384u, wc, lane);
  const uint32_t tz = slab_tr_addr(ring0 + 16384u, wc, lane);
  f32x16 accw, accs;
  zero(accw);
  zero(accs);
  for (int t = 0; t < nst; ++t) {
    wait_steps<PER, kDownSlots - 2>(min(nst - 1, t + kDownSlots - 2) - t);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the last step's slot is free
    if (t + kDownSlots - 1 < nst) issue(t + kDownSlots - 1);
    const uint32_t so = (uint32_t)((t % kDownSlots) * kSlot);
    if (main_split) {
      bf16x8 fh[4], fw[4], fs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) fh[k] = lds_read_bf16x8<0>(th[k] + so);
      slab_frags(tw + so, fw);
      slab_frags(ts + so, fs);
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(fh[0]), "+v"(fh[1]), "+v"(fh[2]), "+v"(fh[3]), "+v"(fw[0]), "+v"(fw[1]), "+v"(fw[2]),
                     "+v"(fw[3]), "+v"(fs[0]), "+v"(fs[1]), "+v"(fs[2]), "+v"(fs[3]));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        accw = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[k], fw[k], accw, 0, 0, 0);
        if (with_s) accs = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[k], fs[k], accs, 0, 0, 0);
      }
    } else {
      bf16x8 fz[4], fa[4];
      slab_frags(tz + so, fz);
#pragma unroll
      for (int k = 0; k < 4; ++k) fa[k] = lds_read_bf16x8<0>(th[k] + so);
      lds_wait_frags(fa, fz);
#pragma unroll
      for (int k = 0; k < 4; ++k) accw = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fz[k], accw, 0, 0, 0);
    }
  }
  float* zp = a.zp + (((int64_t)split * a.B + b) * 64) * a.D + d0;
  const int col = wc + acc_col();
  const float wa = main_split ? ca : 1.f, sb = main_split ? cb : 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) zp[(int64_t)(wr + acc_row(i)) * a.D + col] = wa * accw[i] + sb * accs[i];
}
// ---------------------------------------------------------------------------
// 5. dH = dZ_l (a W_down,s + b S_down,s)^T + sum_j gam_j (dZ_l dZ_j^T) H_j per F tile;
//    dU, dG; this tile's share of <K K^T, dU dU^T + dG dG^T>.
// ---------------------------------------------------------------------------
struct BackArgs {
  int B, L, C, D, F, LL, l;
  const float* coef;
  const void* dz_all;
  const void* wd;
  const void* sd;   // fp32 state or its bf16 copies
  const float* zz;  // (B, 64, LL): dZ_l dZ_j^T
  const bf16* zzb;  // (B, 64, LL): bf16(gamma_j dZ_l dZ_j^T), the bf16 pass's correction operand
  const void* h_all;
  const float* u_cur;
  const float* g_cur;
  const float* kk;
  void* du_all;
  void* dg_all;
  float* npart;  // (B, F / 64)
};

// Stages of the dH loop loaded per global round trip (the kernel runs about one workgroup per
// CU, so registers are spent on loads in flight rather than on occupancy).
template <typename T> constexpr int back_group() { return sizeof(T) == 2 ? 4 : 2; }

template <typename T, typename WT>
__global__ void __launch_bounds__(kThreads) k_chain_back(const BackArgs a) {
  constexpr int LD = lds_ld<T>();
  constexpr int NS = back_group<T>();
  __shared__ __align__(16) T zs[NS * 64 * LD];  // dZ rows, then correction A tiles
  __shared__ __align__(16) T ws[NS * 64 * LD];  // (a W_d + b S_d) rows, then H_j^T tiles
  __shared__ __align__(16) T dus[64 * LD];  // [t][f]
  __shared__ __align__(16) T dgs[64 * LD];
  __shared__ float red[4];
  const RowTile rt = row_tile(blockIdx.x, a.B, a.F / 64);
  if (!rt.valid) return;
  const int ft = rt.tile, b = rt.b, f0 = ft * 64;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const float* cf = a.coef + (int64_t)b * kCoefStride;
  const float ca = cf[0], cb = cf[1];
  const bool with_s = cb != 0.f;
  const T* dz = static_cast<const T*>(a.dz_all) + ((int64_t)a.l * a.B + b) * 64 * a.D;
  const int64_t mat = (int64_t)a.F * a.D;
  const WT* wd = static_cast<const WT*>(a.wd) + b * mat + (int64_t)f0 * a.D;
  const WT* sd = static_cast<const WT*>(a.sd) + b * mat + (int64_t)f0 * a.D;
  f32x16 acc;
  zero(acc);
  {
    RowStage<T, KT> zst[NS];
    CombRowStage<WT> wst[NS];
    auto load_group = [&](int d0) {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        if (d0 + q * KT < a.D) {
          zst[q].load(dz + d0 + q * KT, a.D, 64);
          wst[q].load(wd + d0 + q * KT, sd + d0 + q * KT, a.D, with_s);
        }
      }
    };
    load_group(0);
    for (int d0 = 0; d0 < a.D; d0 += NS * KT) {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        if (d0 + q * KT < a.D) {
          zst[q].template store<T>(zs + q * 64 * LD, LD);
          wst[q].template store<T>(ws + q * 64 * LD, LD, ca, cb);
        }
      }
      __syncthreads();
      if (d0 + NS * KT < a.D) load_group(d0 + NS * KT);
#pragma unroll
      for (int q = 0; q < NS; ++q)
        if (d0 + q * KT < a.D) wave_mma<T, KT>(acc, zs + q * 64 * LD + wr * LD, LD, ws + q * 64 * LD + wc * LD, LD);
      __syncthreads();
    }
  }
  if (a.l > 0) {  // sum_j gam_j (dZ_l dZ_j^T) H_j, two layers per round trip
    constexpr int NJ = 2;
    const T* hsrc = static_cast<const T*>(a.h_all) + (int64_t)b * 64 * a.F + f0;
    const int64_t lstride = (int64_t)a.B * 64 * a.F;
    const float* zz = a.zz + (int64_t)b * 64 * a.LL;
    RowStage<float, 64> zst[NJ];
    ColStage<T, 64> st[NJ];
    auto load_pair = [&](int j0) {
#pragma unroll
      for (int q = 0; q < NJ; ++q) {
        if (j0 + q < a.l) {
          zst[q].load(zz + (j0 + q) * 64, a.LL, 64);
          st[q].load(hsrc + (j0 + q) * lstride, a.F, 64, threadIdx.x);
        }
      }
    };
    load_pair(0);
    for (int j0 = 0; j0 < a.l; j0 += NJ) {
#pragma unroll
      for (int q = 0; q < NJ; ++q) {
        if (j0 + q < a.l) {
          store_scaled<T>(zst[q], zs + q * 64 * LD, LD, cf[kGam + j0 + q]);
          st[q].template store<T>(ws + q * 64 * LD, LD);
        }
      }
      __syncthreads();
      if (j0 + NJ < a.l) load_pair(j0 + NJ);
#pragma unroll
      for (int q = 0; q < NJ; ++q)
        if (j0 + q < a.l) wave_mma<T, 64>(acc, zs + q * 64 * LD + wr * LD, LD, ws + q * 64 * LD + wc * LD, LD);
      __syncthreads();
    }
  }
  const int64_t base = (int64_t)b * 64 * a.F + f0;
  const int64_t lbase = ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
  const int f = wc + acc_col();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = wr + acc_row(i);
    const int64_t off = (int64_t)t * a.F + f;
    const float u = a.u_cur[base + off], g = a.g_cur[base + off];
    const float sg = sigmoidf_acc(g);
    const T du = from_f32<T>(acc[i] * (g * sg));
    const T dg = from_f32<T>(acc[i] * u * (sg * (1.0f + g * (1.0f - sg))));
    static_cast<T*>(a.du_all)[lbase + off] = du;
    static_cast<T*>(a.dg_all)[lbase + off] = dg;
    dus[t * LD + f] = du;
    dgs[t * LD + f] = dg;
  }
  __syncthreads();
  f32x16 gu, gg;
  zero(gu);
  zero(gg);
  wave_mma<T, 64>(gu, dus + wr * LD, LD, dus + wc * LD, LD);
  wave_mma<T, 64>(gg, dgs + wr * LD, LD, dgs + wc * LD, LD);
  const float* kk = a.kk + ((int64_t)b * a.LL + a.l * 64) * a.LL + a.l * 64;
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) part += (gu[i] + gg[i]) * kk[(int64_t)(wr + acc_row(i)) * a.LL + wc + acc_col()];
  const float total = block_sum(part, red);
  if (threadIdx.x == 0) a.npart[(int64_t)b * (a.F / 64) + ft] = total;
}

// bf16 activations and copies: both loops' operands go straight into LDS through one ring of
// kBackSlots steps -- D/64 steps of dZ_l rows with the W_down and S_down rows of this F tile
// (k = d along every row), then l steps of the dZ Gram block gamma_j dZ_l dZ_j^T (bf16, scaled
// and rounded by the Gram launch: a row tile read as is) with the H_j slab (transposing reads).  dZ (a W_d + b S_d)^T is formed as a dZ W_d^T + b dZ S_d^T
// with two accumulators, the combined weights never rounded to bf16.  The cursor values are loaded
// after the loops and the epilogue's dU / dG tiles reuse the ring, so registers (184) and LDS (72 KB)
// leave room for two workgroups per CU: one computes while the other's loads are in flight
// (measured at the config-3 shape: 49 us against 67 us with a four-step ring at one per CU).
constexpr int kBackSlots = 3;

__global__ void __launch_bounds__(kThreads, 2) k_chain_back_lds(const BackArgs a) {
  constexpr int kSlot = 24576;  // dZ, W_d, S_d tiles; or the Gram block (16 KB) and the H slab
  constexpr int PER = 6;        // 24 row groups per step over 4 waves
  constexpr int LD = lds_ld<bf16>();
  static_assert(2 * 64 * LD * 2 <= kBackSlots * kSlot, "the epilogue tiles fit in the ring");
  __shared__ __align__(1024) char ring[kBackSlots * kSlot];
  __shared__ float red[4];
  const int nF = a.F / 64;
  const RowTile rt = row_tile(blockIdx.x, a.B, nF);
  if (!rt.valid) return;
  const int ft = rt.tile, b = rt.b, f0 = ft * 64;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  // the coefficients are read-only here: constant-address-space reads become scalar loads
  const __attribute__((address_space(4))) float* cf =
      (const __attribute__((address_space(4))) float*)(uintptr_t)(a.coef + (int64_t)b * kCoefStride);
  const float ca = cf[0], cb = cf[1];
  const bool with_s = cb != 0.f;
  const int f = wc + acc_col();
  const bf16* dz = static_cast<const bf16*>(a.dz_all) + ((int64_t)a.l * a.B + b) * 64 * a.D;
  const int64_t mat = (int64_t)a.F * a.D;
  const bf16* wd = static_cast<const bf16*>(a.wd) + b * mat + (int64_t)f0 * a.D;
  const bf16* sd = static_cast<const bf16*>(a.sd) + b * mat + (int64_t)f0 * a.D;
  const bf16* zzb = a.zzb + (int64_t)b * 64 * a.LL;  // layer j's block at + 64 j
  const bf16* hsrc = static_cast<const bf16*>(a.h_all) + (int64_t)b * 64 * a.F + f0;
  const int64_t lstride = (int64_t)a.B * 64 * a.F;
  const int n1 = a.D / 64, ns = n1 + a.l;
  // row group g of a step (8 rows each): phase 1: 0..7 dZ rows, 8..15 W_d rows, 16..23 S_d rows;
  // phase 2: 0..7 Gram rows, 8..15 nothing (no range: they keep the per-step count), 16..23 H
  // rows; wave w takes groups w, w + 4, ...
  int v1[PER], v2[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + 4 * i;
    v1[i] = row_src_off(g & 7, lane, a.D);
    v2[i] = g < 8 ? row_src_off(g, lane, a.LL) : (g < 16 ? 0 : slab_src_off(g & 7, lane, a.F));
  }
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int step) {
    const int t = step;
    const uint32_t slot = ring0 + (uint32_t)((t % kBackSlots) * kSlot);
    if (step < n1) {
      const int d0 = step * 64;
      const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(dz + d0, (uint32_t)(64 * a.D * 2));
      const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wd + d0, (uint32_t)(64 * a.D * 2));
      // without S the S loads have no range: they move no data and keep the per-step count
      const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(sd + d0, with_s ? (uint32_t)(64 * a.D * 2) : 0u);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int g = w + 4 * i;
        buffer_load_lds_raw(g < 8 ? rz : (g < 16 ? rw : rs), lds_ptr(slot + (uint32_t)(g * 1024)), 16, v1[i], 0,
                            0, 0);
      }
    } else {
      const int j = step - n1;
      const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(zzb + 64 * j, (uint32_t)(64 * a.LL * 2));
      const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(hsrc + j * lstride, (uint32_t)(64 * a.F * 2));
      const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(zzb, 0u);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int g = w + 4 * i;
        buffer_load_lds_raw(g < 8 ? rg : (g < 16 ? rn : rh), lds_ptr(slot + (uint32_t)(g * 1024)), 16, v2[i], 0, 0,
                            0);
      }
    }
  };
  for (int t = 0; t < min(ns, kBackSlots - 1); ++t) issue(t);
  uint32_t tz[4], tw[4], ts[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    tz[k] = row_frag_addr(ring0, wr, lane, k);  // dZ rows in phase 1, Gram rows in phase 2
    tw[k] = row_frag_addr(ring0 + 8192u, wc, lane, k);
    ts[k] = row_frag_addr(ring0 + 16384u, wc, lane, k);
  }
  const uint32_t th = slab_tr_addr(ring0 + 16384u, wc, lane);
  f32x16 accw, accs, accg;
  zero(accw);
  zero(accs);
  zero(accg);
  for (int t = 0; t < ns; ++t) {
    wait_steps<PER, kBackSlots - 2>(min(ns - 1, t + kBackSlots - 2) - t);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the last step's slot is free
    if (t + kBackSlots - 1 < ns) issue(t + kBackSlots - 1);
    const uint32_t so = (uint32_t)((t % kBackSlots) * kSlot);
    const int step = t;
    if (step < n1) {
      bf16x8 fz[4], fw[4], fs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        fz[k] = lds_read_bf16x8<0>(tz[k] + so);
        fw[k] = lds_read_bf16x8<0>(tw[k] + so);
        fs[k] = lds_read_bf16x8<0>(ts[k] + so);
      }
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(fz[0]), "+v"(fz[1]), "+v"(fz[2]), "+v"(fz[3]), "+v"(fw[0]), "+v"(fw[1]), "+v"(fw[2]),
                     "+v"(fw[3]), "+v"(fs[0]), "+v"(fs[1]), "+v"(fs[2]), "+v"(fs[3]));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        accw = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fz[k], fw[k], accw, 0, 0, 0);
        if (with_s) accs = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fz[k], fs[k], accs, 0, 0, 0);
      }
    } else {
      bf16x8 fh[4], fa[4];
      slab_frags(th + so, fh);
#pragma unroll
      for (int k = 0; k < 4; ++k) fa[k] = lds_read_bf16x8<0>(tz[k] + so);
      lds_wait_frags(fa, fh);
#pragma unroll
      for (int k = 0; k < 4; ++k) accg = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fh[k], accg, 0, 0, 0);
    }
  }
  float dh[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) dh[i] = (ca * accw[i] + cb * accs[i]) + accg[i];
  // epilogue: dU, dG of this tile, and its share of |g_l|^2; dU / dG tiles in the ring's LDS
  __builtin_amdgcn_s_barrier();  // every wave is past its last read of the ring
  bf16* dus = reinterpret_cast<bf16*>(ring);  // [t][f]
  bf16* dgs = dus + 64 * LD;
  const int64_t base = (int64_t)b * 64 * a.F + f0;
  const int64_t lbase = ((int64_t)a.l * a.B + b) * 64 * a.F + f0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = wr + acc_row(i);
    const int64_t off = (int64_t)t * a.F + f;
    const float u = a.u_cur[base + off], g = a.g_cur[base + off];
    const float sg = sigmoidf_acc(g);
    const bf16 du = from_f32<bf16>(dh[i] * (g * sg));
    const bf16 dg = from_f32<bf16>(dh[i] * u * (sg * (1.0f + g * (1.0f - sg))));
    static_cast<bf16*>(a.du_all)[lbase + off] = du;
    static_cast<bf16*>(a.dg_all)[lbase + off] = dg;
    dus[t * LD + f] = du;
    dgs[t * LD + f] = dg;
  }
  __syncthreads();
  f32x16 gu, gg;
  zero(gu);
  zero(gg);
  wave_mma<bf16, 64>(gu, dus + wr * LD, LD, dus + wc * LD, LD);
  wave_mma<bf16, 64>(gg, dgs + wr * LD, LD, dgs + wc * LD, LD);
  const float* kk = a.kk + ((int64_t)b * a.LL + a.l * 64) * a.LL + a.l * 64;
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) part += (gu[i] + gg[i]) * kk[(int64_t)(wr + acc_row(i)) * a.LL + wc + acc_col()];
  const float total = block_sum(part, red);
  if (threadIdx.x == 0) a.npart[(int64_t)b * nF + ft] = total;
}

// ---------------------------------------------------------------------------
// 7. Final state: W' = a W_s + b S_s + sum_j gam_j g_j, S' = e S_s + sum_j sig_j g_j per
//    64 x 64 tile, with g_j tiles rebuilt from the small activations (K = 64 per layer).
// ---------------------------------------------------------------------------
struct ApplyChainArgs {
  int B, L, C, D, F;
  const float* coef;
  Acts acts;
  const void* h_all;
  const void* du_all;
  const void* dg_all;
  const void* dz_all;
  float* w[3];
  float* s[3];
  bf16* wc[3];  // optional bf16 copies of W' and S'
  bf16* sc[3];
};

// 64 x 64 output tiles, one layer's token slabs per stage: double-buffered in LDS and loaded
// two layers ahead into registers (bf16 slabs are staged by all 256 threads; fp32 slabs one
// layer ahead), so the slab round trips overlap MFMA work.  The W and S tile loads are issued
// after the last slab loads (memory counters retire in order) and overlap the last layers.

template <typename T> struct ApplyStage { using type = ColStage<T, 64>; };
template <> struct ApplyStage<bf16> { using type = ColStage4<64>; };
constexpr int kApplyWaves = 4;  // waves per SIMD: the latency hiding comes from resident tiles

template <typename T>
__global__ void __launch_bounds__(kThreads, kApplyWaves) k_chain_apply(const ApplyChainArgs a) {
  constexpr int LD = lds_ld<T>();
  using Stage = typename ApplyStage<T>::type;
  constexpr int kUnits = Stage::kUnits;
  static_assert(2 * kUnits == kThreads, "the two slabs of a stage take one thread each");
  __shared__ __align__(16) T as[2][64 * LD];
  __shared__ __align__(16) T bs[2][64 * LD];
  const int nD = a.D / 64, nF = a.F / 64;
  const int per = nD * nF;
  const RowTile rt = row_tile(blockIdx.x, a.B, 3 * per);
  if (!rt.valid) return;
  const int m = rt.tile / per, jt = rt.tile - m * per, b = rt.b;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const float* cf = a.coef + (int64_t)b * kCoefStride;
  if (cf[3] == 0.f) return;  // no layer updated this row: W and S stay as they are
  // tiles sharing a small token slab run together: for every matrix the F tile is the outer
  // index and the D tile the inner one, so the resident workgroups of a row need the slabs
  // of a few F tiles plus the (small) D-wide slabs
  int r0, c0, ld_out;
  const int ft = jt / nD, dt = jt - ft * nD;
  if (m < 2) {
    r0 = dt * 64;
    c0 = ft * 64;
    ld_out = a.F;
  } else {
    r0 = ft * 64;
    c0 = dt * 64;
    ld_out = a.D;
  }
  const int64_t mat = (int64_t)a.D * a.F;
  // operand sources of layer j: A^T rows are tokens (k), columns this tile's rows
  const bool a_part = threadIdx.x < kUnits;
  const int unit = a_part ? (int)threadIdx.x : (int)threadIdx.x - kUnits;
  const T* src;
  int64_t src_ld, src_lstride;
  int k_valid;
  if (m < 2) {
    if (a_part) {
      src = layer_row<T>(a.acts.k, 0, b, a.acts.kv_rs) + r0;
      src_ld = a.acts.kv_ts;
      src_lstride = 0;  // per-layer pointers
      k_valid = a.C;
    } else {
      src = static_cast<const T*>(m == 0 ? a.du_all : a.dg_all) + (int64_t)b * 64 * a.F + c0;
      src_ld = a.F;
      src_lstride = (int64_t)a.B * 64 * a.F;
      k_valid = 64;
    }
  } else {
    src = a_part ? static_cast<const T*>(a.h_all) + (int64_t)b * 64 * a.F + r0
                 : static_cast<const T*>(a.dz_all) + (int64_t)b * 64 * a.D + c0;
    src_ld = a_part ? a.F : a.D;
    src_lstride = a_part ? (int64_t)a.B * 64 * a.F : (int64_t)a.B * 64 * a.D;
    k_valid = 64;
  }
  const bool per_layer_ptr = m < 2 && a_part;
  auto layer_src = [&](int j) -> const T* {
    return per_layer_ptr ? layer_row<T>(a.acts.k, j, b, a.acts.kv_rs) + r0 : src + j * src_lstride;
  };
  // element i of this lane's accumulator tile sits at the tile base + lane offset + the
  // wave-uniform (8 (i / 4) + i % 4) rows: buffer accesses with one VGPR offset per lane and
  // the row offsets in SGPRs
  const uint32_t mat_bytes = (uint32_t)(mat * 4);
  const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(a.w[m] + b * mat, mat_bytes);
  const __amdgpu_buffer_rsrc_t sres = buffer_rsrc(a.s[m] + b * mat, mat_bytes);
  const int64_t tile0 = (int64_t)(r0 + wr) * ld_out + c0 + wc;
  const int lane_el = (int)tile0 + 4 * ((int)(threadIdx.x & 63) >> 5) * ld_out + acc_col();
  auto row_el = [&](int i) { return (8 * (i >> 2) + (i & 3)) * ld_out; };
  float wv[16], sv[16];
  // the state streams through once: non-temporal accesses keep it from evicting the token
  // slabs that the other workgroups of the row still read from L2
  auto load_state = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      wv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wres, lane_el * 4, row_el(i) * 4,
                                                                             kNonTemporal));
      sv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sres, lane_el * 4, row_el(i) * 4,
                                                                             kNonTemporal));
    }
  };
  f32x16 accw, accs;
  zero(accw);
  zero(accs);
  auto step = [&](Stage& st, int j, bool refill) {
    const int buf = j & 1;
    st.store(a_part ? as[buf] : bs[buf], LD);
    __syncthreads();
    if (refill) st.load(layer_src(j + 2), src_ld, k_valid, unit);
    f32x16 t;
    zero(t);
    wave_mma<T, 64>(t, as[buf] + wr * LD, LD, bs[buf] + wc * LD, LD);
    const float gj = cf[kGam + j], sj = cf[kSig + j];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      accw[i] += gj * t[i];
      accs[i] += sj * t[i];
    }
  };
  if constexpr (sizeof(T) == 2) {
    // layer j sits in register stage j & 1
    Stage st0, st1;
    st0.load(layer_src(0), src_ld, k_valid, unit);
    if (a.L > 1) st1.load(layer_src(1), src_ld, k_valid, unit);
    int j = 0;
    for (; j + 3 < a.L; j += 2) {  // both steps load the layer two ahead
      step(st0, j, true);
      step(st1, j + 1, true);
    }
    if (j + 2 < a.L) step(st0, j++, true);
    load_state();  // after the last slab loads
    for (; j < a.L; ++j) {
      if (j & 1)
        step(st1, j, false);
      else
        step(st0, j, false);
    }
  } else {
    // fp32 slabs take twice the registers: one layer ahead
    Stage st;
    st.load(layer_src(0), src_ld, k_valid, unit);
    for (int j = 0; j < a.L; ++j) {
      const int buf = j & 1;
      st.store(a_part ? as[buf] : bs[buf], LD);
      __syncthreads();
      if (j + 1 < a.L) st.load(layer_src(j + 1), src_ld, k_valid, unit);
      if (j + 1 == a.L) load_state();
      f32x16 t;
      zero(t);
      wave_mma<T, 64>(t, as[buf] + wr * LD, LD, bs[buf] + wc * LD, LD);
      const float gj = cf[kGam + j], sj = cf[kSig + j];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        accw[i] += gj * t[i];
        accs[i] += sj * t[i];
      }
    }
  }
  const float ca = cf[0], cb = cf[1], ce = cf[2];
  const bool copies = a.wc[m] != nullptr;  // W and S copies are given together or not at all
  const __amdgpu_buffer_rsrc_t wcres = buffer_rsrc(copies ? a.wc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
  const __amdgpu_buffer_rsrc_t scres = buffer_rsrc(copies ? a.sc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float w_new = ca * wv[i] + cb * sv[i] + accw[i];
    const float s_new = ce * sv[i] + accs[i];
    // the b32 / b16 buffer builtins move raw bits
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, w_new), wres, lane_el * 4, row_el(i) * 4,
                                          kNonTemporal);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s_new), sres, lane_el * 4, row_el(i) * 4,
                                          kNonTemporal);
    if (copies) {
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<bf16>(w_new)), wcres,
                                            lane_el * 2, row_el(i) * 2, kNonTemporal);
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<bf16>(s_new)), scres,
                                            lane_el * 2, row_el(i) * 2, kNonTemporal);
    }
  }
}

// bf16 activations: the token slabs go straight from global memory into LDS (buffer loads with
// the lds bit, no registers, no staging instructions) through a ring of kApplySlots layer slots,
// and reach the MFMA through transposing LDS reads.  Waits are explicit: each wave issues 4 slab
// loads per layer, and the count of loads still allowed in flight is known at every step.  The
// W and S tile loads follow the loop: the layer loop holds no state registers (81 VGPRs), and
// four workgroups per CU overlap one workgroup's state traffic with the others' layer loops
// (measured: faster than deeper slab prefetch at fewer workgroups, or state loads ahead of the
// loop).
//
constexpr int kApplySlots = 2;
constexpr int kApplyLdsWaves = 4;  // 32 KB of LDS per workgroup: four workgroups per CU

__global__ void __launch_bounds__(kThreads, kApplyLdsWaves) k_chain_apply_lds(const ApplyChainArgs a) {
  __shared__ __align__(1024) bf16 slab[kApplySlots][2][64 * 64];
  const int nD = a.D / 64, nF = a.F / 64;
  const int per = nD * nF;
  const RowTile rt = row_tile(blockIdx.x, a.B, 3 * per);
  if (!rt.valid) return;
  const int m = rt.tile / per, jt = rt.tile - m * per, b = rt.b;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  // the coefficients are read-only here: constant-address-space reads become scalar loads
  const __attribute__((address_space(4))) float* cf =
      (const __attribute__((address_space(4))) float*)(uintptr_t)(a.coef + (int64_t)b * kCoefStride);
  if (cf[3] == 0.f) return;  // no layer updated this row: W and S stay as they are
  int r0, c0, ld_out;
  const int ft = jt / nD, dt = jt - ft * nD;
  if (m < 2) {
    r0 = dt * 64;
    c0 = ft * 64;
    ld_out = a.F;
  } else {
    r0 = ft * 64;
    c0 = dt * 64;
    ld_out = a.D;
  }
  const int64_t mat = (int64_t)a.D * a.F;
  // slab sources of layer j (wave-uniform): A = tokens x this tile's rows, B = tokens x its columns
  const bf16* a_src;
  const bf16* b_src;
  int64_t a_lstride, b_lstride;
  int a_ld, b_ld, a_rows;
  if (m < 2) {
    a_src = nullptr;  // per-layer key pointers
    a_lstride = 0;
    a_ld = (int)a.acts.kv_ts;
    a_rows = a.C;
    b_src = static_cast<const bf16*>(m == 0 ? a.du_all : a.dg_all) + (int64_t)b * 64 * a.F + c0;
    b_ld = a.F;
    b_lstride = (int64_t)a.B * 64 * a.F;
  } else {
    a_src = static_cast<const bf16*>(a.h_all) + (int64_t)b * 64 * a.F + r0;
    a_ld = a.F;
    a_lstride = (int64_t)a.B * 64 * a.F;
    a_rows = 64;
    b_src = static_cast<const bf16*>(a.dz_all) + (int64_t)b * 64 * a.D + c0;
    b_ld = a.D;
    b_lstride = (int64_t)a.B * 64 * a.D;
  }
  auto a_layer = [&](int j) -> const bf16* {
    return m < 2 ? layer_row<bf16>(a.acts.k, j, b, a.acts.kv_rs) + r0 : a_src + j * a_lstride;
  };
  // this wave's slab loads: row groups w and w + 4 (8 token rows each) of both slabs
  int a_off[2], b_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    a_off[i] = slab_src_off(w + 4 * i, lane, a_ld);  // rows past a_rows are out of the buffer range: zeros
    b_off[i] = slab_src_off(w + 4 * i, lane, b_ld);
  }
  const uint32_t slab0 = lds_addr(&slab[0][0][0]);
  // layer j's slabs into slot j % kApplySlots; past the last layer the buffers have no range,
  // so those loads touch no memory and only write zeros (the prologue stays branch-free)
  auto issue = [&](int j) {
    const bool live = j < a.L;
    const int jj = live ? j : a.L - 1;
    const uint32_t base = slab0 + (uint32_t)((j % kApplySlots) * 2 * 64 * 64 * 2);
    const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(a_layer(jj), live ? (uint32_t)(a_rows * a_ld * 2) : 0u);
    const __amdgpu_buffer_rsrc_t br = buffer_rsrc(b_src + jj * b_lstride, live ? (uint32_t)(64 * b_ld * 2) : 0u);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      buffer_load_lds_raw(ar, lds_ptr(base + (uint32_t)((w + 4 * i) * 1024)), 16, a_off[i], 0, 0, 0);
      buffer_load_lds_raw(br, lds_ptr(base + 8192u + (uint32_t)((w + 4 * i) * 1024)), 16, b_off[i], 0, 0, 0);
    }
  };
#pragma unroll
  for (int j = 0; j < kApplySlots - 1; ++j) issue(j);
  const uint32_t ta = slab_tr_addr(slab0, wr, lane), tb = slab_tr_addr(slab0 + 8192u, wc, lane);
  f32x16 accw, accs;
  zero(accw);
  zero(accs);
  for (int j = 0; j < a.L; ++j) {
    // this wave's slab loads of layer j are done once those of the later issued layers remain
    wait_steps<4, kApplySlots - 2>(min(a.L - 1, j + kApplySlots - 2) - j);
    __builtin_amdgcn_s_barrier();  // every wave's loads of layer j landed; layer j - 1's slot is free
    if (j + kApplySlots - 1 < a.L) issue(j + kApplySlots - 1);
    const uint32_t so = (uint32_t)((j % kApplySlots) * 2 * 64 * 64 * 2);
    bf16x8 fa[4], fb[4];
    slab_frags(ta + so, fa);
    slab_frags(tb + so, fb);
    lds_wait_frags(fa, fb);
    f32x16 t;
    zero(t);
#pragma unroll
    for (int s = 0; s < 4; ++s) t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s], fb[s], t, 0, 0, 0);
    const float gj = cf[kGam + j], sj = cf[kSig + j];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      accw[i] += gj * t[i];
      accs[i] += sj * t[i];
    }
  }
  const uint32_t mat_bytes = (uint32_t)(mat * 4);
  const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(a.w[m] + b * mat, mat_bytes);
  const __amdgpu_buffer_rsrc_t sres = buffer_rsrc(a.s[m] + b * mat, mat_bytes);
  const int64_t tile0 = (int64_t)(r0 + wr) * ld_out + c0 + wc;
  const int lane_el = (int)tile0 + 4 * (lane >> 5) * ld_out + acc_col();
  auto row_el = [&](int i) { return (8 * (i >> 2) + (i & 3)) * ld_out; };
  float wv[16], sv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    wv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wres, lane_el * 4, row_el(i) * 4,
                                                                           kNonTemporal));
    sv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sres, lane_el * 4, row_el(i) * 4,
                                                                           kNonTemporal));
  }
  const float ca = cf[0], cb = cf[1], ce = cf[2];
  const bool copies = a.wc[m] != nullptr;
  const __amdgpu_buffer_rsrc_t wcres = buffer_rsrc(copies ? a.wc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
  const __amdgpu_buffer_rsrc_t scres = buffer_rsrc(copies ? a.sc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float w_new = ca * wv[i] + cb * sv[i] + accw[i];
    const float s_new = ce * sv[i] + accs[i];
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, w_new), wres, lane_el * 4, row_el(i) * 4,
                                          kNonTemporal);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s_new), sres, lane_el * 4, row_el(i) * 4,
                                          kNonTemporal);
    // the bf16 copies are what the next chunk reads first: default cache policy
    if (copies) {
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<bf16>(w_new)), wcres,
                                            lane_el * 2, row_el(i) * 2, 0);
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<bf16>(s_new)), scres,
                                            lane_el * 2, row_el(i) * 2, 0);
    }
  }
}

// The same state write with wider output tiles: NA x 64 rows by NB x 64 columns (D and F
// multiples of 64 NA and 64 NB as the matrix needs).  Per layer the workgroup loads 64 token rows
// of NA + NB 64-column slabs, so each output costs (NA + NB) / (2 NA NB) of the slab bytes of a
// 64 x 64 tile, and each layer step carries NA NB times the MFMA work between barriers.  Wave
// (qr, qc) owns rows qr NA 32 .. and columns qc NB 32 .. of the tile as NA x NB MFMA tiles of
// 32 x 32; each tile's layer product is folded into its W and S sums right away.
__device__ __forceinline__ void lds_wait_frag_sets(bf16x8 (&a)[4], bf16x8 (&b)[4], bf16x8 (&c)[4],
                                                   bf16x8 (&d)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]),
                 "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]));
}

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x2v __attribute__((ext_vector_type(2)));

// four floats rounded to bf16 (round to nearest even, as static_cast<bf16>) in 8 bytes
__device__ __forceinline__ u32x2v pack_bf16x4(const f32x4& v) {
  u32x2v r;
  r[0] = (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(v[0])) |
         ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(v[1])) << 16);
  r[1] = (uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(v[2])) |
         ((uint32_t)__builtin_bit_cast(unsigned short, static_cast<bf16>(v[3])) << 16);
  return r;
}

template <int NA, int NB, int SLOTS>
constexpr int apply_wide_occupancy() {
  return (160 * 1024) / (SLOTS * (NA + NB) * 8192) < 1 ? 1 : (160 * 1024) / (SLOTS * (NA + NB) * 8192);
}

// Tile order of the wide state write.  Every output tile reads, per layer, the token slabs of its
// row block and of its column block, and the workgroups resident on one XCD (about 64) share one
// L2.  A row's tiles are listed matrix by matrix, in blocks of kApplyBlock x kApplyBlock tiles,
// and placed on the XCDs by row_tile (a row's 8 / B XCDs take neighbouring tiles side by side
// for 1, 2 or 4 rows, contiguous eighths of the list otherwise).  The resident workgroups of an
// XCD then cover about one block, 2 kApplyBlock slabs per layer, where tiles dealt round-robin in
// row-major order spread over ~55 slabs per layer at the config-3 shape and missed L2 on more
// than half of the slab reads (side by side instead of contiguous halves of a row: config 3
// 519.4-520.1 against 520.6-521.3 ms).
constexpr int kApplyBlock = 8;

// tile q of an R x C tile matrix listed in kApplyBlock x kApplyBlock blocks (row-major blocks,
// row-major inside a block, ragged blocks at the right and bottom edges)
__device__ __forceinline__ void blocked_tile(int q, int R, int C, int& r, int& c) {
  const int i = q / (kApplyBlock * C), rem = q - i * kApplyBlock * C;
  const int h = min(kApplyBlock, R - i * kApplyBlock);
  const int j = rem / (h * kApplyBlock), rem2 = rem - j * h * kApplyBlock;
  const int w = min(kApplyBlock, C - j * kApplyBlock);
  r = i * kApplyBlock + rem2 / w;
  c = j * kApplyBlock + rem2 % w;
}

template <int NA, int NB, int SLOTS>
__global__ void __launch_bounds__(kThreads, (apply_wide_occupancy<NA, NB, SLOTS>() > 4 ? 4 : apply_wide_occupancy<NA, NB, SLOTS>()))
k_chain_apply_wide(const ApplyChainArgs a) {
  constexpr int NS = NA + NB;  // 64-column slabs per layer: A halves, then B halves
  __shared__ __align__(1024) bf16 slab[SLOTS][NS][64 * 64];
  const int nD = a.D / 64, nF = a.F / 64;
  // tiles: W_up / W_gate (D x F) take NA 64-row blocks of D by NB of F; W_down (F x D) NA of F by NB of D
  const int per_ug = (nD / NA) * (nF / NB), per_dn = (nF / NA) * (nD / NB);
  const int per_row = 2 * per_ug + per_dn;
  const RowTile pl = row_tile(blockIdx.x, a.B, per_row);  // the grid is row_tile_blocks(B, per_row)
  if (!pl.valid) return;
  const int b = pl.b, tile = pl.tile;
  const int m = tile < 2 * per_ug ? tile / per_ug : 2;
  const int jt = m < 2 ? tile - m * per_ug : tile - 2 * per_ug;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int qr = w >> 1, qc = w & 1;
  const __attribute__((address_space(4))) float* cf =
      (const __attribute__((address_space(4))) float*)(uintptr_t)(a.coef + (int64_t)b * kCoefStride);
  if (cf[3] == 0.f) return;  // no layer updated this row: W and S stay as they are
  int rt, ct;
  if (m < 2)
    blocked_tile(jt, nD / NA, nF / NB, rt, ct);
  else
    blocked_tile(jt, nF / NA, nD / NB, rt, ct);
  const int r0 = rt * 64 * NA, c0 = ct * 64 * NB, ld_out = m < 2 ? a.F : a.D;
  const int64_t mat = (int64_t)a.D * a.F;
  const bf16* a_src;
  const bf16* b_src;
  int64_t a_lstride, b_lstride;
  int a_ld, b_ld, a_rows;
  if (m < 2) {
    a_src = nullptr;  // per-layer key pointers
    a_lstride = 0;
    a_ld = (int)a.acts.kv_ts;
    a_rows = a.C;
    b_src = static_cast<const bf16*>(m == 0 ? a.du_all : a.dg_all) + (int64_t)b * 64 * a.F + c0;
    b_ld = a.F;
    b_lstride = (int64_t)a.B * 64 * a.F;
  } else {
    a_src = static_cast<const bf16*>(a.h_all) + (int64_t)b * 64 * a.F + r0;
    a_ld = a.F;
    a_lstride = (int64_t)a.B * 64 * a.F;
    a_rows = 64;
    b_src = static_cast<const bf16*>(a.dz_all) + (int64_t)b * 64 * a.D + c0;
    b_ld = a.D;
    b_lstride = (int64_t)a.B * 64 * a.D;
  }
  auto a_layer = [&](int j) -> const bf16* {
    return m < 2 ? layer_row<bf16>(a.acts.k, j, b, a.acts.kv_rs) + r0 : a_src + j * a_lstride;
  };
  // this wave's slab loads: row groups w and w + 4 (8 token rows each) of every slab
  int a_off[2], b_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    a_off[i] = slab_src_off(w + 4 * i, lane, a_ld);
    b_off[i] = slab_src_off(w + 4 * i, lane, b_ld);
  }
  const uint32_t slab0 = lds_addr(&slab[0][0][0]);
  // layer j's slabs into slot j % SLOTS.  Slab h of a side starts 64 h columns into the row; its
  // range ends 128 h bytes before the side's, so rows past the valid ones read as zeros (a row
  // stride of at least 64 (h + 1) elements keeps every valid row inside).  Past the last layer
  // the buffers have no range.
  auto issue = [&](int j) {
    const bool live = j < a.L;
    const int jj = live ? j : a.L - 1;
    const uint32_t base = slab0 + (uint32_t)((j % SLOTS) * NS * 8192);
    const bf16* al = a_layer(jj);
    const bf16* bl = b_src + jj * b_lstride;
#pragma unroll
    for (int h = 0; h < NA; ++h) {
      const __amdgpu_buffer_rsrc_t ar =
          buffer_rsrc(al + 64 * h, live ? (uint32_t)(a_rows * a_ld * 2 - 128 * h) : 0u);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        buffer_load_lds_raw(ar, lds_ptr(base + (uint32_t)(h * 8192 + (w + 4 * i) * 1024)), 16, a_off[i], 0, 0, 0);
    }
#pragma unroll
    for (int h = 0; h < NB; ++h) {
      const __amdgpu_buffer_rsrc_t br = buffer_rsrc(bl + 64 * h, live ? (uint32_t)(64 * b_ld * 2 - 128 * h) : 0u);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        buffer_load_lds_raw(br, lds_ptr(base + (uint32_t)((NA + h) * 8192 + (w + 4 * i) * 1024)), 16, b_off[i], 0,
                            0, 0);
    }
  };
#pragma unroll
  for (int j = 0; j < SLOTS - 1; ++j) issue(j);
  // this wave's operand columns: A rows qr NA 32 + 32 ra of the tile, B columns qc NB 32 + 32 cb
  uint32_t ta[NA], tb[NB];
#pragma unroll
  for (int ra = 0; ra < NA; ++ra) {
    const int row = qr * NA * 32 + 32 * ra;
    ta[ra] = slab_tr_addr(slab0 + (uint32_t)((row >> 6) * 8192), row & 63, lane);
  }
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const int col = qc * NB * 32 + 32 * cb;
    tb[cb] = slab_tr_addr(slab0 + (uint32_t)((NA + (col >> 6)) * 8192), col & 63, lane);
  }
  f32x16 accw[NA][NB], accs[NA][NB];
#pragma unroll
  for (int ra = 0; ra < NA; ++ra)
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      zero(accw[ra][cb]);
      zero(accs[ra][cb]);
    }
  bf16x8 fa[2][4], fb[2][4];  // the second set stays unused (zero) with one 32-row or column block
  if constexpr (NA == 1)
    for (int s = 0; s < 4; ++s) fa[1][s] = bf16x8{};
  if constexpr (NB == 1)
    for (int s = 0; s < 4; ++s) fb[1][s] = bf16x8{};
  for (int j = 0; j < a.L; ++j) {
    // this wave's slab loads of layer j are done once those of the later issued layers remain
    wait_steps<2 * NS, SLOTS - 2>(min(a.L - 1, j + SLOTS - 2) - j);
    __builtin_amdgcn_s_barrier();  // every wave's loads of layer j landed; layer j - 1's slot is free
    if (j + SLOTS - 1 < a.L) issue(j + SLOTS - 1);
    const uint32_t so = (uint32_t)((j % SLOTS) * NS * 8192);
#pragma unroll
    for (int ra = 0; ra < NA; ++ra) slab_frags(ta[ra] + so, fa[ra]);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) slab_frags(tb[cb] + so, fb[cb]);
    lds_wait_frag_sets(fa[0], fa[1], fb[0], fb[1]);
    const float gj = cf[kGam + j], sj = cf[kSig + j];
#pragma unroll
    for (int ra = 0; ra < NA; ++ra)
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        f32x16 t;
        zero(t);
#pragma unroll
        for (int s = 0; s < 4; ++s) t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ra][s], fb[cb][s], t, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          accw[ra][cb][i] += gj * t[i];
          accs[ra][cb][i] += sj * t[i];
        }
      }
  }
  const uint32_t mat_bytes = (uint32_t)(mat * 4);
  const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(a.w[m] + b * mat, mat_bytes);
  const __amdgpu_buffer_rsrc_t sres = buffer_rsrc(a.s[m] + b * mat, mat_bytes);
  const float ca = cf[0], cb_ = cf[1], ce = cf[2];
  const bool copies = a.wc[m] != nullptr;
  const __amdgpu_buffer_rsrc_t wcres = buffer_rsrc(copies ? a.wc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
  const __amdgpu_buffer_rsrc_t scres = buffer_rsrc(copies ? a.sc[m] + b * mat : nullptr, copies ? mat_bytes / 2 : 0);
  // The accumulators hold column strips (4 consecutive rows of one column per group of 4).  A
  // transpose through LDS gives each lane 4 consecutive columns of a row instead, so W and S move
  // in 16-byte accesses (8 lanes per 128-byte row segment) and the bf16 copies in 8-byte ones:
  // 24 memory instructions per 32 x 32 tile instead of 96, which also keeps the wave's
  // outstanding memory operations under the 63 the counter tracks.  The W and S loads of tile
  // u + 2 are issued once tile u is stored.
  __syncthreads();  // every wave is done with the slab ring: it becomes the transpose space
  constexpr int XLD = 36;  // padded row of a 32 x 32 transpose tile (rows stay 16-byte aligned)
  float* xt = reinterpret_cast<float*>(&slab[0][0][0]) + w * 32 * XLD;
  const int xr = lane >> 3, xc = 4 * (lane & 7);  // row layout: rows xr + 8 k, columns xc .. xc + 3
  const int acc_r = 4 * (lane >> 5), acc_c = lane & 31;
  constexpr int NT = NA * NB;
  auto tile_el = [&](int u) {
    const int ra = u / NB, cb = u % NB;
    return (r0 + qr * NA * 32 + 32 * ra + xr) * ld_out + c0 + qc * NB * 32 + 32 * cb + xc;
  };
  f32x4 wo[2][4], so[2][4];
  auto load_tile = [&](int u) {
    const int el = tile_el(u);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      wo[u & 1][k] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, el * 4, 8 * k * ld_out * 4, kNonTemporal));
      so[u & 1][k] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(sres, el * 4, 8 * k * ld_out * 4, kNonTemporal));
    }
  };
  auto transpose = [&](const f32x16& acc, f32x4 (&out)[4]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) xt[(8 * (i >> 2) + acc_r + (i & 3)) * XLD + acc_c] = acc[i];
    // the same wave reads back: one wave's LDS operations complete in order
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = *reinterpret_cast<const f32x4*>(xt + (xr + 8 * k) * XLD + xc);
  };
  load_tile(0);
  if constexpr (NT > 1) load_tile(1);
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int ra = u / NB, cb = u % NB, el = tile_el(u);
    f32x4 gw[4], gs[4];
    transpose(accw[ra][cb], gw);
    transpose(accs[ra][cb], gs);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f32x4 wn, sn;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wn[e] = ca * wo[u & 1][k][e] + cb_ * so[u & 1][k][e] + gw[k][e];
        sn[e] = ce * so[u & 1][k][e] + gs[k][e];
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, wn), wres, el * 4, 8 * k * ld_out * 4,
                                             kNonTemporal);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, sn), sres, el * 4, 8 * k * ld_out * 4,
                                             kNonTemporal);
      if (copies) {
        __builtin_amdgcn_raw_buffer_store_b64(pack_bf16x4(wn), wcres, el * 2, 8 * k * ld_out * 2, 0);
        __builtin_amdgcn_raw_buffer_store_b64(pack_bf16x4(sn), scres, el * 2, 8 * k * ld_out * 2, 0);
      }
    }
    if (u + 2 < NT) load_tile(u + 2);
  }
}

// the wide state write's tile shape (rows x columns in 64-blocks) and ring depth
constexpr int kApplyNA = 2, kApplyNB = 2, kApplySlotsWide = 2;

inline bool apply_wide_fits(int64_t D, int64_t F) {
  return D % (64 * kApplyNA) == 0 && D % (64 * kApplyNB) == 0 && F % (64 * kApplyNA) == 0 && F % (64 * kApplyNB) == 0;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
size_t act_size(int32_t dtype) { return dtype == UTTT_DTYPE_BF16 ? 2 : 4; }

struct ChainLayout {
  size_t pq, kk, hh, zz, zzb, hhb, h_all, du_all, dg_all, dz_all, u_cur, g_cur, zp, loss, npart, coef, total;
  size_t gpart_k, gpart_l, gcnt;  // split-feature Gram partials (key Gram; H / dZ Grams) and counters
  int nsplit, max_key_blocks, ncounters;
};

ChainLayout chain_layout(int64_t B, int64_t L, int64_t D, int64_t F, int32_t dtype) {
  ChainLayout c;
  const size_t e = act_size(dtype);
  const int64_t LL = L * 64, nF = F / 64;
  // the down pass's F splits: about 256 workgroups before the correction splits (config 3: 2
  // splits; measured in the prefills against 1, 3, 4 and 8)
  int64_t s = (256 + (D / 64) * B - 1) / ((D / 64) * B);
  c.nsplit = (int)(s < 1 ? 1 : (s > nF ? nF : s));
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t at = off; off += align_up(bytes); return at; };
  c.pq = take(e * 4 * L * B * 64 * F);
  c.kk = take(sizeof(float) * B * LL * LL);
  c.hh = take(sizeof(float) * B * 64 * LL);
  c.zz = take(sizeof(float) * B * 64 * LL);
  c.zzb = take(sizeof(uint16_t) * B * 64 * LL);
  c.hhb = take(sizeof(uint16_t) * B * 64 * LL);
  c.h_all = take(e * L * B * 64 * F);
  c.du_all = take(e * L * B * 64 * F);
  c.dg_all = take(e * L * B * 64 * F);
  c.dz_all = take(e * L * B * 64 * D);
  c.u_cur = take(sizeof(float) * B * 64 * F);
  c.g_cur = take(sizeof(float) * B * 64 * F);
  c.zp = take(sizeof(float) * (c.nsplit + (L - 1 + kCorrPerSplit - 1) / kCorrPerSplit + 1) * B * 64 * D);
  c.loss = take(sizeof(float) * B * 64);
  c.npart = take(sizeof(float) * B * nF);
  c.coef = take(sizeof(float) * 2 * B * kCoefStride);  // tables of even / odd layers
  // a key Gram launch covers one layer group (at most kPqGroup layers of at most L blocks each);
  // an H or dZ Gram launch one layer's row of blocks.  The two kinds may run at once (the key Gram
  // of stage l beside the rest of stage l - 1), so they have separate partials and counters.
  c.max_key_blocks = (int)(kPqGroup * L);
  const int sk = gram_splits((int)D), sl = std::max(gram_splits((int)D), gram_splits((int)F));
  c.gpart_k = take(sizeof(float) * 4096 * B * c.max_key_blocks * sk);
  c.gpart_l = take(sizeof(float) * 4096 * B * L * sl);
  c.ncounters = (int)(B * (c.max_key_blocks + L));
  c.gcnt = take(sizeof(unsigned) * c.ncounters);
  c.total = off;
  return c;
}

constexpr int kPqTail = 1;
constexpr double kPqSingleBytes = 128.0 * (1 << 20);

// Layers per snapshot-product launch.  A launch reads the four bf16 state tensors once (8 D F
// bytes per row): while that is small, every layer gets its own launch, so the chain can start
// after the first layer's projections and stay one layer behind the forward pass; when it is
// large, groups of kPqGroup layers share it.  Measured: config 2 (100 MB per launch) 74.5 ms
// with single layers against 79.0 ms with groups of four; config 3 (360 MB) 825 ms with groups
// against 882 ms with single layers.
int pq_group_size(int64_t B, int64_t D, int64_t F) {
  return 8.0 * (double)D * (double)F * (double)B <= kPqSingleBytes ? 1 : kPqGroup;
}

// Layer groups of the snapshot products: [0, L - kPqTail) in groups of `size`, then the last
// kPqTail layers one by one, so that little of the chain is left when the forward pass ends.
void pq_group(int l, int L, int size, int& g0, int& g1) {
  const int head = L - min(L, kPqTail);
  if (l >= head || size == 1) {
    g0 = l;
    g1 = l + 1;
    return;
  }
  g0 = l - l % size;
  g1 = min(head, g0 + size);
}

// Selects which of the launches of a stage part are enqueued: those numbered in [begin, end) in
// enqueue order (all of them by default).  Every launch site asks next() with its kernel's name,
// so the numbering and names follow the launch sequence.
struct LaunchGate {
  int begin = 0;
  int end = 1 << 30;
  int count = 0;
  const char** names = nullptr;
  int cap = 0;
  bool next(const char* name) {
    if (names != nullptr && count < cap) names[count] = name;
    const bool go = begin <= count && count < end;
    ++count;
    return go;
  }
};

// Gram block rows [l0, l1) of every row b
template <typename T>
void launch_gram(int B, int l0, int l1, GramArgs g, hipStream_t st, LaunchGate& gate) {
  g.layer = l0;
  g.layer_end = l1;
  if constexpr (sizeof(T) == 2) {
    g.splits = gram_splits(g.kd);
    if (gate.next("k_chain_gram_lds"))
      hipLaunchKernelGGL(k_chain_gram_lds, dim3(row_tile_blocks(B, gram_blocks(l0, l1) * g.splits)), dim3(kThreads), 0,
                         st, g);
  } else if (gate.next("k_chain_gram")) {
    hipLaunchKernelGGL(k_chain_gram<T>, dim3(row_tile_blocks(B, gram_tiles(l0, l1))), dim3(kGramWaves * 64), 0, st, g);
  }
}

template <typename T>
// parts: bit 0 the snapshot products and key Gram rows of the stages, bit 1 the rest
void launch_chain(const uttt_chunk_chain_args& a, char* ws, const ChainLayout& c, hipStream_t st, int first,
                  int last, int parts, LaunchGate& gate) {
  const int B = (int)a.batch, L = (int)a.layers, C = (int)a.tokens, D = (int)a.d_model, F = (int)a.d_ff;
  const int LL = L * 64, nF = F / 64;
  const dim3 blk(kThreads);
  Acts acts{};
  for (int l = 0; l < L; ++l) {
    acts.k.p[l] = a.k[l];
    acts.v.p[l] = a.v[l];
    acts.eta.p[l] = a.eta[l];
    acts.alpha.p[l] = a.alpha[l];
  }
  acts.kv_rs = a.kv_row_stride;
  acts.kv_ts = D;
  acts.ea_rs = a.ea_row_stride;
  acts.ea_ts = 1;
  float* coef = reinterpret_cast<float*>(ws + c.coef);
  float* kk = reinterpret_cast<float*>(ws + c.kk);
  float* hh = reinterpret_cast<float*>(ws + c.hh);
  float* zz = reinterpret_cast<float*>(ws + c.zz);
  float* u_cur = reinterpret_cast<float*>(ws + c.u_cur);
  float* g_cur = reinterpret_cast<float*>(ws + c.g_cur);
  float* zp = reinterpret_cast<float*>(ws + c.zp);
  float* loss = reinterpret_cast<float*>(ws + c.loss);
  float* npart = reinterpret_cast<float*>(ws + c.npart);
  void* h_all = ws + c.h_all;
  void* du_all = ws + c.du_all;
  void* dg_all = ws + c.dg_all;
  void* dz_all = ws + c.dz_all;
  const int64_t lf = (int64_t)B * 64 * F, ld = (int64_t)B * 64 * D;
  const size_t e = sizeof(T);

  // stage l (< L): layer l (stage 0 also initialises the coefficient table); stage L: the last
  // layer's recurrence step and the state write
  auto want = [&](int stage) { return first <= stage && stage <= last; };
  const bool keys_part = parts & 1, rest_part = parts & 2;
  const int ncoef = B * kCoefStride;  // table of layer 0
  unsigned* gcnt = reinterpret_cast<unsigned*>(ws + c.gcnt);
  if (want(0) && keys_part && gate.next("k_chain_init")) {
    const int n = std::max(ncoef, c.ncounters);
    hipLaunchKernelGGL(k_chain_init, dim3((n + kThreads - 1) / kThreads), blk, 0, st, coef, ncoef, gcnt, c.ncounters);
  }

  // the chunk-start state the bf16 kernels read: its bf16 copies when given, else the masters
  const bool bf16_src = a.w_up_copy != nullptr;
  PqArgs pa{};
  pa.B = B; pa.L = L; pa.C = C; pa.D = D; pa.F = F; pa.acts = acts;
  if (bf16_src) {
    pa.x[0] = a.w_up_copy; pa.x[1] = a.s_up_copy; pa.x[2] = a.w_gate_copy; pa.x[3] = a.s_gate_copy;
  } else {
    pa.x[0] = a.w_up; pa.x[1] = a.s_up; pa.x[2] = a.w_gate; pa.x[3] = a.s_gate;
  }
  pa.pq = ws + c.pq;
  pa.s_only = a.w_products_given != 0;
  const dim3 pq_grid(row_tile_blocks(B, (pa.s_only ? 2 : 4) * nF));  // one layer group per launch
  const void* wd_src = bf16_src ? a.w_down_copy : static_cast<const void*>(a.w_down);
  const void* sd_src = bf16_src ? a.s_down_copy : static_cast<const void*>(a.s_down);

  GramArgs ka{};  // K_l K_j^T rows of the key Gram (B, LL, LL)
  ka.B = B; ka.L = L; ka.C = C; ka.kd = D; ka.LL = LL; ka.rs = a.kv_row_stride; ka.ts = D;
  ka.x = acts.k; ka.out = kk; ka.out_rows = LL; ka.out_r0 = 0; ka.out_lstep = 64;
  ka.part = reinterpret_cast<float*>(ws + c.gpart_k); ka.counters = gcnt;

  GramArgs ha{};  // H_l H_j^T and dZ_l dZ_j^T: the layer buffers have stride 64 rows per row b
  ha.B = B; ha.L = L; ha.C = C; ha.LL = LL; ha.out_rows = 64; ha.out_r0 = 0; ha.out_lstep = 0;
  ha.part = reinterpret_cast<float*>(ws + c.gpart_l); ha.counters = gcnt + (size_t)B * c.max_key_blocks;
  GramArgs za = ha;
  ha.kd = F; ha.rs = (int64_t)64 * F; ha.ts = F; ha.out = hh;
  za.kd = D; za.rs = (int64_t)64 * D; za.ts = D; za.out = zz;
  for (int l = 0; l < L; ++l) {
    ha.x.p[l] = static_cast<char*>(h_all) + e * l * lf;
    za.x.p[l] = static_cast<char*>(dz_all) + e * l * ld;
  }

  // coefficient table of layer l (the state before layer l's update) at table(l); layer l's
  // recurrence step runs inside layer l + 1's k_chain_up, the last one in k_chain_coef
  auto table = [&](int l) { return coef + (size_t)(l & 1) * B * kCoefStride; };
  auto coef_step = [&](int l) {
    CoefArgs ca{};
    ca.B = B; ca.C = C; ca.LL = LL; ca.l = l; ca.nF = nF;
    ca.beta = a.momentum_beta; ca.max_norm = a.max_inner_grad_norm; ca.min_row_surprise = a.min_row_surprise;
    ca.npart = npart; ca.hh = hh; ca.zz = zz; ca.acts = acts;
    ca.mask = a.token_mask; ca.mask_rs = a.mask_row_stride; ca.loss = loss;
    ca.src = table(l); ca.dst = table(l + 1);
    ca.surprise = a.surprise; ca.row_loss = a.row_loss;
    return ca;
  };
  // Layers run in groups of kPqGroup: once a group's last layer is known (its stage), one
  // launch forms the snapshot products of the whole group, then each layer of the group runs.
  // Stages of the other layers of a group launch nothing.
  // with the W products given (S products only, half the state read per launch) single layers
  // measured as fast or faster at every config (config 5: 1.41 s against 1.43 s per batch)
  const int gsize = a.w_products_given ? 1 : pq_group_size(B, D, F);
  for (int l = 0; l < L; ++l) {
    int g0, g1;  // this layer's group [g0, g1)
    pq_group(l, L, gsize, g0, g1);
    if (!want(g1 - 1)) continue;
    if (l == g0 && keys_part) {
      pa.l_begin = g0;
      pa.l_count = g1 - g0;
      if (g1 - g0 == 1) {  // a single layer: one staged K tile, less LDS per workgroup
        if (sizeof(T) == 2 && bf16_src) {
          // the snapshot products and the key Gram row in one launch
          ka.layer = g0;
          ka.layer_end = g1;
          ka.splits = gram_splits(ka.kd);
          const int npq = (int)pq_grid.x;
          const int ngram = row_tile_blocks(B, gram_blocks(g0, g1) * ka.splits);
          if (gate.next("k_chain_keys_lds"))
            hipLaunchKernelGGL(k_chain_keys_lds, dim3(npq + ngram), blk, 0, st, pa, ka, npq);
        } else if (bf16_src) {
          if (gate.next("k_chain_pq")) hipLaunchKernelGGL((k_chain_pq<T, bf16, 1>), pq_grid, blk, 0, st, pa);
        } else if (gate.next("k_chain_pq")) {
          hipLaunchKernelGGL((k_chain_pq<T, float, 1>), pq_grid, blk, 0, st, pa);
        }
      } else if (bf16_src) {
        if (gate.next("k_chain_pq")) hipLaunchKernelGGL((k_chain_pq<T, bf16, kPqGroup>), pq_grid, blk, 0, st, pa);
      } else if (gate.next("k_chain_pq")) {
        hipLaunchKernelGGL((k_chain_pq<T, float, kPqGroup>), pq_grid, blk, 0, st, pa);
      }
    }
    const bool keys_fused = sizeof(T) == 2 && bf16_src && g1 - g0 == 1;  // launched with the products
    if (l == g0 && keys_part && !keys_fused) {  // key Gram rows of the whole group
      ka.layer = g0;
      ka.layer_end = g1;
      launch_gram<T>(B, g0, g1, ka, st, gate);
    }
    if (!rest_part) continue;
    const float* cl = table(l);

    UpArgs ua{};
    ua.B = B; ua.L = L; ua.C = C; ua.D = D; ua.F = F; ua.LL = LL; ua.l = l;
    if (l > 0) ua.prev = coef_step(l - 1);
    ua.coef = cl; ua.pq = ws + c.pq; ua.kk = kk; ua.du_all = du_all; ua.dg_all = dg_all;
    ua.u_cur = u_cur; ua.g_cur = g_cur; ua.h_all = h_all;
    if constexpr (sizeof(T) == 2) {
      if (gate.next("k_chain_up_lds")) hipLaunchKernelGGL(k_chain_up_lds, dim3(row_tile_blocks(B, nF)), blk, 0, st, ua);
    } else if (gate.next("k_chain_up")) {
      hipLaunchKernelGGL(k_chain_up<T>, dim3(row_tile_blocks(B, nF)), blk, 0, st, ua);
    }

    ha.layer = l;
    ha.layer_end = l + 1;
    if (sizeof(T) == 2 && bf16_src) {  // the bf16 down pass reads the row scaled by this layer's gammas
      ha.scaled = reinterpret_cast<bf16*>(ws + c.hhb);
      ha.coef = cl;
    }
    launch_gram<T>(B, l, l + 1, ha, st, gate);

    DownArgs da{};
    da.B = B; da.L = L; da.C = C; da.D = D; da.F = F; da.LL = LL; da.l = l; da.nsplit = c.nsplit;
    da.coef = cl; da.h_all = h_all; da.wd = wd_src; da.sd = sd_src; da.hh = hh; da.dz_all = dz_all; da.zp = zp;
    da.hhb = reinterpret_cast<const bf16*>(ws + c.hhb);
    const int ncorr = (l + kCorrPerSplit - 1) / kCorrPerSplit;
    const dim3 down_grid(row_tile_blocks(B, (D / 64) * (c.nsplit + ncorr)));
    if (sizeof(T) == 2 && bf16_src) {
      if (gate.next("k_chain_down_lds")) hipLaunchKernelGGL(k_chain_down_lds, down_grid, blk, 0, st, da);
    } else if (bf16_src) {
      if (gate.next("k_chain_down")) hipLaunchKernelGGL((k_chain_down<T, bf16>), down_grid, blk, 0, st, da);
    } else if (gate.next("k_chain_down")) {
      hipLaunchKernelGGL((k_chain_down<T, float>), down_grid, blk, 0, st, da);
    }

    LnGradArgs g{};
    g.B = B; g.C = C; g.D = D; g.nsplit = c.nsplit + ncorr; g.tok_pad = 64;
    g.normalize = a.normalize_by_dim; g.eps = a.eps; g.zp = zp;
    g.k = a.k[l]; g.k_rs = a.kv_row_stride; g.v = a.v[l]; g.v_rs = a.kv_row_stride;
    g.eta = a.eta[l]; g.eta_rs = a.ea_row_stride;
    g.mask = a.token_mask; g.mask_rs = a.mask_row_stride;
    g.ln_w = a.ln_weight; g.ln_b = a.ln_bias;
    g.dz = static_cast<char*>(dz_all) + e * l * ld;
    g.loss = loss;
    if (gate.next("k_ln_grad")) launch_ln_grad<T>(dim3(64, B), st, g);

    za.layer = l;
    za.layer_end = l + 1;
    if (sizeof(T) == 2 && bf16_src) {  // the bf16 back pass reads the row scaled by this layer's gammas
      za.scaled = reinterpret_cast<bf16*>(ws + c.zzb);
      za.coef = cl;
    }
    launch_gram<T>(B, l, l + 1, za, st, gate);

    BackArgs ba{};
    ba.B = B; ba.L = L; ba.C = C; ba.D = D; ba.F = F; ba.LL = LL; ba.l = l;
    ba.coef = cl; ba.dz_all = dz_all; ba.wd = wd_src; ba.sd = sd_src; ba.zz = zz; ba.h_all = h_all;
    ba.zzb = reinterpret_cast<const bf16*>(ws + c.zzb);
    ba.u_cur = u_cur; ba.g_cur = g_cur; ba.kk = kk; ba.du_all = du_all; ba.dg_all = dg_all; ba.npart = npart;
    if (sizeof(T) == 2 && bf16_src) {
      if (gate.next("k_chain_back_lds"))
        hipLaunchKernelGGL(k_chain_back_lds, dim3(row_tile_blocks(B, nF)), blk, 0, st, ba);
    } else if (bf16_src) {
      if (gate.next("k_chain_back")) hipLaunchKernelGGL((k_chain_back<T, bf16>), dim3(row_tile_blocks(B, nF)), blk, 0, st, ba);
    } else if (gate.next("k_chain_back")) {
      hipLaunchKernelGGL((k_chain_back<T, float>), dim3(row_tile_blocks(B, nF)), blk, 0, st, ba);
    }

  }

  if (want(L) && rest_part && gate.next("k_chain_coef")) {
    const CoefArgs last = coef_step(L - 1);
    hipLaunchKernelGGL(k_chain_coef<T>, dim3(B), blk, 0, st, last);
  }
  ApplyChainArgs aa{};
  aa.B = B; aa.L = L; aa.C = C; aa.D = D; aa.F = F; aa.coef = table(L); aa.acts = acts;
  aa.h_all = h_all; aa.du_all = du_all; aa.dg_all = dg_all; aa.dz_all = dz_all;
  aa.w[0] = a.w_up; aa.w[1] = a.w_gate; aa.w[2] = a.w_down;
  aa.s[0] = a.s_up; aa.s[1] = a.s_gate; aa.s[2] = a.s_down;
  aa.wc[0] = static_cast<bf16*>(a.w_up_copy);
  aa.wc[1] = static_cast<bf16*>(a.w_gate_copy);
  aa.wc[2] = static_cast<bf16*>(a.w_down_copy);
  aa.sc[0] = static_cast<bf16*>(a.s_up_copy);
  aa.sc[1] = static_cast<bf16*>(a.s_gate_copy);
  aa.sc[2] = static_cast<bf16*>(a.s_down_copy);
  if (want(L) && rest_part) {
    const dim3 grid(row_tile_blocks(B, 3 * (D / 64) * nF));
    if constexpr (sizeof(T) == 2) {
      if (gate.next("k_chain_apply_lds")) {
        if (apply_wide_fits(D, F)) {
          const int tiles = 2 * (int)((D / (64 * kApplyNA)) * (F / (64 * kApplyNB))) +
                            (int)((F / (64 * kApplyNA)) * (D / (64 * kApplyNB)));
          hipLaunchKernelGGL((k_chain_apply_wide<kApplyNA, kApplyNB, kApplySlotsWide>), dim3(row_tile_blocks(B, tiles)),
                             blk, 0, st, aa);
        } else {
          hipLaunchKernelGGL(k_chain_apply_lds, grid, blk, 0, st, aa);
        }
      }
    } else if (gate.next("k_chain_apply")) {
      hipLaunchKernelGGL(k_chain_apply<T>, grid, blk, 0, st, aa);
    }
  }
}

int check_chain_dims(int64_t B, int64_t L, int64_t D, int64_t F, int32_t dtype) {
  UTTT_REQUIRE(B >= 1 && B <= 65535, "batch must be in [1, 65535] (got %lld)", (long long)B);
  UTTT_REQUIRE(L >= 1 && L <= kMaxChain, "layers must be in [1, %d] (got %lld)", kMaxChain, (long long)L);
  UTTT_REQUIRE(D >= 64 && D % 64 == 0 && D <= 4096, "d_model must be a multiple of 64 in [64, 4096] (got %lld)",
               (long long)D);
  UTTT_REQUIRE(F >= 64 && F % 64 == 0, "d_ff must be a positive multiple of 64 (got %lld)", (long long)F);
  UTTT_REQUIRE(dtype == UTTT_DTYPE_F32 || dtype == UTTT_DTYPE_BF16, "act_dtype must be F32 or BF16 (got %d)", dtype);
  UTTT_REQUIRE(3 * (D / 64) * (F / 64) <= 2147483647LL, "state too large");
  UTTT_REQUIRE(D * F * 4 <= 2147483647LL, "d_model * d_ff * 4 must fit 31 bits (got %lld)", (long long)(D * F * 4));
  return UTTT_OK;
}

}  // namespace

}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_chunk_chain_workspace(int64_t batch, int64_t layers, int64_t d_model, int64_t d_ff,
                                             int32_t act_dtype) {
  if (check_chain_dims(batch, layers, d_model, d_ff, act_dtype) != UTTT_OK) return 0;
  return chain_layout(batch, layers, d_model, d_ff, act_dtype).total;
}

static int run_chain(const uttt_chunk_chain_args* a, void* workspace, size_t workspace_bytes, uttt_stream_t stream,
                     int first, int last, int parts = 3, LaunchGate* gate = nullptr) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  int rc = check_chain_dims(a->batch, a->layers, a->d_model, a->d_ff, a->act_dtype);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->tokens >= 1 && a->tokens <= 64, "tokens per chunk must be in [1, 64] (got %lld)",
               (long long)a->tokens);
  const int64_t vec = a->act_dtype == UTTT_DTYPE_BF16 ? 8 : 4;
  const int64_t known = last < a->layers ? (int64_t)last + 1 : a->layers;  // layers these stages read
  for (int64_t l = 0; l < known; ++l) {
    UTTT_REQUIRE(a->k[l] && a->v[l] && a->eta[l] && a->alpha[l], "k/v/eta/alpha of layer %lld must be non-NULL",
                 (long long)l);
    UTTT_REQUIRE(aligned16(a->k[l]) && aligned16(a->v[l]), "k/v of layer %lld must be 16-byte aligned", (long long)l);
  }
  UTTT_REQUIRE(a->kv_row_stride % vec == 0, "k/v row stride must be a multiple of 16 bytes");
  UTTT_REQUIRE(a->batch == 1 || (a->kv_row_stride >= a->tokens * a->d_model && a->ea_row_stride >= a->tokens),
               "k/v and eta/alpha row strides must cover the chunk's tokens");
  UTTT_REQUIRE(a->w_up && a->w_gate && a->w_down && a->s_up && a->s_gate && a->s_down, "state pointers must be non-NULL");
  UTTT_REQUIRE(aligned16(a->w_up) && aligned16(a->w_gate) && aligned16(a->w_down) && aligned16(a->s_up) &&
               aligned16(a->s_gate) && aligned16(a->s_down), "state pointers must be 16-byte aligned");
  UTTT_REQUIRE(a->ln_weight && a->ln_bias && a->surprise, "ln_weight/ln_bias/surprise must be non-NULL");
  const bool any_copy = a->w_up_copy || a->w_gate_copy || a->w_down_copy || a->s_up_copy || a->s_gate_copy ||
                        a->s_down_copy;
  const bool all_copy = a->w_up_copy && a->w_gate_copy && a->w_down_copy && a->s_up_copy && a->s_gate_copy &&
                        a->s_down_copy;
  UTTT_REQUIRE(!any_copy || (all_copy && a->act_dtype == UTTT_DTYPE_BF16),
               "bf16 state copies must be given all six or none, and only with bf16 activations");
  UTTT_REQUIRE(!any_copy || (aligned16(a->w_up_copy) && aligned16(a->w_gate_copy) && aligned16(a->w_down_copy) &&
                             aligned16(a->s_up_copy) && aligned16(a->s_gate_copy) && aligned16(a->s_down_copy)),
               "bf16 state copies must be 16-byte aligned");
  UTTT_REQUIRE(a->momentum_beta >= 0.f && a->max_inner_grad_norm >= 0.f && a->min_row_surprise >= 0.f,
               "momentum_beta, max_inner_grad_norm and min_row_surprise must be >= 0");
  UTTT_REQUIRE(!a->w_products_given || all_copy, "w_products_given needs the bf16 state copies");
  const ChainLayout c = chain_layout(a->batch, a->layers, a->d_model, a->d_ff, a->act_dtype);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= c.total, "workspace too small: need %zu bytes, got %zu",
               c.total, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  LaunchGate every;
  LaunchGate& g = gate != nullptr ? *gate : every;
  if (a->act_dtype == UTTT_DTYPE_BF16)
    launch_chain<bf16>(*a, ws, c, st, first, last, parts, g);
  else
    launch_chain<float>(*a, ws, c, st, first, last, parts, g);
  return launch_status("uttt_chunk_chain");
}

extern "C" int uttt_chunk_chain(const uttt_chunk_chain_args* a, void* workspace, size_t workspace_bytes,
                                uttt_stream_t stream) {
  return run_chain(a, workspace, workspace_bytes, stream, 0, 1 << 30);
}

extern "C" int uttt_chunk_chain_stage(const uttt_chunk_chain_args* a, void* workspace, size_t workspace_bytes,
                                      int32_t stage, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(stage >= 0 && stage <= a->layers, "stage must be in [0, layers] (got %d)", stage);
  return run_chain(a, workspace, workspace_bytes, stream, stage, stage);
}

extern "C" int uttt_chunk_chain_stage_part(const uttt_chunk_chain_args* a, void* workspace, size_t workspace_bytes,
                                           int32_t stage, int32_t part, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(stage >= 0 && stage <= a->layers, "stage must be in [0, layers] (got %d)", stage);
  UTTT_REQUIRE(part >= 0 && part <= 2, "part must be 0 (whole stage), 1 or 2 (got %d)", part);
  return run_chain(a, workspace, workspace_bytes, stream, stage, stage, part == 0 ? 3 : part);
}

extern "C" int uttt_chunk_chain_stage_launch(const uttt_chunk_chain_args* a, void* workspace, size_t workspace_bytes,
                                             int32_t stage, int32_t part, int32_t launch_begin, int32_t launch_end,
                                             const char** names, int32_t names_cap, int32_t* count,
                                             uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(stage >= 0 && stage <= a->layers, "stage must be in [0, layers] (got %d)", stage);
  UTTT_REQUIRE(part >= 0 && part <= 2, "part must be 0 (whole stage), 1 or 2 (got %d)", part);
  UTTT_REQUIRE(names_cap >= 0 && (names != nullptr || names_cap == 0), "names_cap must be >= 0 with names");
  UTTT_REQUIRE(launch_begin >= 0, "launch_begin must be >= 0 (got %d)", launch_begin);
  LaunchGate gate;
  gate.begin = launch_begin;
  gate.end = launch_end;
  gate.names = names;
  gate.cap = names_cap;
  const int rc = run_chain(a, workspace, workspace_bytes, stream, stage, stage, part == 0 ? 3 : part, &gate);
  if (count != nullptr) *count = gate.count;
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(launch_end <= launch_begin || launch_end <= gate.count,
               "launches [%d, %d) out of range: stage %d part %d makes %d launches", launch_begin, launch_end, stage,
               part, gate.count);
  return UTTT_OK;
}

extern "C" int uttt_chunk_chain_w_products(int64_t batch, int64_t layers, int64_t d_model, int64_t d_ff,
                                           int32_t act_dtype, int32_t layer, size_t* up_offset, size_t* gate_offset) {
  int rc = check_chain_dims(batch, layers, d_model, d_ff, act_dtype);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(layer >= 0 && layer < layers, "layer must be in [0, layers) (got %d)", layer);
  UTTT_REQUIRE(up_offset != nullptr && gate_offset != nullptr, "offset outputs must be non-NULL");
  const ChainLayout c = chain_layout(batch, layers, d_model, d_ff, act_dtype);
  const size_t slot = act_size(act_dtype) * (size_t)batch * 64 * (size_t)d_ff;  // one (m, layer) slot
  *up_offset = c.pq + slot * (size_t)(0 * layers + layer);
  *gate_offset = c.pq + slot * (size_t)(2 * layers + layer);
  return UTTT_OK;
}
