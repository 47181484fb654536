// Fused chunk fast-weight update and frozen readout for the uTTT shared fast-weight
// pool, written for gfx950 (MI355X).
//
// Math (per row b; K, V, Q are C x D chunk activations, W fp32 master state):
//   U = K W_up, G = K W_gate, H = SiLU(G) * U, Z = H W_down
//   Zh = LN(Z) (fp32 stats), E = K + gamma*Zh + beta - V, loss_t = 0.5 |E_t|^2 / s
//   dZh = (w_t / s) E gamma, dZ = rstd (dZh - mean(dZh) - Zh mean(dZh Zh))
//   gW_down = H^T dZ, dH = dZ W_down^T, dU = dH G sig(G), dG = dH U sig(G)(1 + G(1 - sig(G)))
//   gW_up = K^T dU, gW_gate = K^T dG
//   clip c = min(1, tau / sqrt(|g|^2 + 1e-8)); S' = beta S - c g; W' = (1 - mean alpha) W + S'
//   readout O = Q + LN((SiLU(Q R_gate) * Q R_up) R_down)   (R = read snapshot)
// (reference: model/uttt_layer.py:279-534)
//
// Kernel sequence for one chunk (all rows in each launch):
//   1. k_up_gate      U/G/H for the K path (cursor W) and the Q path (read W), per F tile
//   2. k_down_partial Z partial sums over F splits, per D tile
//   3. k_ln_grad      LN + loss + dZ per token (K path)
//   4. k_ln_readout   LN + residual readout per token (Q path)
//   5. k_backward     dH, dU, dG per F tile + the per-row squared gradient norm partial
//   6. k_apply        recompute each gradient tile from the small activations and apply
//                     clip / momentum / decay / inactive-row select to W and S in one pass
// Steps 1, 2 and 4 alone are the frozen readout.
#include <algorithm>
#include <mutex>

#include "update_ln.h"
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {

constexpr int KT = 64;  // K depth of one LDS stage

template <typename T> constexpr int lds_ld() { return KT + Mma<T>::kPad; }

struct FwdArgs {
  int B, D, F, ntok, ntb, tok_pad, nsplit;
  const void* x[2];
  int64_t x_rs[2];
  const void* wu[2];  // fp32 (update) or the weight type WT of the readout
  const void* wg[2];
  const void* wd[2];
  int64_t w_rs[2];
  float* u_store;  // fp32 (B, tok_pad, F), path 0 only; may be null
  float* g_store;
  void* h[2];      // act dtype (B, tok_pad, F)
  float* zp;       // fp32 (paths, nsplit, B, tok_pad, D)
  // optional key block (readout only): the last z block multiplies these rows (token stride D)
  // by path 0's W_up / W_gate and writes both products (act dtype, (B, 64, F)) instead of H
  const void* kx;
  int64_t kx_rs;
  void* ku;
  void* kg;
  // one token per row (the GEMV readout) only: optional RMSNorm of x, and the LN + residual
  // in each row's last F block when row counters are given
  const void* xn_w;
  float xn_eps;
  unsigned* counters;
  float ln_eps;
  const float* ln_w;
  const float* ln_b;
  void* out;
  int64_t out_rs;
  int rev;  // GEMV only: walk the weight rows in descending order
};

// ---------------------------------------------------------------------------
// 1. U, G, H for one (F tile, row, path, token block)
// ---------------------------------------------------------------------------
template <typename T, typename WT, int KTL = KT>
__global__ void __launch_bounds__(kThreads) k_up_gate(const FwdArgs a) {
  constexpr int LD = KTL + Mma<T>::kPad;
  __shared__ __align__(16) T xs[64 * LD];
  __shared__ __align__(16) T us[64 * LD];
  __shared__ __align__(16) T gs[64 * LD];
  const int ft = blockIdx.x, b = blockIdx.y;
  const bool key_block = a.kx != nullptr && blockIdx.z == gridDim.z - 1;
  const int path = key_block ? 0 : blockIdx.z / a.ntb, tb = key_block ? 0 : blockIdx.z - path * a.ntb;
  const int f0 = ft * 64, t0 = tb * 64;
  const int rows = min(64, a.ntok - t0);
  const T* x = key_block ? static_cast<const T*>(a.kx) + (int64_t)b * a.kx_rs
                         : static_cast<const T*>(a.x[path]) + (int64_t)b * a.x_rs[path] + (int64_t)t0 * a.D;
  // threads [0, U) stage W_up, [U, 2U) W_gate (U units of 8 rows x one 16-byte chunk)
  constexpr int U = ColStage<WT, KTL>::kUnits;
  static_assert(2 * U <= kThreads, "W_up and W_gate stage in separate halves of the workgroup");
  const bool up_half = threadIdx.x < U;
  const WT* wsrc = static_cast<const WT*>(up_half ? a.wu[path] : a.wg[path]) + (int64_t)b * a.w_rs[path] + f0;
  T* wdst = up_half ? us : gs;
  const int unit = up_half ? (int)threadIdx.x : min((int)threadIdx.x - U, U);
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;

  RowStage<T, KTL> xst;
  ColStage<WT, KTL> wst;
  xst.load(x, a.D, rows);
  wst.load(wsrc, a.F, KTL, unit);
  f32x16 au, ag;
  zero(au);
  zero(ag);
  for (int d0 = 0; d0 < a.D; d0 += KTL) {
    xst.template store<T>(xs, LD);
    wst.template store<T>(wdst, LD);
    __syncthreads();
    if (d0 + KTL < a.D) {
      xst.load(x + d0 + KTL, a.D, rows);
      wst.load(wsrc + (int64_t)(d0 + KTL) * a.F, a.F, KTL, unit);
    }
    wave_mma<T, KTL>(au, xs + wr * LD, LD, us + wc * LD, LD);
    wave_mma<T, KTL>(ag, xs + wr * LD, LD, gs + wc * LD, LD);
    __syncthreads();
  }

  const int col = wc + acc_col();
  if (key_block) {  // both products, rows past ntok are 0 (zero-filled key rows)
    T* ku = static_cast<T*>(a.ku) + (int64_t)b * 64 * a.F + f0;
    T* kg = static_cast<T*>(a.kg) + (int64_t)b * 64 * a.F + f0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
      ku[off] = from_f32<T>(au[i]);
      kg[off] = from_f32<T>(ag[i]);
    }
    return;
  }
  const int64_t base = ((int64_t)b * a.tok_pad + t0) * a.F + f0;
  T* h = static_cast<T*>(a.h[path]) + base;
  const bool store_ug = path == 0 && a.u_store != nullptr;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = wr + acc_row(i);
    const float u = au[i], g = ag[i];
    const int64_t off = (int64_t)row * a.F + col;
    h[off] = from_f32<T>((g * sigmoidf_acc(g)) * u);
    if (store_ug) {
      a.u_store[base + off] = u;
      a.g_store[base + off] = g;
    }
  }
}

// Readout with bf16 activations and weights over one token block (tokens <= 64): the token rows
// (and key rows) and the W_up / W_gate tiles go straight from global memory into LDS through a
// ring of k steps of 64 (up to SLOTS - 1 steps' loads in flight); the W tiles reach the MFMA
// through transposing reads.  With keys, 8 waves: waves 0-3 take the token rows, 4-7 the key
// rows, and every W tile in LDS serves both.  A workgroup covers NB 64-column slabs of F: with
// NB = 2 (F a multiple of 128) the config-3 grid is 43 x 4 = 172 workgroups, one round on the
// GPU's CUs, instead of 86 x 4 = 344 (two rounds at one workgroup per CU), and each token row
// tile serves twice the weight columns.  The products accumulate over d in the same order as
// k_up_gate's and the chain's snapshot products for every NB.
template <int NB> constexpr int ug_slots() { return NB == 1 ? 4 : 3; }

template <bool KEYS, int NB>
__global__ void __launch_bounds__(KEYS ? 512 : 256) k_up_gate_lds(const FwdArgs a) {
  constexpr int NW = KEYS ? 8 : 4;
  constexpr int NA = KEYS ? 2 : 1;            // row tiles per step
  constexpr int NS = NA + 2 * NB;             // 8 KB tiles per step: row tiles, W_up slabs, W_gate slabs
  constexpr int SLOTS = ug_slots<NB>();
  constexpr int kSlot = NS * 8192;
  constexpr int PER = NS * 8 / NW;            // load instructions per wave per step
  static_assert((NS * 8) % NW == 0, "the step's row groups split evenly over the waves");
  __shared__ __align__(1024) char ring[SLOTS * kSlot];
  const RowTile rt = row_tile(blockIdx.x, a.B, a.F / (64 * NB));  // a row's tiles share its token rows
  if (!rt.valid) return;
  const int ft = rt.tile, b = rt.b, f0 = ft * 64 * NB;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int set = w >> 2, w4 = w & 3;  // row set: 0 token rows, 1 key rows
  const int wr = (w4 >> 1) * 32, wc = (w4 & 1) * 32 * NB;
  const int rows = min(64, a.ntok);
  const bf16* xq = static_cast<const bf16*>(a.x[0]) + (int64_t)b * a.x_rs[0];
  const bf16* xk = KEYS ? static_cast<const bf16*>(a.kx) + (int64_t)b * a.kx_rs : xq;
  const bf16* wu = static_cast<const bf16*>(a.wu[0]) + (int64_t)b * a.w_rs[0] + f0;
  const bf16* wg = static_cast<const bf16*>(a.wg[0]) + (int64_t)b * a.w_rs[0] + f0;
  // row group g of a step: g < 8 NA row tiles (8 rows each), then NB W_up slabs and NB W_gate
  // slabs (8 d rows each); wave w loads groups w, w + NW, ...; its LDS destination is slot + 1 KB g
  int voff[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + NW * i;
    voff[i] = g < NA * 8 ? row_src_off(g & 7, lane, a.D) : slab_src_off(g & 7, lane, a.F);
  }
  const uint32_t ring0 = lds_addr(ring);
  const int nsteps = a.D / 64;
  const bool nt = stream_nt(a.B, a.D, a.F);  // the streamed state copies: non-temporal
  auto issue = [&](int step) {
    const int d0 = step * 64;
    const uint32_t base = ring0 + (uint32_t)((step % SLOTS) * kSlot);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int g = w + NW * i, ti = g / 8;
      __amdgpu_buffer_rsrc_t r;
      if (ti < NA) {  // rows past `rows` are out of the buffer range: zeros
        r = buffer_rsrc((ti == 0 ? xq : xk) + d0, (uint32_t)(rows * a.D * 2));
      } else {  // slab h of W_up or W_gate: 64 h columns in, its range ends 128 h bytes early
        const int sl = ti - NA, h = sl % NB;
        r = buffer_rsrc((sl < NB ? wu : wg) + (int64_t)d0 * a.F + 64 * h, (uint32_t)(64 * a.F * 2 - 128 * h));
      }
      buffer_load_lds16(ti >= NA && nt, r, lds_ptr(base + (uint32_t)(g * 1024)), voff[i]);
    }
  };
  for (int j = 0; j < min(nsteps, SLOTS - 1); ++j) issue(j);
  uint32_t ta[4], tu[NB], tg[NB];
#pragma unroll
  for (int k = 0; k < 4; ++k) ta[k] = row_frag_addr(ring0 + (uint32_t)(set * 8192), wr, lane, k);
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const int c = wc + 32 * cb;
    tu[cb] = slab_tr_addr(ring0 + (uint32_t)((NA + c / 64) * 8192), c % 64, lane);
    tg[cb] = slab_tr_addr(ring0 + (uint32_t)((NA + NB + c / 64) * 8192), c % 64, lane);
  }
  f32x16 au[NB], ag[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    zero(au[cb]);
    zero(ag[cb]);
  }
  for (int step = 0; step < nsteps; ++step) {
    wait_steps<PER, SLOTS - 2>(min(nsteps - 1, step + SLOTS - 2) - step);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the last step's slot is free
    if (step + SLOTS - 1 < nsteps) issue(step + SLOTS - 1);
    const uint32_t so = (uint32_t)((step % SLOTS) * kSlot);
    bf16x8 fa[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) fa[k] = lds_read_bf16x8<0>(ta[k] + so);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      bf16x8 fu[4], fg[4];
      slab_frags(tu[cb] + so, fu);
      slab_frags(tg[cb] + so, fg);
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fu[0]), "+v"(fu[1]), "+v"(fu[2]),
                     "+v"(fu[3]), "+v"(fg[0]), "+v"(fg[1]), "+v"(fg[2]), "+v"(fg[3]));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        au[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fu[k], au[cb], 0, 0, 0);
        ag[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fg[k], ag[cb], 0, 0, 0);
      }
    }
  }
  if (KEYS && set == 1) {  // both key products, rows past ntok are 0 (zero key rows)
    bf16* ku = static_cast<bf16*>(a.ku) + (int64_t)b * 64 * a.F + f0;
    bf16* kg = static_cast<bf16*>(a.kg) + (int64_t)b * 64 * a.F + f0;
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const int col = wc + 32 * cb + acc_col();
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t off = (int64_t)(wr + acc_row(i)) * a.F + col;
        ku[off] = from_f32<bf16>(au[cb][i]);
        kg[off] = from_f32<bf16>(ag[cb][i]);
      }
    }
    return;
  }
  bf16* h = static_cast<bf16*>(a.h[0]) + (int64_t)b * a.tok_pad * a.F + f0;
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const int col = wc + 32 * cb + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float u = au[cb][i], g = ag[cb][i];
      h[(int64_t)(wr + acc_row(i)) * a.F + col] = from_f32<bf16>((g * sigmoidf_acc(g)) * u);
    }
  }
}

// ---------------------------------------------------------------------------
// 2. Z partial = H[:, split] W_down[split, D tile]
// ---------------------------------------------------------------------------
template <typename T, typename WT, int KTL = KT>
__global__ void __launch_bounds__(kThreads) k_down_partial(const FwdArgs a) {
  constexpr int LD = KTL + Mma<T>::kPad;
  __shared__ __align__(16) T hs[64 * LD];
  __shared__ __align__(16) T ws[64 * LD];
  const int dt = blockIdx.x, split = blockIdx.y;
  const int b = blockIdx.z % a.B, pt = blockIdx.z / a.B;
  const int path = pt / a.ntb, tb = pt - path * a.ntb;
  const int d0 = dt * 64, t0 = tb * 64;
  const int nK = a.F / KTL;  // F ranges in whole K tiles
  const int f_begin = (nK * split / a.nsplit) * KTL, f_end = (nK * (split + 1) / a.nsplit) * KTL;
  const T* h = static_cast<const T*>(a.h[path]) + ((int64_t)b * a.tok_pad + t0) * a.F;
  const WT* wd = static_cast<const WT*>(a.wd[path]) + (int64_t)b * a.w_rs[path] + d0;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;

  RowStage<T, KTL> hst;
  ColStage<WT, KTL> wst;  // W_down rows f, columns d -> [d][f]
  f32x16 acc;
  zero(acc);
  if (f_begin < f_end) {
    hst.load(h + f_begin, a.F, 64);
    wst.load(wd + (int64_t)f_begin * a.D, a.D, KTL, threadIdx.x);
  }
  for (int f0 = f_begin; f0 < f_end; f0 += KTL) {
    hst.template store<T>(hs, LD);
    wst.template store<T>(ws, LD);
    __syncthreads();
    if (f0 + KTL < f_end) {
      hst.load(h + f0 + KTL, a.F, 64);
      wst.load(wd + (int64_t)(f0 + KTL) * a.D, a.D, KTL, threadIdx.x);
    }
    wave_mma<T, KTL>(acc, hs + wr * LD, LD, ws + wc * LD, LD);
    __syncthreads();
  }
  float* zp = a.zp + ((((int64_t)path * a.nsplit + split) * a.B + b) * a.tok_pad + t0) * a.D + d0;
  const int col = wc + acc_col();
#pragma unroll
  for (int i = 0; i < 16; ++i) zp[(int64_t)(wr + acc_row(i)) * a.D + col] = acc[i];
}

// bf16 activations and weights: the H rows and W_down tiles of each F step go straight into LDS
// through a ring of kDpSlots steps of 64 (W_down rows f hold 64 d columns: transposing reads);
// the same split boundaries and the same accumulation order as k_down_partial.
constexpr int kDpSlots = 4;

__global__ void __launch_bounds__(kThreads) k_down_partial_lds(const FwdArgs a, int kb) {
  constexpr int kSlot = 2 * 8192;  // H tile, W_down tile
  constexpr int PER = 4;           // 16 row groups per step over 4 waves
  __shared__ __align__(1024) char ring[kDpSlots * kSlot];
  // groups z = (token block, row) of (D / 64) x nsplit tiles, which share the group's H rows
  const int nD = a.D / 64;
  const RowTile rt = row_tile(blockIdx.x, a.ntb * a.B, nD * a.nsplit);
  if (!rt.valid) return;
  const int dt = rt.tile % nD, split = rt.tile / nD;
  const int b = rt.b % a.B, pt = rt.b / a.B;
  const int path = pt / a.ntb, tb = pt - path * a.ntb;
  const int d0 = dt * 64, t0 = tb * 64;
  const int nK = a.F / kb;  // F ranges in whole blocks of kb, as k_down_partial<.., kb>
  const int f_begin = (nK * split / a.nsplit) * kb, f_end = (nK * (split + 1) / a.nsplit) * kb;
  const int nsteps = (f_end - f_begin) / 64;
  const bf16* h = static_cast<const bf16*>(a.h[path]) + ((int64_t)b * a.tok_pad + t0) * a.F + f_begin;
  const bf16* wd = static_cast<const bf16*>(a.wd[path]) + (int64_t)b * a.w_rs[path] + (int64_t)f_begin * a.D + d0;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
  int voff[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + 4 * i;  // groups 0..7: H rows, 8..15: W_down rows
    voff[i] = g < 8 ? row_src_off(g & 7, lane, a.F) : slab_src_off(g & 7, lane, a.D);
  }
  const uint32_t ring0 = lds_addr(ring);
  const bool nt = stream_nt(a.B, a.D, a.F);  // the streamed state copies: non-temporal
  auto issue = [&](int step) {
    const uint32_t base = ring0 + (uint32_t)((step % kDpSlots) * kSlot);
    const __amdgpu_buffer_rsrc_t rh = buffer_rsrc(h + step * 64, (uint32_t)(64 * a.F * 2));
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wd + (int64_t)step * 64 * a.D, (uint32_t)(64 * a.D * 2));
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int g = w + 4 * i;
      buffer_load_lds16(g >= 8 && nt, g < 8 ? rh : rw, lds_ptr(base + (uint32_t)(g * 1024)), voff[i]);
    }
  };
  for (int j = 0; j < min(nsteps, kDpSlots - 1); ++j) issue(j);
  uint32_t ta[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) ta[k] = row_frag_addr(ring0, wr, lane, k);
  const uint32_t tw = slab_tr_addr(ring0 + 8192u, wc, lane);
  f32x16 acc;
  zero(acc);
  for (int step = 0; step < nsteps; ++step) {
    wait_steps<PER, kDpSlots - 2>(min(nsteps - 1, step + kDpSlots - 2) - step);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the last step's slot is free
    if (step + kDpSlots - 1 < nsteps) issue(step + kDpSlots - 1);
    const uint32_t so = (uint32_t)((step % kDpSlots) * kSlot);
    bf16x8 fa[4], fw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) fa[k] = lds_read_bf16x8<0>(ta[k] + so);
    slab_frags(tw + so, fw);
    lds_wait_frags(fa, fw);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k], fw[k], acc, 0, 0, 0);
  }
  float* zp = a.zp + ((((int64_t)path * a.nsplit + split) * a.B + b) * a.tok_pad + t0) * a.D + d0;
  const int col = wc + acc_col();
#pragma unroll
  for (int i = 0; i < 16; ++i) zp[(int64_t)(wr + acc_row(i)) * a.D + col] = acc[i];
}

// ---------------------------------------------------------------------------
// 3. LayerNorm, reconstruction error, token loss and dZ (K path): k_ln_grad, update_ln.h
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// 4. Readout: out = x + LN(Z) with LN parameters rounded to the activation dtype
// ---------------------------------------------------------------------------
struct LnOutArgs {
  int B, ntok, D, nsplit, tok_pad;
  float eps;
  const float* zp;  // partials of the readout path (nsplit, B, tok_pad, D)
  const void* x; int64_t x_rs;
  const float* ln_w;
  const float* ln_b;
  void* out; int64_t out_rs;
  const void* xn_w;  // optional RMSNorm weight applied to x first (one token per row only)
  float xn_eps;
};

// A token row of x into LDS as fp32.  With a norm weight the row becomes RMSNorm(x) with that
// weight, rounded to T as a separate norm's output would be.  Each thread rewrites only the
// entries it staged; the caller synchronises before other threads read them.
template <typename T>
__device__ __forceinline__ void stage_row(const T* x, int D, const T* nw, float neps, float* xs, float* red) {
  float ss = 0.f;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    const float v = to_f32(x[d]);
    xs[d] = v;
    ss += v * v;
  }
  if (nw != nullptr) {
    const float rstd = rsqrtf(block_sum(ss, red) / (float)D + neps);
    for (int d = threadIdx.x; d < D; d += kThreads) xs[d] = to_f32(from_f32<T>(xs[d] * rstd * to_f32(nw[d])));
  }
}

// out = xres + LN(z) for one token row, z the sum of the row's nsplit partials (rows sp_stride
// floats apart), xres the row's residual (the staged fp32 row in LDS, or the row of x itself).  KPER values per thread
// (D <= KPER * 256); the partial rows are loaded four at a time with all their loads in flight
// before any is summed, and always summed in split order.
// AGENT: the partials were written by other workgroups of this launch with device-coherent
// stores; read them the same way (past this CU's L2, which may hold none of them yet)
template <typename T, int KPER, bool AGENT = false, typename XR>
__device__ __forceinline__ void ln_readout_row(const float* z0, int64_t sp_stride, int nsplit, int D, float eps,
                                               const float* ln_w, const float* ln_b, const XR* xres, T* o,
                                               float* red) {
  const float inv_d = 1.0f / (float)D;
  float z[KPER];
#pragma unroll
  for (int i = 0; i < KPER; ++i) z[i] = 0.f;
  constexpr int kGroup = 4;
  for (int sp0 = 0; sp0 < nsplit; sp0 += kGroup) {
    float v[kGroup][KPER];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const float* src = z0 + (int64_t)(sp0 + u) * sp_stride;
#pragma unroll
      for (int i = 0; i < KPER; ++i) {
        const int d = threadIdx.x + i * kThreads;
        if constexpr (AGENT)
          v[u][i] = sp0 + u < nsplit && d < D
                        ? __hip_atomic_load(src + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : 0.f;
        else
          v[u][i] = sp0 + u < nsplit && d < D ? src[d] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u)
#pragma unroll
      for (int i = 0; i < KPER; ++i) z[i] += v[u][i];
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < KPER; ++i) s += z[i];
  const float mean = block_sum(s, red) * inv_d;
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < KPER; ++i) {
    const int d = threadIdx.x + i * kThreads;
    if (d < D) {
      const float c = z[i] - mean;
      s2 += c * c;
    }
  }
  const float rstd = 1.0f / sqrtf(block_sum(s2, red) * inv_d + eps);
#pragma unroll
  for (int i = 0; i < KPER; ++i) {
    const int d = threadIdx.x + i * kThreads;
    if (d < D) {
      const float g = to_f32(from_f32<T>(ln_w[d]));
      const float be = to_f32(from_f32<T>(ln_b[d]));
      o[d] = from_f32<T>(to_f32(xres[d]) + ((z[i] - mean) * rstd * g + be));
    }
  }
}

template <typename T, int KPER>
__global__ void __launch_bounds__(kThreads) k_ln_readout(const LnOutArgs a) {
  __shared__ float red[4];
  __shared__ float xs[KPER * kThreads];
  const int t = blockIdx.x, b = blockIdx.y;
  if (t >= a.ntok) return;
  const T* xr = static_cast<const T*>(a.x) + (int64_t)b * a.x_rs + (int64_t)t * a.D;
  T* o = static_cast<T*>(a.out) + (int64_t)b * a.out_rs + (int64_t)t * a.D;
  const float* z0 = a.zp + ((int64_t)b * a.tok_pad + t) * a.D;
  const int64_t sp_stride = (int64_t)a.B * a.tok_pad * a.D;
  if (a.xn_w == nullptr) {  // the residual is x itself, read where it is used
    ln_readout_row<T, KPER>(z0, sp_stride, a.nsplit, a.D, a.eps, a.ln_w, a.ln_b, xr, o, red);
    return;
  }
  stage_row<T>(xr, a.D, static_cast<const T*>(a.xn_w), a.xn_eps, xs, red);
  __syncthreads();
  ln_readout_row<T, KPER>(z0, sp_stride, a.nsplit, a.D, a.eps, a.ln_w, a.ln_b, xs, o, red);
}

template <typename T>
static void launch_ln_readout(dim3 grid, hipStream_t st, const LnOutArgs& o) {
  if (o.D <= 4 * kThreads)
    hipLaunchKernelGGL((k_ln_readout<T, 4>), grid, dim3(kThreads), 0, st, o);
  else if (o.D <= 8 * kThreads)
    hipLaunchKernelGGL((k_ln_readout<T, 8>), grid, dim3(kThreads), 0, st, o);
  else
    hipLaunchKernelGGL((k_ln_readout<T, 16>), grid, dim3(kThreads), 0, st, o);
}

// ---------------------------------------------------------------------------
// 5. dH = dZ W_down^T per F tile; dU, dG; squared-norm partial of all three gradients
// ---------------------------------------------------------------------------
struct BwdArgs {
  int B, C, D, F, ntb, tok_pad;  // ntb token blocks of 64, tok_pad = 64 ntb
  const void* k; int64_t k_rs;
  const float* wd; int64_t w_rs;
  const float* u_store;
  const float* g_store;
  const void* h;   // K-path H (B, tok_pad, F)
  const void* dz;  // (B, tok_pad, D)
  void* du;        // (B, tok_pad, F)
  void* dg;
  float* nrm;      // (B, F/64), one token block only (longer chunks: k_apply<.., true>)
};

template <typename T>
__global__ void __launch_bounds__(kThreads) k_backward(const BwdArgs a) {
  constexpr int LD = lds_ld<T>();
  __shared__ __align__(16) T buf0[64 * LD];  // dZ rows, then K^T tiles
  __shared__ __align__(16) T buf1[64 * LD];  // W_down rows, then dZ^T tiles
  __shared__ __align__(16) T hts[64 * LD];   // H^T  [f][t]
  __shared__ __align__(16) T dus[64 * LD];   // dU^T [f][t]
  __shared__ __align__(16) T dgs[64 * LD];   // dG^T [f][t]
  __shared__ float red[4];
  const int ft = blockIdx.x, b = blockIdx.y, t0 = blockIdx.z * 64;  // token block blockIdx.z
  const int f0 = ft * 64;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;
  const T* dz = static_cast<const T*>(a.dz) + ((int64_t)b * a.tok_pad + t0) * a.D;
  const float* wd = a.wd + (int64_t)b * a.w_rs + (int64_t)f0 * a.D;
  const T* kr = static_cast<const T*>(a.k) + (int64_t)b * a.k_rs;
  const int64_t rowbase = ((int64_t)b * a.tok_pad + t0) * a.F + f0;

  // dH tile [t][f] over the full D (A = dZ rows, B^T = W_down rows)
  {
    RowStage<T, KT> zst;
    RowStage<float, KT> wst;
    zst.load(dz, a.D, 64);
    wst.load(wd, a.D, 64);
    f32x16 acc;
    zero(acc);
    for (int d0 = 0; d0 < a.D; d0 += KT) {
      zst.template store<T>(buf0, LD);
      wst.template store<T>(buf1, LD);
      __syncthreads();
      if (d0 + KT < a.D) {
        zst.load(dz + d0 + KT, a.D, 64);
        wst.load(wd + d0 + KT, a.D, 64);
      }
      wave_mma<T, KT>(acc, buf0 + wr * LD, LD, buf1 + wc * LD, LD);
      __syncthreads();
    }
    const int f = wc + acc_col();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = wr + acc_row(i);
      const int64_t off = rowbase + (int64_t)t * a.F + f;
      const float u = a.u_store[off], g = a.g_store[off];
      const float sg = sigmoidf_acc(g);
      const float dh = acc[i];
      const T du = from_f32<T>(dh * (g * sg));
      const T dg = from_f32<T>(dh * u * (sg * (1.0f + g * (1.0f - sg))));
      static_cast<T*>(a.du)[off] = du;
      static_cast<T*>(a.dg)[off] = dg;
      dus[f * LD + t] = du;
      dgs[f * LD + t] = dg;
    }
  }
  // with several token blocks the gradient norm needs every block's products: a later launch
  // (k_apply<T, true>) forms it from the whole chunk
  if (a.ntb > 1) return;
  // H^T for this F tile
  {
    ColStage<T, 64> hst;
    hst.load(static_cast<const T*>(a.h) + rowbase, a.F, 64, threadIdx.x);
    hst.template store<T>(hts, LD);
  }

  // |gW_up[:, tile]|^2 + |gW_gate[:, tile]|^2 (rows d) and |gW_down[tile, :]|^2 (cols d)
  constexpr int kUnits = ColStage<T, 64>::kUnits;  // 64 (bf16) or 128 (fp32)
  const bool k_part = threadIdx.x < kUnits;
  const int unit = k_part ? threadIdx.x : threadIdx.x - kUnits;
  ColStage<T, 64> cst;
  const T* csrc = k_part ? kr : dz;
  const int cvalid = k_part ? a.C : 64;
  T* cdst = k_part ? buf0 : buf1;
  cst.load(csrc, a.D, cvalid, unit < kUnits ? unit : kUnits);
  float sq = 0.f;
  for (int d0 = 0; d0 < a.D; d0 += 64) {
    __syncthreads();
    cst.template store<T>(cdst, LD);
    __syncthreads();
    if (d0 + 64 < a.D) cst.load(csrc + d0 + 64, a.D, cvalid, unit < kUnits ? unit : kUnits);
    f32x16 au, ag, ad;
    zero(au);
    zero(ag);
    zero(ad);
    wave_mma<T, 64>(au, buf0 + wr * LD, LD, dus + wc * LD, LD);
    wave_mma<T, 64>(ag, buf0 + wr * LD, LD, dgs + wc * LD, LD);
    wave_mma<T, 64>(ad, hts + wr * LD, LD, buf1 + wc * LD, LD);
#pragma unroll
    for (int i = 0; i < 16; ++i) sq += au[i] * au[i] + ag[i] * ag[i] + ad[i] * ad[i];
  }
  const float total = block_sum(sq, red);
  if (threadIdx.x == 0) a.nrm[b * (a.F / 64) + ft] = total;
}

// ---------------------------------------------------------------------------
// 6. Apply: recompute one gradient tile (K = the chunk's 64 token slots), then
//    S' = beta S - c g, W' = (1 - alpha_bar) W + S', inactive rows copied through.
// ---------------------------------------------------------------------------
struct ApplyArgs {
  int B, C, D, F, ntb, tok_pad;  // ntb token blocks of 64, tok_pad = 64 ntb
  int n_norm;                     // squared-norm partials per row in nrm
  float beta, max_norm;
  const void* k; int64_t k_rs;
  const void* alpha; int64_t alpha_rs;
  const float* mask; int64_t mask_rs;
  const void* h;
  const void* dz;
  const void* du;
  const void* dg;
  float* nrm;  // read by the apply; written (one partial per tile) by the norm-only form
  const float* loss;
  const float* w[3];
  const float* s[3];
  float* w_out[3];
  float* s_out[3];
  float* surprise;
  float* row_loss;  // optional (B, 2): per row sum of masked token losses, number of valid tokens
  float min_row_surprise;  // > 0: rows whose chunk surprise is below it keep W and S
};

// The last wave of an apply workgroup derives its row's clip factor, decay and active flag (and,
// in the first workgroups, the row's loss sums and the batch-global surprise).
template <typename T>
__device__ __forceinline__ void apply_row_scalars(const ApplyArgs& a, int b, float* row_scalar) {
  {
    const int lane = threadIdx.x - 192;
    float n2 = 0.f;
    for (int i = lane; i < a.n_norm; i += 64) n2 += a.nrm[(int64_t)b * a.n_norm + i];
    n2 = wave_sum(n2);
    float asum = 0.f, msum = 0.f, any = 0.f;
    const T* al = static_cast<const T*>(a.alpha) + (int64_t)b * a.alpha_rs;
    for (int t = lane; t < a.C; t += 64) {
      if (a.mask != nullptr) {
        const float mt = a.mask[(int64_t)b * a.mask_rs + t];
        asum += to_f32(al[t]) * mt;
        msum += mt;
        any += (mt != 0.f) ? 1.f : 0.f;
      } else {
        asum += to_f32(al[t]);
      }
    }
    asum = wave_sum(asum);
    msum = wave_sum(msum);
    any = wave_sum(any);
    // this row's chunk surprise (masked mean token loss), for the optional update gate
    float lpart = 0.f;
    for (int t = lane; t < a.C; t += 64) lpart += a.loss[(int64_t)b * a.tok_pad + t];
    const float lsum = wave_sum(lpart);
    const float row_mean = lsum / fmaxf(a.mask != nullptr ? msum : (float)a.C, 1.f);
    if (lane == 0) {
      const float abar = a.mask != nullptr ? asum / fmaxf(msum, 1.f) : asum / (float)a.C;
      row_scalar[0] = a.max_norm > 0.f ? fminf(a.max_norm * (1.0f / sqrtf(n2 + 1e-8f)), 1.0f) : 1.0f;
      row_scalar[1] = 1.0f - abar;
      const bool gated_off = a.min_row_surprise > 0.f && row_mean < a.min_row_surprise;
      row_scalar[2] = ((a.mask == nullptr || any > 0.f) && !gated_off) ? 1.f : 0.f;
    }
    if (blockIdx.x == 0 && a.row_loss != nullptr) {
      float lt = 0.f, mt = 0.f;
      for (int t = lane; t < a.C; t += 64) {
        lt += a.loss[(int64_t)b * a.tok_pad + t];
        mt += a.mask != nullptr ? a.mask[(int64_t)b * a.mask_rs + t] : 1.f;
      }
      const float sl = wave_sum(lt), sm = wave_sum(mt);
      if (lane == 0) {
        a.row_loss[2 * b] = sl;
        a.row_loss[2 * b + 1] = sm;
      }
    }
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      // batch-global surprise: sum of masked token losses over all rows / valid tokens
      float num = 0.f, den = 0.f;
      for (int i = lane; i < a.B * a.tok_pad; i += 64) {
        const int bb = i / a.tok_pad, t = i - bb * a.tok_pad;
        num += a.loss[i];
        if (t < a.C) den += a.mask != nullptr ? a.mask[(int64_t)bb * a.mask_rs + t] : 1.f;
      }
      num = wave_sum(num);
      den = wave_sum(den);
      if (lane == 0) *a.surprise = a.mask != nullptr ? num / fmaxf(den, 1.f) : num / den;
    }
  }
}

// NORM: instead of applying, write the tile's squared Frobenius norm to nrm (one partial per tile):
// the clip norm of a chunk longer than one token block, whose gradient tiles sum over its blocks.
template <typename T, bool NORM = false>
__global__ void __launch_bounds__(kThreads) k_apply(const ApplyArgs a) {
  constexpr int LD = lds_ld<T>();
  __shared__ __align__(16) T as[64 * LD];
  __shared__ __align__(16) T bs[64 * LD];
  __shared__ float row_scalar[3];
  __shared__ float red[4];
  const int nD = a.D / 64, nF = a.F / 64;
  const int per = nD * nF;
  const int m = blockIdx.x / per, j = blockIdx.x - m * per, b = blockIdx.y;
  const int w = threadIdx.x >> 6, wr = (w >> 1) * 32, wc = (w & 1) * 32;

  int r0, c0, ld_out;
  const T *asrc, *bsrc;
  int64_t a_ld, b_ld;
  int a_valid;
  if (m < 2) {  // W_up / W_gate tile (d, f) = K^T dU / K^T dG
    const int dt = j / nF, ft = j - dt * nF;
    r0 = dt * 64;
    c0 = ft * 64;
    ld_out = a.F;
    asrc = static_cast<const T*>(a.k) + (int64_t)b * a.k_rs + r0;
    a_ld = a.D;
    a_valid = a.C;
    bsrc = static_cast<const T*>(m == 0 ? a.du : a.dg) + (int64_t)b * a.tok_pad * a.F + c0;
    b_ld = a.F;
  } else {      // W_down tile (f, d) = H^T dZ
    const int ft = j / nD, dt = j - ft * nD;
    r0 = ft * 64;
    c0 = dt * 64;
    ld_out = a.D;
    asrc = static_cast<const T*>(a.h) + (int64_t)b * a.tok_pad * a.F + r0;
    a_ld = a.F;
    a_valid = a.tok_pad;  // rows past the chunk are zero
    bsrc = static_cast<const T*>(a.dz) + (int64_t)b * a.tok_pad * a.D + c0;
    b_ld = a.D;
  }
  // the state tile is the bulk of the traffic: issue its loads first
  const int64_t mat = (int64_t)a.D * a.F;
  const float* wsrc = a.w[m] + b * mat;
  const float* ssrc = a.s[m] + b * mat;
  const int col = c0 + wc + acc_col();
  float wv[16], sv[16];
  if constexpr (!NORM) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t off = (int64_t)(r0 + wr + acc_row(i)) * ld_out + col;
      wv[i] = wsrc[off];
      sv[i] = ssrc[off];
    }
  }
  constexpr int kUnits = ColStage<T, 64>::kUnits;
  f32x16 acc;
  zero(acc);
  // the gradient tile: K = the chunk's tokens, one block of 64 per step
  for (int tb = 0; tb < a.ntb; ++tb) {
    const int t0 = tb * 64;
    if (tb > 0) __syncthreads();  // the previous block's products are done with as / bs
    {
      ColStage<T, 64> cst;
      const bool a_part = threadIdx.x < kUnits;
      const int unit = a_part ? threadIdx.x : threadIdx.x - kUnits;
      cst.load(a_part ? asrc + (int64_t)t0 * a_ld : bsrc + (int64_t)t0 * b_ld, a_part ? a_ld : b_ld,
               a_part ? min(64, a_valid - t0) : 64, unit < kUnits ? unit : kUnits);
      cst.template store<T>(a_part ? as : bs, LD);
    }
    if (!NORM && tb == 0 && threadIdx.x >= 192) apply_row_scalars<T>(a, b, row_scalar);
    __syncthreads();
    wave_mma<T, 64>(acc, as + wr * LD, LD, bs + wc * LD, LD);
  }
  if constexpr (NORM) {
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) sq += acc[i] * acc[i];
    const float total = block_sum(sq, red);
    if (threadIdx.x == 0) a.nrm[(int64_t)b * a.n_norm + blockIdx.x] = total;
    return;
  }

  const float clip = row_scalar[0], decay = row_scalar[1];
  const bool active = row_scalar[2] != 0.f;
  float* wdst = a.w_out[m] + b * mat;
  float* sdst = a.s_out[m] + b * mat;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t off = (int64_t)(r0 + wr + acc_row(i)) * ld_out + col;
    float s_new, w_new;
    {
#pragma clang fp contract(off)
      const float step = acc[i] * clip;
      s_new = a.beta * sv[i] - step;
      w_new = decay * wv[i] + s_new;
    }
    wdst[off] = active ? w_new : wv[i];
    sdst[off] = active ? s_new : sv[i];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int pick_nsplit(int64_t blocks_without_split, int64_t nF) {
  int64_t s = (512 + blocks_without_split - 1) / blocks_without_split;
  if (s < 1) s = 1;
  if (s > nF) s = nF;
  return (int)s;
}

static size_t act_bytes(int32_t dtype) { return dtype == UTTT_DTYPE_BF16 ? 2 : 4; }

struct UpdateLayout {
  size_t u, g, h0, h1, zp, dz, du, dg, loss, nrm, total;
  int nsplit, ntb, tok_pad, n_norm;
};

// Workspace of one update of chunks of up to `tokens` tokens: the activations of ntb blocks of 64
// tokens; with more than one block, one squared-norm partial per gradient tile (the norm of a
// tile sums over every block) instead of one per F tile.
static UpdateLayout update_layout(int64_t B, int64_t tokens, int64_t D, int64_t F, int32_t dtype) {
  UpdateLayout L;
  const size_t e = act_bytes(dtype);
  L.ntb = (int)std::max<int64_t>(1, (tokens + 63) / 64);
  L.tok_pad = 64 * L.ntb;
  L.n_norm = L.ntb > 1 ? (int)(3 * (D / 64) * (F / 64)) : (int)(F / 64);
  const size_t TP = (size_t)L.tok_pad;
  L.nsplit = pick_nsplit((D / 64) * B * 2 * L.ntb, F / 64);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t at = off; off += align_up(bytes); return at; };
  L.u = take(sizeof(float) * B * TP * F);
  L.g = take(sizeof(float) * B * TP * F);
  L.h0 = take(e * B * TP * F);
  L.h1 = take(e * B * TP * F);
  L.zp = take(sizeof(float) * 2 * L.nsplit * B * TP * D);
  L.dz = take(e * B * TP * D);
  L.du = take(e * B * TP * F);
  L.dg = take(e * B * TP * F);
  L.loss = take(sizeof(float) * B * TP);
  L.nrm = take(sizeof(float) * B * L.n_norm);
  L.total = off;
  return L;
}

template <typename T>
static void launch_update(const uttt_chunk_update_args& a, char* ws, const UpdateLayout& L, hipStream_t st,
                          int first_phase, int last_phase) {
  const int B = (int)a.batch, C = (int)a.tokens, D = (int)a.d_model, F = (int)a.d_ff;
  const int ntb = L.ntb, TP = L.tok_pad;
  FwdArgs f{};
  f.B = B; f.D = D; f.F = F; f.ntok = C; f.ntb = ntb; f.tok_pad = TP; f.nsplit = L.nsplit;
  f.x[0] = a.k; f.x_rs[0] = a.k_row_stride;
  f.x[1] = a.q; f.x_rs[1] = a.q_row_stride;
  f.wu[0] = a.w_up; f.wg[0] = a.w_gate; f.wd[0] = a.w_down; f.w_rs[0] = (int64_t)D * F;
  f.wu[1] = a.r_up; f.wg[1] = a.r_gate; f.wd[1] = a.r_down; f.w_rs[1] = a.r_row_stride;
  f.u_store = reinterpret_cast<float*>(ws + L.u);
  f.g_store = reinterpret_cast<float*>(ws + L.g);
  f.h[0] = ws + L.h0;
  f.h[1] = ws + L.h1;
  f.zp = reinterpret_cast<float*>(ws + L.zp);
  const dim3 blk(kThreads);
  auto want = [&](int phase) { return first_phase <= phase && phase <= last_phase; };

  if (want(0)) hipLaunchKernelGGL((k_up_gate<T, float>), dim3(F / 64, B, 2 * ntb), blk, 0, st, f);
  if (want(1)) hipLaunchKernelGGL((k_down_partial<T, float>), dim3(D / 64, L.nsplit, 2 * ntb * B), blk, 0, st, f);

  LnGradArgs g{};
  g.B = B; g.C = C; g.D = D; g.nsplit = L.nsplit; g.tok_pad = TP; g.normalize = a.normalize_by_dim;
  g.eps = a.eps; g.zp = f.zp;
  g.k = a.k; g.k_rs = a.k_row_stride; g.v = a.v; g.v_rs = a.v_row_stride;
  g.eta = a.eta; g.eta_rs = a.eta_row_stride; g.mask = a.token_mask; g.mask_rs = a.mask_row_stride;
  g.ln_w = a.ln_weight; g.ln_b = a.ln_bias;
  g.dz = ws + L.dz; g.loss = reinterpret_cast<float*>(ws + L.loss);
  LnOutArgs o{};
  o.B = B; o.ntok = C; o.D = D; o.nsplit = L.nsplit; o.tok_pad = TP; o.eps = a.eps;
  o.zp = f.zp + (size_t)L.nsplit * B * TP * D;
  o.x = a.q; o.x_rs = a.q_row_stride; o.ln_w = a.ln_weight; o.ln_b = a.ln_bias;
  o.out = a.out; o.out_rs = a.out_row_stride;
  if (want(2)) {
    launch_ln_grad<T>(dim3(TP, B), st, g);
    launch_ln_readout<T>(dim3(C, B), st, o);
  }

  BwdArgs bw{};
  bw.B = B; bw.C = C; bw.D = D; bw.F = F; bw.ntb = ntb; bw.tok_pad = TP;
  bw.k = a.k; bw.k_rs = a.k_row_stride; bw.wd = a.w_down; bw.w_rs = (int64_t)D * F;
  bw.u_store = f.u_store; bw.g_store = f.g_store; bw.h = f.h[0]; bw.dz = g.dz;
  bw.du = ws + L.du; bw.dg = ws + L.dg; bw.nrm = reinterpret_cast<float*>(ws + L.nrm);
  ApplyArgs ap{};
  ap.B = B; ap.C = C; ap.D = D; ap.F = F; ap.ntb = ntb; ap.tok_pad = TP; ap.n_norm = L.n_norm;
  ap.beta = a.momentum_beta; ap.max_norm = a.max_inner_grad_norm;
  ap.k = a.k; ap.k_rs = a.k_row_stride; ap.alpha = a.alpha; ap.alpha_rs = a.alpha_row_stride;
  ap.mask = a.token_mask; ap.mask_rs = a.mask_row_stride;
  ap.h = f.h[0]; ap.dz = g.dz; ap.du = bw.du; ap.dg = bw.dg; ap.nrm = bw.nrm; ap.loss = g.loss;
  ap.w[0] = a.w_up; ap.w[1] = a.w_gate; ap.w[2] = a.w_down;
  ap.s[0] = a.s_up; ap.s[1] = a.s_gate; ap.s[2] = a.s_down;
  ap.w_out[0] = a.w_up_out; ap.w_out[1] = a.w_gate_out; ap.w_out[2] = a.w_down_out;
  ap.s_out[0] = a.s_up_out; ap.s_out[1] = a.s_gate_out; ap.s_out[2] = a.s_down_out;
  ap.surprise = a.surprise;
  ap.row_loss = a.row_loss;
  ap.min_row_surprise = a.min_row_surprise;
  const dim3 tiles(3 * (D / 64) * (F / 64), B);
  if (want(3)) {
    hipLaunchKernelGGL(k_backward<T>, dim3(F / 64, B, ntb), blk, 0, st, bw);
    // a chunk of several token blocks: each gradient tile's squared norm over the whole chunk
    if (ntb > 1) hipLaunchKernelGGL((k_apply<T, true>), tiles, blk, 0, st, ap);
  }
  if (want(4)) hipLaunchKernelGGL((k_apply<T, false>), tiles, blk, 0, st, ap);
}

void launch_saved_readout(int B, int ntok, int D, int F, int nsplit, const float* h, const float* w_down,
                          int64_t wd_rs, float* zp, const float* x, int64_t x_rs, const float* ln_w,
                          const float* ln_b, float eps, float* out, int64_t out_rs, hipStream_t st) {
  FwdArgs f{};
  f.B = B; f.D = D; f.F = F; f.ntok = ntok; f.ntb = 1; f.tok_pad = 64; f.nsplit = nsplit;
  f.wd[0] = w_down; f.w_rs[0] = wd_rs;
  f.h[0] = const_cast<float*>(h);
  f.zp = zp;
  hipLaunchKernelGGL((k_down_partial<float, float>), dim3(D / 64, nsplit, B), dim3(kThreads), 0, st, f);
  LnOutArgs o{};
  o.B = B; o.ntok = ntok; o.D = D; o.nsplit = nsplit; o.tok_pad = 64; o.eps = eps;
  o.zp = zp;
  o.x = x; o.x_rs = x_rs; o.ln_w = ln_w; o.ln_b = ln_b;
  o.out = out; o.out_rs = out_rs;
  launch_ln_readout<float>(dim3(ntok, B), st, o);
}

// One token per row (decode), bf16 activations: a streaming GEMV.  One workgroup per (row, block
// of gemv_fb(F) F columns): u and g over all of d (threads split d, partial sums meet in LDS), h
// rounded to bf16 as the matrix path rounds it, then this block's Z partial over all of D from
// the block's W_down rows; k_ln_readout sums the blocks.  Every weight row is read as 16-byte
// (bf16) or 32-byte (fp32) pieces by consecutive threads; fp32 masters are rounded to the bf16
// operands the matrix path uses, so both weight types give the same readout.
__host__ __device__ inline int gemv_fb(int64_t F) { return F % 256 == 0 ? 256 : (F % 128 == 0 ? 128 : 64); }
constexpr int kGemvRowsBf16 = 8;

// raw 8-column pieces of a weight row: bf16 kept packed until used (so that many rows fit in
// flight), fp32 masters as two 16-byte halves
template <typename WT> struct Piece8;
template <> struct Piece8<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ float get(int e) const { return to_f32(v[e]); }
};
template <> struct Piece8<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float get(int e) const { return to_f32(from_f32<bf16>(e < 4 ? lo[e] : hi[e - 4])); }
};

// rows of each matrix in flight per thread: 8 packed bf16 pieces, 4 fp32 pairs
template <typename WT> constexpr int gemv_rows() { return sizeof(WT) == 2 ? kGemvRowsBf16 : 4; }

template <int FB, typename WT, int CW>
__global__ void __launch_bounds__(kThreads) k_readout_gemv(const FwdArgs a) {
  constexpr int TF = FB / 8;         // threads across one weight row piece (8 columns each)
  constexpr int DG = kThreads / TF;  // row groups of the u / g loop
  constexpr int RB = gemv_rows<WT>();
  constexpr int NP = CW / 8;         // 8-column pieces per thread in the W_down loop
  __shared__ float xs[2048];         // the token's row (D <= 2048 checked by the caller)
  __shared__ float red[2][DG][FB];
  __shared__ float hs[FB];
  __shared__ float sred[4];
  __shared__ int last;
  const int fb = blockIdx.x, b = blockIdx.y, f0 = fb * FB;
  const bf16* x = static_cast<const bf16*>(a.x[0]) + (int64_t)b * a.x_rs[0];
  stage_row<bf16>(x, a.D, static_cast<const bf16*>(a.xn_w), a.xn_eps, xs, sred);
  __syncthreads();
  const WT* gu = static_cast<const WT*>(a.wu[0]) + (int64_t)b * a.w_rs[0] + f0;
  const WT* gg = static_cast<const WT*>(a.wg[0]) + (int64_t)b * a.w_rs[0] + f0;
  const int col = (threadIdx.x % TF) * 8, grp = threadIdx.x / TF;
  const int d_per = (a.D + DG - 1) / DG, d_begin = grp * d_per, d_end = min(a.D, d_begin + d_per);
  float au[8], ag[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) au[e] = ag[e] = 0.f;
  // the i-th row of this thread's range: ascending, or descending with a.rev
  const int d_n = d_end - d_begin, d_first = a.rev ? d_end - 1 : d_begin, d_step = a.rev ? -1 : 1;
  int i = 0;
  for (; i + RB <= d_n; i += RB) {  // RB rows of both matrices in flight
    Piece8<WT> pu[RB], pg[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int d = d_first + (i + r) * d_step;
      pu[r].load(gu + (int64_t)d * a.F + col);
      pg[r].load(gg + (int64_t)d * a.F + col);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first use
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const float xv = xs[d_first + (i + r) * d_step];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        au[e] += xv * pu[r].get(e);
        ag[e] += xv * pg[r].get(e);
      }
    }
  }
  for (; i < d_n; ++i) {
    const int d = d_first + i * d_step;
    Piece8<WT> pu, pg;
    pu.load(gu + (int64_t)d * a.F + col);
    pg.load(gg + (int64_t)d * a.F + col);
    const float xv = xs[d];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      au[e] += xv * pu.get(e);
      ag[e] += xv * pg.get(e);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][grp][col + e] = au[e];
    red[1][grp][col + e] = ag[e];
  }
  __syncthreads();
  if (threadIdx.x < FB) {
    float u = 0.f, g = 0.f;
#pragma unroll
    for (int q = 0; q < DG; ++q) {
      u += red[0][q][threadIdx.x];
      g += red[1][q][threadIdx.x];
    }
    hs[threadIdx.x] = to_f32(from_f32<bf16>((g * sigmoidf_acc(g)) * u));
  }
  __syncthreads();
  // Z partial of this block: thread (column group c, F part p) takes CW columns of D and a share
  // of the block's FB rows
  const WT* gd = static_cast<const WT*>(a.wd[0]) + (int64_t)b * a.w_rs[0] + (int64_t)f0 * a.D;
  const int ncol = a.D / CW, nparts = kThreads / ncol;
  float* zp = a.zp + ((int64_t)fb * a.B + b) * a.tok_pad * a.D;
  const int c = threadIdx.x % ncol, p = threadIdx.x / ncol;
  constexpr int RD = RB / NP > 0 ? RB / NP : 1;  // W_down rows in flight (same loads in flight)
  float az[CW];
#pragma unroll
  for (int e = 0; e < CW; ++e) az[e] = 0.f;
  if (p < nparts) {
    const int f_per = FB / nparts + (FB % nparts != 0), fb0 = p * f_per, fb1 = min(FB, fb0 + f_per);
    const int f_n = fb1 - fb0, f_first = a.rev ? fb1 - 1 : fb0, f_step = a.rev ? -1 : 1;
    int j = 0;
    for (; j + RD <= f_n; j += RD) {
      Piece8<WT> pw[RD][NP];
#pragma unroll
      for (int r = 0; r < RD; ++r)
#pragma unroll
        for (int q = 0; q < NP; ++q)
          pw[r][q].load(gd + (int64_t)(f_first + (j + r) * f_step) * a.D + c * CW + q * 8);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < RD; ++r) {
        const float hv = hs[f_first + (j + r) * f_step];
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
          for (int e = 0; e < 8; ++e) az[q * 8 + e] += hv * pw[r][q].get(e);
      }
    }
    for (; j < f_n; ++j) {
      const int f = f_first + j * f_step;
      const float hv = hs[f];
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        Piece8<WT> pw;
        pw.load(gd + (int64_t)f * a.D + c * CW + q * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) az[q * 8 + e] += hv * pw.get(e);
      }
    }
  }
  __syncthreads();  // red is free again: the parts' sums meet there
  float* zred = &red[0][0][0];  // nparts x D floats (nparts * D <= 256 * CW <= 4096 <= 2 * DG * FB)
  if (p < nparts) {
#pragma unroll
    for (int e = 0; e < CW; ++e) zred[p * a.D + c * CW + e] = az[e];
  }
  __syncthreads();
  if (a.counters == nullptr) {  // k_ln_readout follows
    for (int dd = threadIdx.x; dd < a.D; dd += kThreads) {
      float v = 0.f;
      for (int q = 0; q < nparts; ++q) v += zred[q * a.D + dd];
      zp[dd] = v;
    }
    return;
  }
  // The row's last block to finish sums the row's partials.  The partials are written with
  // device-coherent stores (through this CU's L2), every thread waits until its stores are
  // done, and only then is the row's count raised; the last block reads the partials with
  // device-coherent loads.  So no cache write-back or invalidate is needed.  The last block
  // returns the count to zero for the next call.
  for (int dd = threadIdx.x; dd < a.D; dd += kThreads) {
    float v = 0.f;
    for (int q = 0; q < nparts; ++q) v += zred[q * a.D + dd];
    __hip_atomic_store(zp + dd, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(a.counters + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  bf16* o = static_cast<bf16*>(a.out) + (int64_t)b * a.out_rs;
  const float* z0 = a.zp + (int64_t)b * a.tok_pad * a.D;
  const int64_t sp_stride = (int64_t)a.B * a.tok_pad * a.D;
  if (a.D <= 4 * kThreads)
    ln_readout_row<bf16, 4, true>(z0, sp_stride, gridDim.x, a.D, a.ln_eps, a.ln_w, a.ln_b, xs, o, sred);
  else
    ln_readout_row<bf16, 8, true>(z0, sp_stride, gridDim.x, a.D, a.ln_eps, a.ln_w, a.ln_b, xs, o, sred);
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct ReadoutLayout {
  size_t h, zp, total;
  int nsplit, ntb;
};

static ReadoutLayout readout_layout(int64_t B, int64_t T, int64_t D, int64_t F, int32_t dtype) {
  ReadoutLayout L;
  L.ntb = (int)((T + 63) / 64);
  L.nsplit = pick_nsplit((D / 64) * B * L.ntb, F / 64);
  // one token: room for the GEMV's F-block partials too
  const int64_t zsplits = T == 1 ? std::max<int64_t>(L.nsplit, F / gemv_fb(F)) : L.nsplit;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t at = off; off += align_up(bytes); return at; };
  L.h = take(act_bytes(dtype) * B * L.ntb * 64 * F);
  L.zp = take(sizeof(float) * zsplits * B * L.ntb * 64 * D);
  L.total = off;
  return L;
}

template <typename WT, int CW>
static void launch_gemv(int fbw, dim3 grid, hipStream_t st, const FwdArgs& f) {
  if (fbw == 256)
    hipLaunchKernelGGL((k_readout_gemv<256, WT, CW>), grid, dim3(kThreads), 0, st, f);
  else if (fbw == 128)
    hipLaunchKernelGGL((k_readout_gemv<128, WT, CW>), grid, dim3(kThreads), 0, st, f);
  else
    hipLaunchKernelGGL((k_readout_gemv<64, WT, CW>), grid, dim3(kThreads), 0, st, f);
}

template <typename T, typename WT>
static void launch_readout(const uttt_readout_args& a, char* ws, const ReadoutLayout& L, hipStream_t st) {
  const int B = (int)a.batch, D = (int)a.d_model, F = (int)a.d_ff;
  FwdArgs f{};
  f.B = B; f.D = D; f.F = F; f.ntok = (int)a.tokens; f.ntb = L.ntb; f.tok_pad = L.ntb * 64; f.nsplit = L.nsplit;
  f.x[0] = a.x; f.x_rs[0] = a.x_row_stride;
  f.wu[0] = a.w_up; f.wg[0] = a.w_gate; f.wd[0] = a.w_down; f.w_rs[0] = a.w_row_stride;
  f.u_store = nullptr; f.g_store = nullptr;
  f.h[0] = ws + L.h;
  f.zp = reinterpret_cast<float*>(ws + L.zp);
  f.kx = a.keys; f.kx_rs = a.keys_row_stride; f.ku = a.key_up_out; f.kg = a.key_gate_out;
  f.xn_w = a.x_norm_weight; f.xn_eps = a.x_norm_eps; f.counters = a.row_counters;
  f.ln_eps = a.eps; f.ln_w = a.ln_weight; f.ln_b = a.ln_bias; f.out = a.out; f.out_rs = a.out_row_stride;
  f.rev = a.sweep_reverse != 0;
  const dim3 blk(kThreads);
  if constexpr (sizeof(T) == 2) {
    if (a.tokens == 1 && a.keys == nullptr && D <= 2048 && D % 8 == 0) {  // decode: streaming GEMV
      const int fbw = gemv_fb(F);
      if (D % 16 == 0)
        launch_gemv<WT, 16>(fbw, dim3(F / fbw, B), st, f);
      else
        launch_gemv<WT, 8>(fbw, dim3(F / fbw, B), st, f);
      if (a.row_counters != nullptr) return;  // the LN ran in each row's last block
      LnOutArgs o{};
      o.B = B; o.ntok = 1; o.D = D; o.nsplit = F / fbw; o.tok_pad = f.tok_pad; o.eps = a.eps;
      o.zp = f.zp; o.x = a.x; o.x_rs = a.x_row_stride; o.ln_w = a.ln_weight; o.ln_b = a.ln_bias;
      o.out = a.out; o.out_rs = a.out_row_stride;
      o.xn_w = a.x_norm_weight; o.xn_eps = a.x_norm_eps;
      launch_ln_readout<T>(dim3(1, B), st, o);
      return;
    }
  }
  // bf16 weights: K tiles of 128 halve the staged steps of these latency-bound loops where the
  // shape allows.  The key block (when asked for) is one more z block: it runs beside the token
  // blocks of the same F tile and row, on the same XCD, so its weight tiles come from that L2.
  constexpr bool wide = sizeof(WT) == 2;
  const dim3 ug_grid(F / 64, B, L.ntb + (a.keys != nullptr ? 1 : 0));
  if constexpr (sizeof(T) == 2 && sizeof(WT) == 2) {
    if (L.ntb == 1) {  // one token block: the LDS-ring kernel
      if (F % 128 == 0) {
        if (a.keys != nullptr)
          hipLaunchKernelGGL((k_up_gate_lds<true, 2>), dim3(row_tile_blocks(B, F / 128)), dim3(512), 0, st, f);
        else
          hipLaunchKernelGGL((k_up_gate_lds<false, 2>), dim3(row_tile_blocks(B, F / 128)), dim3(256), 0, st, f);
      } else if (a.keys != nullptr) {
        hipLaunchKernelGGL((k_up_gate_lds<true, 1>), dim3(row_tile_blocks(B, F / 64)), dim3(512), 0, st, f);
      } else {
        hipLaunchKernelGGL((k_up_gate_lds<false, 1>), dim3(row_tile_blocks(B, F / 64)), dim3(256), 0, st, f);
      }
    } else if (D % 128 == 0) {
      hipLaunchKernelGGL((k_up_gate<T, WT, 128>), ug_grid, blk, 0, st, f);
    } else {
      hipLaunchKernelGGL((k_up_gate<T, WT>), ug_grid, blk, 0, st, f);
    }
  } else if (wide && D % 128 == 0) {
    hipLaunchKernelGGL((k_up_gate<T, WT, wide ? 128 : KT>), ug_grid, blk, 0, st, f);
  } else {
    hipLaunchKernelGGL((k_up_gate<T, WT>), ug_grid, blk, 0, st, f);
  }
  const dim3 dp_grid(D / 64, L.nsplit, L.ntb * B);
  if constexpr (sizeof(T) == 2 && sizeof(WT) == 2)
    hipLaunchKernelGGL(k_down_partial_lds, dim3(row_tile_blocks(L.ntb * B, (D / 64) * L.nsplit)), blk, 0, st, f,
                       F % 128 == 0 ? 128 : KT);
  else if (wide && F % 128 == 0)
    hipLaunchKernelGGL((k_down_partial<T, WT, wide ? 128 : KT>), dp_grid, blk, 0, st, f);
  else
    hipLaunchKernelGGL((k_down_partial<T, WT>), dp_grid, blk, 0, st, f);
  LnOutArgs o{};
  o.B = B; o.ntok = (int)a.tokens; o.D = D; o.nsplit = L.nsplit; o.tok_pad = f.tok_pad; o.eps = a.eps;
  o.zp = f.zp; o.x = a.x; o.x_rs = a.x_row_stride; o.ln_w = a.ln_weight; o.ln_b = a.ln_bias;
  o.out = a.out; o.out_rs = a.out_row_stride;
  launch_ln_readout<T>(dim3(f.tok_pad, B), st, o);
}

static int check_dims(int64_t B, int64_t D, int64_t F, int32_t dtype) {
  UTTT_REQUIRE(B >= 1, "batch must be >= 1 (got %lld)", (long long)B);
  UTTT_REQUIRE(D >= 64 && D % 64 == 0 && D <= 4096, "d_model must be a multiple of 64 in [64, 4096] (got %lld)", (long long)D);
  UTTT_REQUIRE(F >= 64 && F % 64 == 0, "d_ff must be a positive multiple of 64 (got %lld)", (long long)F);
  UTTT_REQUIRE(dtype == UTTT_DTYPE_F32 || dtype == UTTT_DTYPE_BF16, "act_dtype must be F32 or BF16 (got %d)", dtype);
  UTTT_REQUIRE(B <= 65535, "batch must be <= 65535");
  return UTTT_OK;
}

}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_chunk_update_workspace(int64_t batch, int64_t d_model, int64_t d_ff, int32_t act_dtype) {
  if (check_dims(batch, d_model, d_ff, act_dtype) != UTTT_OK) return 0;
  return update_layout(batch, 64, d_model, d_ff, act_dtype).total;
}

extern "C" size_t uttt_chunk_update_workspace_tokens(int64_t batch, int64_t tokens, int64_t d_model, int64_t d_ff,
                                                     int32_t act_dtype) {
  if (check_dims(batch, d_model, d_ff, act_dtype) != UTTT_OK || tokens < 1 || tokens > UTTT_MAX_UPDATE_TOKENS)
    return 0;
  return update_layout(batch, tokens, d_model, d_ff, act_dtype).total;
}

static int validate_update(const uttt_chunk_update_args* a, void* workspace, size_t workspace_bytes,
                           UpdateLayout& L) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  int rc = check_dims(a->batch, a->d_model, a->d_ff, a->act_dtype);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->tokens >= 1 && a->tokens <= UTTT_MAX_UPDATE_TOKENS, "tokens per chunk must be in [1, %d] (got %lld)",
               UTTT_MAX_UPDATE_TOKENS, (long long)a->tokens);
  UTTT_REQUIRE(a->q && a->k && a->v && a->eta && a->alpha, "q/k/v/eta/alpha must be non-NULL");
  UTTT_REQUIRE(a->w_up && a->w_gate && a->w_down && a->s_up && a->s_gate && a->s_down, "state pointers must be non-NULL");
  UTTT_REQUIRE(a->r_up && a->r_gate && a->r_down, "read-state pointers must be non-NULL");
  UTTT_REQUIRE(a->ln_weight && a->ln_bias, "ln_weight/ln_bias must be non-NULL");
  UTTT_REQUIRE(a->w_up_out && a->w_gate_out && a->w_down_out && a->s_up_out && a->s_gate_out && a->s_down_out,
               "output state pointers must be non-NULL");
  UTTT_REQUIRE(a->out && a->surprise, "out/surprise must be non-NULL");
  UTTT_REQUIRE(a->r_row_stride == 0 || a->r_row_stride == a->d_model * a->d_ff,
               "read-state row stride must be 0 (shared) or d_model*d_ff");
  const int64_t vec = a->act_dtype == UTTT_DTYPE_BF16 ? 8 : 4;
  UTTT_REQUIRE(aligned16(a->q) && aligned16(a->k) && aligned16(a->v) && aligned16(a->w_up) && aligned16(a->w_gate) &&
               aligned16(a->w_down) && aligned16(a->s_up) && aligned16(a->s_gate) && aligned16(a->s_down) &&
               aligned16(a->r_up) && aligned16(a->r_gate) && aligned16(a->r_down),
               "activation and state pointers must be 16-byte aligned");
  UTTT_REQUIRE(a->q_row_stride % vec == 0 && a->k_row_stride % vec == 0 && a->v_row_stride % vec == 0,
               "q/k/v row strides must be multiples of 16 bytes");
  L = update_layout(a->batch, a->tokens, a->d_model, a->d_ff, a->act_dtype);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
               "workspace too small: need %zu bytes, got %zu", L.total, workspace_bytes);
  return UTTT_OK;
}

static int run_update(const uttt_chunk_update_args* a, void* workspace, size_t workspace_bytes,
                      uttt_stream_t stream, int first_phase, int last_phase) {
  UpdateLayout L;
  const int rc = validate_update(a, workspace, workspace_bytes, L);
  if (rc != UTTT_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->act_dtype == UTTT_DTYPE_BF16)
    launch_update<bf16>(*a, static_cast<char*>(workspace), L, st, first_phase, last_phase);
  else
    launch_update<float>(*a, static_cast<char*>(workspace), L, st, first_phase, last_phase);
  return launch_status("uttt_chunk_update");
}

extern "C" int uttt_chunk_update(const uttt_chunk_update_args* a, void* workspace, size_t workspace_bytes,
                                 uttt_stream_t stream) {
  return run_update(a, workspace, workspace_bytes, stream, 0, UTTT_UPDATE_PHASES - 1);
}

extern "C" int uttt_chunk_update_phase(const uttt_chunk_update_args* a, void* workspace, size_t workspace_bytes,
                                       int32_t phase, uttt_stream_t stream) {
  UTTT_REQUIRE(phase >= 0 && phase < UTTT_UPDATE_PHASES, "phase must be in [0, %d)", UTTT_UPDATE_PHASES);
  return run_update(a, workspace, workspace_bytes, stream, phase, phase);
}

// ---------------------------------------------------------------------------------------------
// The same update without a caller workspace, for callers that cannot allocate device memory.
// Its workspace is `scratch`, a device-resident array of the library (each GPU holds its own copy
// while the process lives).  In host code the array's name is only a stand-in: its device address
// comes from hipGetSymbolAddress, fetched once per device with that device current and kept in
// scratch_device_ptr.  Nothing in the update's workspace needs to start at zero (every phase writes
// what a later phase reads), so the array is not cleared; calls on one GPU share it and must not
// overlap.
// ---------------------------------------------------------------------------------------------
namespace {

static_assert(UTTT_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size must keep 256-byte alignment");
__device__ __align__(256) unsigned char scratch[UTTT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_device_ptr[kMaxDevices] = {};

// The device address of `scratch` on the calling thread's current device, which must be the
// stream's device.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(UTTT_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return fail(UTTT_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    UTTT_REQUIRE(sdev == dev, "the stream's device (%d) must be the current device (%d)", sdev, dev);
  }
  UTTT_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_device_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(UTTT_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    scratch_device_ptr[dev] = p;
  }
  *out = scratch_device_ptr[dev];
  return UTTT_OK;
}

}  // namespace

extern "C" int uttt_chunk_update_noalloc(const uttt_chunk_update_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  const int rc = check_dims(a->batch, a->d_model, a->d_ff, a->act_dtype);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->tokens >= 1 && a->tokens <= UTTT_MAX_UPDATE_TOKENS, "tokens per chunk must be in [1, %d] (got %lld)",
               UTTT_MAX_UPDATE_TOKENS, (long long)a->tokens);
  const size_t need = update_layout(a->batch, a->tokens, a->d_model, a->d_ff, a->act_dtype).total;
  UTTT_REQUIRE(need <= UTTT_NOALLOC_SCRATCH_BYTES,
               "uttt_chunk_update_noalloc: this shape needs %zu bytes of workspace, more than the %llu-byte "
               "device-resident scratch; use uttt_chunk_update with a workspace",
               need, (unsigned long long)UTTT_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int src = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (src != UTTT_OK) return src;
  return run_update(a, ws, UTTT_NOALLOC_SCRATCH_BYTES, stream, 0, UTTT_UPDATE_PHASES - 1);
}

extern "C" size_t uttt_readout_workspace(int64_t batch, int64_t tokens, int64_t d_model, int64_t d_ff, int32_t act_dtype) {
  if (check_dims(batch, d_model, d_ff, act_dtype) != UTTT_OK || tokens < 1) return 0;
  return readout_layout(batch, tokens, d_model, d_ff, act_dtype).total;
}

extern "C" int uttt_swiglu_readout(const uttt_readout_args* a, void* workspace, size_t workspace_bytes,
                                   uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  int rc = check_dims(a->batch, a->d_model, a->d_ff, a->act_dtype);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->tokens >= 1 && a->tokens <= (1 << 20), "tokens must be in [1, 2^20]");
  UTTT_REQUIRE(a->x && a->out && a->w_up && a->w_gate && a->w_down && a->ln_weight && a->ln_bias,
               "pointers must be non-NULL");
  UTTT_REQUIRE(a->w_row_stride == 0 || a->w_row_stride == a->d_model * a->d_ff,
               "weight row stride must be 0 (shared) or d_model*d_ff");
  UTTT_REQUIRE(aligned16(a->x) && aligned16(a->w_up) && aligned16(a->w_gate) && aligned16(a->w_down),
               "x and weight pointers must be 16-byte aligned");
  UTTT_REQUIRE(a->x_row_stride % (a->act_dtype == UTTT_DTYPE_BF16 ? 8 : 4) == 0,
               "x row stride must be a multiple of 16 bytes");
  const ReadoutLayout L = readout_layout(a->batch, a->tokens, a->d_model, a->d_ff, a->act_dtype);
  UTTT_REQUIRE((int64_t)L.ntb * a->batch <= 65535, "batch * ceil(tokens / 64) must be <= 65535");
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
               "workspace too small: need %zu bytes, got %zu", L.total, workspace_bytes);
  UTTT_REQUIRE(a->w_dtype == UTTT_DTYPE_F32 || (a->w_dtype == UTTT_DTYPE_BF16 && a->act_dtype == UTTT_DTYPE_BF16),
               "w_dtype must be F32, or BF16 with BF16 activations");
  if (a->keys != nullptr) {
    UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_BF16, "key products need bf16 activations");
    UTTT_REQUIRE(a->tokens <= 64, "key products need tokens <= 64 (got %lld)", (long long)a->tokens);
    UTTT_REQUIRE(a->key_up_out != nullptr && a->key_gate_out != nullptr, "key product outputs must be non-NULL");
    UTTT_REQUIRE(aligned16(a->keys) && a->keys_row_stride % 8 == 0,
                 "keys must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
  }
  if (a->x_norm_weight != nullptr || a->row_counters != nullptr) {
    UTTT_REQUIRE(a->tokens == 1 && a->act_dtype == UTTT_DTYPE_BF16 && a->keys == nullptr && a->d_model <= 2048,
                 "x_norm_weight and row_counters need one bf16 token per row, no keys and d_model <= 2048");
    UTTT_REQUIRE(a->x_norm_weight == nullptr || a->x_norm_eps > 0.f, "x_norm_eps must be > 0");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (a->act_dtype == UTTT_DTYPE_BF16) {
    if (a->w_dtype == UTTT_DTYPE_BF16)
      launch_readout<bf16, bf16>(*a, ws, L, st);
    else
      launch_readout<bf16, float>(*a, ws, L, st);
  } else {
    launch_readout<float, float>(*a, ws, L, st);
  }
  return launch_status("uttt_swiglu_readout");
}
