// Slow-weight products of the chunk-first forward pass, out = x W^T (+ residual), written for
// gfx950 (MI355X): bf16 operands, fp32 accumulation, x (m, k) and W (n, k) row-major, so both
// operands are k-contiguous and reach the MFMA without transposes.  Replaces the F.linear /
// h + linear(x) calls of the per-chunk forward pass (the packed QKV projection and the packed
// uTTT projections, reference model/uttt_layer.py:1058-1081 and :1193-1231, and the residual
// projections of uTTTBlock.forward, :1528-1555) at the shapes the chunk-first schedule runs them:
// m = rows x 64 tokens (256 at config 3), k = d_model.
//
// At those shapes the product waits on its operand loads: every tile load misses the CU's L1
// (the operands are re-read per tile from L2, 75% L2 hits at m 256, k 2048), a CU keeps only a
// few dozen such misses in flight (measured: about 430 cycles per miss, ~20 bytes per clock per
// CU), so the time follows the largest per-CU share of the tile traffic, 2 k (MT + 64) bytes per
// tile.  The launch plan spreads that traffic over the CUs: tiles of MT x 64 (MT 128 or 64) and,
// when the tiles alone leave CUs idle, a split of the k loop over `splits` workgroups per tile,
// whose fp32 partial tiles meet in the workspace; the last workgroup of a tile to finish (a
// counter per tile) adds the others' partials to its own and writes the output.  The kernel
// times match the library GEMM's at these shapes within about 15% either way; its point is
// that a native caller can launch it without a library call's host cost.
//
// Per k step of 64, the x rows and W rows of the tile go straight from global memory into LDS
// (buffer loads with the lds bit, 64-row tiles of 8 KB with their 16-byte pieces swizzled per
// row) through a ring of SLOTS steps.  Eight waves, two per SIMD, so that one wave's loads and
// LDS waits overlap the other's MFMAs (v_mfma_f32_32x32x16_bf16).  MT 128: wave w owns the
// 32 x 32 block (32 (w & 3), 32 (w >> 2)); MT 64: waves w and w + 4 own the block
// (32 ((w & 3) >> 1), 32 (w & 1)) and split each step's four k pieces two and two, summed through
// LDS at the end.  Rows past m and columns past n read as zeros (buffer ranges) and are not
// stored.
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {
namespace {

constexpr int kLinThreads = 512;
constexpr int kLinNT = 64;

struct LinArgs {
  int m, n, k;
  const bf16* x;
  int64_t xs;
  const bf16* w;
  int64_t ws;
  const bf16* r;  // residual (may alias out) or null
  int64_t rs;
  bf16* out;
  int64_t os;
  int mtiles, splits;
  unsigned* counters;  // one per tile, zero between launches
  float* part;         // splits fp32 partial tiles per tile
};

// Workgroup -> (tile, split): the hardware deals consecutive workgroups round-robin to the 8
// XCDs; renumber so that each XCD takes a consecutive run of ids, so that the splits of a tile
// and the m tiles of one W tile meet in one XCD's L2.
__device__ __forceinline__ int xcd_id(int L, int G) {
  const int x = L % 8, per = G / 8, rem = G % 8;
  return x * per + min(x, rem) + L / 8;
}

template <int MT>
constexpr int lin_acc_waves() {
  return MT == 128 ? 8 : 4;  // waves that hold a distinct block after the in-workgroup k sum
}

template <int MT, int SLOTS>
__global__ void __launch_bounds__(kLinThreads, 1) k_linear(const LinArgs a) {
  constexpr int NT = kLinNT;
  constexpr int XT = MT / 64;           // 64-row x tiles per step
  constexpr int STEP = (XT + 1) * 8192;  // bytes per k step: x tiles, then the W tile
  constexpr int PER = XT + 1;            // row-group loads per wave and step (8 (XT + 1) / 8 waves)
  constexpr int KP = MT == 128 ? 4 : 2;  // k pieces of 16 per step and wave
  constexpr int NWA = lin_acc_waves<MT>();
  static_assert(SLOTS >= 2 && SLOTS * STEP >= NWA * 16 * 64 * 4, "ring too small");
  __shared__ __align__(1024) char ring[SLOTS * STEP];
  __shared__ int last;
  const int id = xcd_id(blockIdx.x, gridDim.x);
  const int split = id % a.splits, tile = id / a.splits;
  const int n0 = (tile / a.mtiles) * NT, m0 = (tile % a.mtiles) * MT;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int mrows = min(MT, a.m - m0), ncols = min(NT, a.n - n0);
  const int nsteps_all = a.k / 64;
  const int s_begin = split * nsteps_all / a.splits;
  const int nsteps = (split + 1) * nsteps_all / a.splits - s_begin;
  const bf16* xr = a.x + (int64_t)m0 * a.xs + (int64_t)s_begin * 64;
  const bf16* wr = a.w + (int64_t)n0 * a.ws + (int64_t)s_begin * 64;
  int voff[PER];
  const bf16* vsrc[PER];
  uint32_t vdst[PER];
  uint32_t vbytes[PER];  // buffer range: the tile's valid rows
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int g = w + 8 * i;  // row group 0 .. 8 (XT + 1) - 1: x tiles' groups, then W's
    const int t = g / 8, rg = g % 8;
    const bool is_x = t < XT;
    const int64_t ld = is_x ? a.xs : a.ws;
    voff[i] = row_src_off(rg, lane, (int)ld);
    vsrc[i] = is_x ? xr + (int64_t)t * 64 * a.xs : wr;
    vbytes[i] = (uint32_t)((is_x ? max(0, min(64, mrows - 64 * t)) : ncols) * ld * 2);
    vdst[i] = (uint32_t)(t * 8192 + rg * 1024);
  }
  const uint32_t ring0 = lds_addr(ring);
  auto issue = [&](int step) {
    const uint32_t base = ring0 + (uint32_t)((step % SLOTS) * STEP);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(vsrc[i] + step * 64, vbytes[i]);
      buffer_load_lds_raw(rs, lds_ptr(base + vdst[i]), 16, voff[i], 0, 0, 0);
    }
  };
  for (int j = 0; j < min(nsteps, SLOTS - 1); ++j) issue(j);
  const int rb = MT == 128 ? 32 * (w & 3) : 32 * ((w & 3) >> 1);
  const int cb = MT == 128 ? 32 * (w >> 2) : 32 * (w & 1);
  const int kp0 = MT == 128 ? 0 : 2 * (w >> 2);
  f32x16 acc;
  zero(acc);
  for (int step = 0; step < nsteps; ++step) {
    wait_steps<PER, SLOTS - 2>(min(nsteps - 1, step + SLOTS - 2) - step);
    __builtin_amdgcn_s_barrier();  // every wave's loads of this step landed; the oldest slot is free
    if (step + SLOTS - 1 < nsteps) issue(step + SLOTS - 1);
    const uint32_t so = ring0 + (uint32_t)((step % SLOTS) * STEP);
    const uint32_t xt = so + (uint32_t)((rb >> 6) * 8192), wt = so + (uint32_t)(XT * 8192);
    bf16x8 fa[4], fb[4];
#pragma unroll
    for (int s = 0; s < KP; ++s) {
      fa[s] = lds_read_bf16x8<0>(row_frag_addr(xt, rb & 63, lane, kp0 + s));
      fb[s] = lds_read_bf16x8<0>(row_frag_addr(wt, cb, lane, kp0 + s));
    }
    lds_wait_frags(fa, fb);
#pragma unroll
    for (int s = 0; s < KP; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s], fb[s], acc, 0, 0, 0);
  }
  float* red = reinterpret_cast<float*>(ring);  // the ring is idle after the loop
  if constexpr (MT == 64) {
    // waves 4..7 hand their half sums to waves 0..3
    __syncthreads();
    if (w >= 4) {
#pragma unroll
      for (int i = 0; i < 16; ++i) red[((w - 4) * 16 + i) * 64 + lane] = acc[i];
    }
    __syncthreads();
    if (w < 4) {
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] += red[(w * 16 + i) * 64 + lane];
    }
  }
  const bool holds = w < NWA;  // this wave holds a distinct block of the tile
  if (a.splits > 1) {
    // store this split's partial tile ([wave][i][lane]) device-coherently, then count; the
    // workgroup that completes the count adds the other splits' partials (read past its L2)
    constexpr int TILE = MT * NT;
    float* mine = a.part + ((int64_t)tile * a.splits + split) * TILE;
    if (holds) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __hip_atomic_store(mine + (w * 16 + i) * 64 + lane, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned* c = a.counters + tile;
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == (unsigned)(a.splits - 1);
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    if (holds) {
      const float* base = a.part + (int64_t)tile * a.splits * TILE + (w * 16) * 64 + lane;
      for (int s = 0; s < a.splits; ++s) {
        if (s == split) continue;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[i] = __hip_atomic_load(base + (int64_t)s * TILE + i * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] += v[i];
      }
    }
  }
  if (!holds) return;
  // out[row][col] = acc (+ residual): lane holds rows rb + acc_row(i), column cb + acc_col()
  const int col = cb + acc_col();
  if (col >= ncols) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = rb + acc_row(i);
    if (row >= mrows) continue;
    float v = acc[i];
    if (a.r != nullptr) v += to_f32(a.r[(int64_t)(m0 + row) * a.rs + n0 + col]);
    a.out[(int64_t)(m0 + row) * a.os + n0 + col] = from_f32<bf16>(v);
  }
}

constexpr int kSlots128 = 4, kSlots64 = 3;
constexpr int kMaxSplits = 8;
// the workspace starts with a fixed counter region, so that one zero-filled buffer serves every
// shape (a launch's partial tiles never overlap another shape's counters)
constexpr int64_t kMaxSplitTiles = 16384;
constexpr size_t kCounterBytes = kMaxSplitTiles * 4;

// Launch plan: the tile height and k split with the least per-CU work, counted as the k steps of
// (MT + 64) rows each workgroup streams, times the rounds of one workgroup per CU the grid takes,
// plus a fixed cost for the partial-tile handoff of a split (measured on the config-2/3 shapes:
// the handoff costs about as much as 12 MT-row tile loads).
struct LinPlan {
  int mt, splits;
  int64_t tiles;
};

LinPlan plan_linear(int64_t m, int64_t n, int64_t k, int cus) {
  LinPlan best{64, 1, ((m + 63) / 64) * ((n + kLinNT - 1) / kLinNT)};
  double best_cost = 1e300;
  const int64_t nsteps = k / 64;
  for (int mt : {128, 64}) {
    const int64_t tiles = ((m + mt - 1) / mt) * ((n + kLinNT - 1) / kLinNT);
    for (int s = 1; s <= kMaxSplits && s <= nsteps && (s == 1 || tiles <= kMaxSplitTiles); ++s) {
      const int64_t rounds = (tiles * s + cus - 1) / cus;
      const double cost =
          (double)rounds * ((double)((nsteps + s - 1) / s) * (mt + kLinNT) + (s > 1 ? 12.0 * mt : 0.0));
      if (cost < best_cost * 0.97) {
        best_cost = cost;
        best = LinPlan{mt, s, tiles};
      }
    }
  }
  return best;
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

size_t linear_workspace_bytes(const LinPlan& p) {
  if (p.splits <= 1) return 0;
  return kCounterBytes + (size_t)p.tiles * p.splits * p.mt * kLinNT * 4;
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_linear_workspace(int64_t m, int64_t n, int64_t k) {
  if (m < 1 || n < 1 || k < 64 || k % 64 != 0) return 0;
  return linear_workspace_bytes(plan_linear(m, n, k, device_cus()));
}

namespace uttt {

int linear_enqueue(const uttt_linear_args* a, hipStream_t st, int tile_rows) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(tile_rows == 0 || tile_rows == 128, "tile_rows must be 0 or 128");
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_BF16, "uttt_linear takes bf16 operands");
  UTTT_REQUIRE(a->m >= 1 && a->n >= 1 && a->k >= 64 && a->k % 64 == 0 && a->m <= (1 << 24) && a->n <= (1 << 24) &&
                   a->k <= (1 << 16),
               "shape m %lld, n %lld, k %lld: k must be a positive multiple of 64", (long long)a->m,
               (long long)a->n, (long long)a->k);
  UTTT_REQUIRE(a->x && a->w && a->out, "x, w and out must be non-NULL");
  UTTT_REQUIRE(aligned16(a->x) && aligned16(a->w) && a->x_row_stride % 8 == 0 && a->w_row_stride % 8 == 0 &&
                   a->x_row_stride >= a->k && a->w_row_stride >= a->k,
               "x and w must be 16-byte aligned with row strides of at least k, multiples of 8 elements");
  UTTT_REQUIRE(a->out_row_stride >= a->n && (a->residual == nullptr || a->residual_row_stride >= a->n),
               "out / residual row strides must be at least n");
  UTTT_REQUIRE((int64_t)64 * a->x_row_stride * 2 <= 0xffffffffLL && (int64_t)64 * a->w_row_stride * 2 <= 0xffffffffLL,
               "row strides too large");
  const LinPlan p = tile_rows == 128 ? LinPlan{128, 1, ((a->m + 127) / 128) * ((a->n + kLinNT - 1) / kLinNT)}
                                     : plan_linear(a->m, a->n, a->k, device_cus());
  UTTT_REQUIRE(p.tiles * p.splits < (1LL << 31) && (p.splits == 1 || p.tiles <= kMaxSplitTiles), "too many tiles");
  const size_t need = linear_workspace_bytes(p);
  UTTT_REQUIRE(a->workspace_bytes >= need && (need == 0 || (a->workspace != nullptr && aligned16(a->workspace))),
               "workspace of %zu bytes (zero-filled, 16-byte aligned) needed, got %zu", need,
               (size_t)a->workspace_bytes);
  LinArgs l{};
  l.m = (int)a->m; l.n = (int)a->n; l.k = (int)a->k;
  l.x = static_cast<const bf16*>(a->x); l.xs = a->x_row_stride;
  l.w = static_cast<const bf16*>(a->w); l.ws = a->w_row_stride;
  l.r = static_cast<const bf16*>(a->residual); l.rs = a->residual_row_stride;
  l.out = static_cast<bf16*>(a->out); l.os = a->out_row_stride;
  l.mtiles = (int)((a->m + p.mt - 1) / p.mt);
  l.splits = p.splits;
  if (need > 0) {
    l.counters = static_cast<unsigned*>(a->workspace);
    l.part = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + kCounterBytes);
  }
  const dim3 grid((unsigned)(p.tiles * p.splits));
  if (p.mt == 128)
    hipLaunchKernelGGL((k_linear<128, kSlots128>), grid, dim3(kLinThreads), 0, st, l);
  else
    hipLaunchKernelGGL((k_linear<64, kSlots64>), grid, dim3(kLinThreads), 0, st, l);
  return launch_status("uttt_linear");
}

}  // namespace uttt

extern "C" int uttt_linear(const uttt_linear_args* a, uttt_stream_t stream) {
  return linear_enqueue(a, static_cast<hipStream_t>(stream), 0);
}
