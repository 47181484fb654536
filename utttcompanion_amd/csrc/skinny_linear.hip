// Skinny slow-weight products of a decode step, written for gfx950 (MI355X): a few rows per
// call (one token per request), y = x W^T, optionally + a residual, bf16 in and out with fp32
// accumulation.  Replaces the F.linear / h + linear(x) calls of the batched decode step
// (reference engine/inference.py:263-276, the block residuals of model/uttt_layer.py:1528-1555
// and the LM head of model/uttt_model.py) where the library GEMM is launch- and
// latency-bound at these shapes.
//
// With x_eps > 0 the rows of x are RMS-normalised over k on the way (the norm weight folded into
// W's columns beforehand): each wave also sums the squares of the x pieces it reads, and the row
// scale 1 / sqrt(mean + eps) multiplies the finished sum, so the norm costs no pass of its own.
//
// One workgroup per (32 output columns, 32 rows).  Its four waves take a quarter of K each: a
// wave loads its x rows and W rows straight into its own LDS region (buffer loads with the lds
// bit, up to three k steps of 64 per round, all in flight at once), reads them back as MFMA
// fragments, and the quarters' sums meet in LDS.  No barrier is needed until that reduction,
// since each wave reads only what it loaded itself.
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {
namespace {

constexpr int kSkWaves = 4;
constexpr int kSkStepBytes = 8192;  // 32 x rows + 32 W rows of 64 k
// k steps per load round of a wave: three (K = 768 in one round) where the grid is small and
// each workgroup's latency is the time; one for wide products (the LM head), so that five
// workgroups fit in a CU's LDS and the grid runs in about one round
constexpr int kSkRoundNarrow = 3, kSkRoundWide = 1;
constexpr int kSkWideBlocks = 512;  // column blocks from which a product counts as wide

struct SkArgs {
  int m, n, k;
  float eps;  // > 0: rows of x are RMS-normalised over k first (the norm weight sits in W)
  const bf16* x;
  int64_t xs;
  const bf16* w;
  int64_t ws;
  const bf16* r;
  int64_t rs;
  bf16* out;
  int64_t os;
};

template <int kSkRound>
__global__ void __launch_bounds__(kSkWaves * 64) k_skinny_linear(const SkArgs a) {
  __shared__ __align__(1024) char lds[kSkWaves * kSkRound * kSkStepBytes];  // >= the 12.5 KB of partial sums
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int rows = min(32, a.m - m0);
  const int nst = a.k / 64, per = (nst + kSkWaves - 1) / kSkWaves;
  const int s_begin = w * per, s_end = min(nst, s_begin + per);
  const bf16* xr = a.x + (int64_t)m0 * a.xs;
  const bf16* wr = a.w + (int64_t)n0 * a.ws;
  const uint32_t region = lds_addr(lds) + (uint32_t)(w * kSkRound * kSkStepBytes);
  int xo[4], wo[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    xo[g] = row_src_off(g, lane, (int)a.xs);
    wo[g] = row_src_off(g, lane, (int)a.ws);
  }
  // wave 0 writes the output: its residual values load first, beside the operand loads (every
  // residual load issued before any store: out may alias the residual; each workgroup reads and
  // writes only its own 32 x 32 block)
  const int col = n0 + acc_col();
  float rv[16];
  if (w == 0 && a.r != nullptr) {
#pragma unroll
    for (int i = 0; i < 16; ++i) rv[i] = to_f32(a.r[(int64_t)(m0 + min(acc_row(i), rows - 1)) * a.rs + col]);
  }
  f32x16 acc;
  zero(acc);
  float ss = 0.f;  // sum of squares of this lane's x pieces (row lane & 31)
  for (int s0 = s_begin; s0 < s_end; s0 += kSkRound) {
    const int cnt = min(kSkRound, s_end - s0);
    for (int i = 0; i < cnt; ++i) {  // rows past `rows` are out of the buffer range: zeros
      const int k0 = (s0 + i) * 64;
      const uint32_t base = region + (uint32_t)(i * kSkStepBytes);
      const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(xr + k0, (uint32_t)(rows * a.xs * 2));
      const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wr + k0, (uint32_t)(32 * a.ws * 2));
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        buffer_load_lds_raw(rx, lds_ptr(base + (uint32_t)(g * 1024)), 16, xo[g], 0, 0, 0);
        buffer_load_lds_raw(rw, lds_ptr(base + 4096u + (uint32_t)(g * 1024)), 16, wo[g], 0, 0, 0);
      }
    }
    wait_vmcnt<0>();  // this wave's loads only: no barrier
    for (int i = 0; i < cnt; ++i) {
      const uint32_t base = region + (uint32_t)(i * kSkStepBytes);
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        fa[kk] = lds_read_bf16x8<0>(row_frag_addr(base, 0, lane, kk));
        fb[kk] = lds_read_bf16x8<0>(row_frag_addr(base + 4096u, 0, lane, kk));
      }
      lds_wait_frags(fa, fb);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk], fb[kk], acc, 0, 0, 0);
      if (a.eps > 0.f) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float e = to_f32(fa[kk][j]);
            ss = fmaf(e, e, ss);
          }
      }
    }
  }
  __syncthreads();  // every wave's reads are done: the regions take the partial sums
  float* red = reinterpret_cast<float*>(lds);
  float* red_ss = red + (kSkWaves - 1) * 16 * 64;  // [wave][row]
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) red[((w - 1) * 16 + i) * 64 + lane] = acc[i];
  }
  if (a.eps > 0.f) {
    ss += __shfl_xor(ss, 32, 64);  // both k halves of row lane & 31
    if (lane < 32) red_ss[w * 32 + lane] = ss;
  }
  __syncthreads();
  if (w != 0) return;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    v[i] = acc[i];
#pragma unroll
    for (int q = 0; q < kSkWaves - 1; ++q) v[i] += red[(q * 16 + i) * 64 + lane];
  }
  if (a.eps > 0.f) {
    const float inv_k = 1.f / (float)a.k;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = acc_row(i);
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < kSkWaves; ++q) t += red_ss[q * 32 + row];
      v[i] *= rsqrtf(t * inv_k + a.eps);
    }
  }
  if (a.r != nullptr) {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] += rv[i];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = acc_row(i);
    if (row < rows) a.out[(int64_t)(m0 + row) * a.os + col] = from_f32<bf16>(v[i]);
  }
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_skinny_linear(const uttt_skinny_linear_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_BF16, "skinny products take bf16 operands");
  UTTT_REQUIRE(a->x_eps >= 0.f, "x_eps must be >= 0 (0: no norm)");
  UTTT_REQUIRE(a->m >= 1 && a->m <= 64, "m must be in [1, 64] (got %lld)", (long long)a->m);
  UTTT_REQUIRE(a->n >= 32 && a->n % 32 == 0 && a->n <= 65535LL * 32, "n must be a positive multiple of 32 (got %lld)",
               (long long)a->n);
  UTTT_REQUIRE(a->k >= 64 && a->k % 64 == 0 && a->k <= 16384, "k must be a multiple of 64 in [64, 16384] (got %lld)",
               (long long)a->k);
  UTTT_REQUIRE(a->x && a->w && a->out, "x, w and out must be non-NULL");
  UTTT_REQUIRE(aligned16(a->x) && aligned16(a->w), "x and w must be 16-byte aligned");
  UTTT_REQUIRE(a->x_row_stride >= a->k && a->x_row_stride % 8 == 0 && a->w_row_stride >= a->k &&
                   a->w_row_stride % 8 == 0,
               "x and w row strides must cover k and be multiples of 16 bytes");
  UTTT_REQUIRE(a->out_row_stride >= a->n && (a->residual == nullptr || a->residual_row_stride >= a->n),
               "out and residual row strides must cover n");
  UTTT_REQUIRE((int64_t)a->m * a->x_row_stride * 2 <= 2147483647LL && 32LL * a->w_row_stride * 2 <= 2147483647LL,
               "operands too large for 32-bit buffer offsets");
  SkArgs s{};
  s.m = (int)a->m;
  s.n = (int)a->n;
  s.k = (int)a->k;
  s.eps = a->x_eps;
  s.x = static_cast<const bf16*>(a->x);
  s.xs = a->x_row_stride;
  s.w = static_cast<const bf16*>(a->w);
  s.ws = a->w_row_stride;
  s.r = static_cast<const bf16*>(a->residual);
  s.rs = a->residual_row_stride;
  s.out = static_cast<bf16*>(a->out);
  s.os = a->out_row_stride;
  const dim3 grid((unsigned)(a->n / 32), (unsigned)((a->m + 31) / 32));
  if (a->n / 32 >= kSkWideBlocks)
    hipLaunchKernelGGL(k_skinny_linear<kSkRoundWide>, grid, dim3(kSkWaves * 64), 0, static_cast<hipStream_t>(stream), s);
  else
    hipLaunchKernelGGL(k_skinny_linear<kSkRoundNarrow>, grid, dim3(kSkWaves * 64), 0, static_cast<hipStream_t>(stream),
                       s);
  return launch_status("uttt_skinny_linear");
}
