// Epilogue of the uTTT slow projections (reference fused_slow_projections,
// model/uttt_layer.py:1193-1231), written for gfx950 (MI355X).
//
// Input: y = x [W_q; W_k; W_v; w_eta; w_alpha]^T + [0; 0; 0; b_eta; b_alpha] per token row,
// (rows, 3 D + 2) in the activation dtype; or, with the block's input RMSNorm folded in,
// y = h [W_q; ...]'^T of the un-normalised rows h with the norm weight folded into the weight
// columns, scaled here by 1 / rms(h) per row before the biases.  Output per row:
//   q = RMSNorm(y[0:D]) * q_weight, k = RMSNorm(y[D:2D]) * k_weight, v = RMSNorm(y[2D:3D]),
//   eta = inner_lr * sigmoid(y[3D]), alpha = weight_decay * sigmoid(y[3D + 1])
// with RMSNorm(z) = z / sqrt(mean(z^2) + eps), statistics and products in fp32 and one
// rounding to the activation dtype.  One 256-thread workgroup per row replaces the three
// RMSNorm launches and the four elementwise launches of the eager form.
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {
namespace {

constexpr int kMaxPer = 16;  // d_model <= 4096 (KPER of the widest instance)

struct ProjArgs {
  int rows, D;
  float eps, lr, wd;
  const void* y;
  int64_t y_rs;
  const void* qw;  // activation dtype
  const void* kw;
  void* out[3];
  int64_t out_rs;
  void* eta;
  void* alpha;
  const void* x;  // folded input RMSNorm: un-normalised rows, or null
  int64_t x_rs;
  float x_eps;
  const void* ea_bias;  // eta / alpha biases with a folded norm
};

// One 256-thread workgroup per row, KPER values per thread and segment (D <= KPER * 256).  The
// row's q, k, v (and folded-norm input) values are all loaded before any is used, and the four
// sums of squares meet in one LDS reduction.
template <typename T, int KPER>
__global__ void __launch_bounds__(kThreads) k_proj_epilogue(const ProjArgs a) {
  __shared__ float red[4][kThreads / 64];
  const int r = blockIdx.x;
  const T* y = static_cast<const T*>(a.y) + (int64_t)r * a.y_rs;
  const T* x = a.x != nullptr ? static_cast<const T*>(a.x) + (int64_t)r * a.x_rs : nullptr;
  const float inv_d = 1.0f / (float)a.D;
  float v[3][KPER], xv[KPER];
#pragma unroll
  for (int i = 0; i < KPER; ++i) {
    const int d = threadIdx.x + i * kThreads;
    const bool in = d < a.D;
#pragma unroll
    for (int seg = 0; seg < 3; ++seg) v[seg][i] = in ? to_f32(y[seg * a.D + d]) : 0.f;
    xv[i] = in && x != nullptr ? to_f32(x[d]) : 0.f;
  }
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KPER; ++i) {
#pragma unroll
    for (int seg = 0; seg < 3; ++seg) ss[seg] += v[seg][i] * v[seg][i];
    ss[3] += xv[i] * xv[i];
  }
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float t = wave_sum(ss[k]);
    if ((threadIdx.x & 63) == 0) red[k][w] = t;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float t = 0.f;
#pragma unroll
    for (int u = 0; u < kThreads / 64; ++u) t += red[k][u];
    ss[k] = t;
  }
  // folded input norm: every projected value of the row scales by the row's 1 / rms
  const float xs = x != nullptr ? 1.0f / sqrtf(ss[3] * inv_d + a.x_eps) : 1.0f;
#pragma unroll
  for (int seg = 0; seg < 3; ++seg) {
    // RMSNorm of the scaled segment: mean((xs z)^2) = xs^2 mean(z^2)
    const float rstd = 1.0f / sqrtf(xs * xs * ss[seg] * inv_d + a.eps);
    const T* wt = static_cast<const T*>(seg == 0 ? a.qw : seg == 1 ? a.kw : nullptr);
    T* o = static_cast<T*>(a.out[seg]) + (int64_t)r * a.out_rs;
#pragma unroll
    for (int i = 0; i < KPER; ++i) {
      const int d = threadIdx.x + i * kThreads;
      if (d < a.D) {
        const float g = wt != nullptr ? to_f32(wt[d]) : 1.0f;
        o[d] = from_f32<T>(xs * v[seg][i] * rstd * g);
      }
    }
  }
  if (threadIdx.x == 0) {
    const T* eab = static_cast<const T*>(a.ea_bias);
    const float be = eab != nullptr ? to_f32(eab[0]) : 0.f, ba = eab != nullptr ? to_f32(eab[1]) : 0.f;
    const float ye = xs * to_f32(y[3 * a.D]) + be, ya = xs * to_f32(y[3 * a.D + 1]) + ba;
    static_cast<T*>(a.eta)[r] = from_f32<T>(a.lr * sigmoidf_acc(ye));
    static_cast<T*>(a.alpha)[r] = from_f32<T>(a.wd * sigmoidf_acc(ya));
  }
}

// The same epilogue with one wave per row and 16-byte accesses (rows, weights and outputs
// 16-byte aligned with row strides in whole vectors): each lane holds KV vectors of every
// segment, the four sums of squares are reduced inside the wave, and the kernel uses no LDS,
// so it can share a CU with the other stream's LDS-heavy kernels.  The products and roundings
// are those of k_proj_epilogue; only the order of the sums of squares differs.
template <typename T> struct Vec16;
template <> struct Vec16<bf16> { using type = bf16x8; };
template <> struct Vec16<float> { using type = f32x4; };

template <typename T, int KV>
__global__ void __launch_bounds__(64) k_proj_epilogue_vec(const ProjArgs a) {
  using V = typename Vec16<T>::type;
  constexpr int VEC = 16 / sizeof(T);
  const int r = blockIdx.x, lane = threadIdx.x;
  const int nvec = a.D / VEC;
  const T* y = static_cast<const T*>(a.y) + (int64_t)r * a.y_rs;
  const T* x = a.x != nullptr ? static_cast<const T*>(a.x) + (int64_t)r * a.x_rs : nullptr;
  V v[3][KV], xv[KV];
#pragma unroll
  for (int i = 0; i < KV; ++i) {
    const int c = lane + 64 * i;
    const bool in = c < nvec;
#pragma unroll
    for (int seg = 0; seg < 3; ++seg) v[seg][i] = in ? *reinterpret_cast<const V*>(y + seg * a.D + c * VEC) : V{};
    xv[i] = in && x != nullptr ? *reinterpret_cast<const V*>(x + c * VEC) : V{};
  }
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KV; ++i)
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
#pragma unroll
      for (int seg = 0; seg < 3; ++seg) ss[seg] += to_f32(v[seg][i][e]) * to_f32(v[seg][i][e]);
      ss[3] += to_f32(xv[i][e]) * to_f32(xv[i][e]);
    }
#pragma unroll
  for (int k = 0; k < 4; ++k) ss[k] = wave_sum(ss[k]);
  const float inv_d = 1.0f / (float)a.D;
  const float xs = x != nullptr ? 1.0f / sqrtf(ss[3] * inv_d + a.x_eps) : 1.0f;
#pragma unroll
  for (int seg = 0; seg < 3; ++seg) {
    const float rstd = 1.0f / sqrtf(xs * xs * ss[seg] * inv_d + a.eps);
    const T* wt = static_cast<const T*>(seg == 0 ? a.qw : seg == 1 ? a.kw : nullptr);
    T* o = static_cast<T*>(a.out[seg]) + (int64_t)r * a.out_rs;
#pragma unroll
    for (int i = 0; i < KV; ++i) {
      const int c = lane + 64 * i;
      if (c >= nvec) continue;
      V g{};
      if (wt != nullptr) g = *reinterpret_cast<const V*>(wt + c * VEC);
      V out;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        out[e] = from_f32<T>(xs * to_f32(v[seg][i][e]) * rstd * (wt != nullptr ? to_f32(g[e]) : 1.0f));
      *reinterpret_cast<V*>(o + c * VEC) = out;
    }
  }
  if (lane == 0) {
    const T* eab = static_cast<const T*>(a.ea_bias);
    const float be = eab != nullptr ? to_f32(eab[0]) : 0.f, ba = eab != nullptr ? to_f32(eab[1]) : 0.f;
    const float ye = xs * to_f32(y[3 * a.D]) + be, ya = xs * to_f32(y[3 * a.D + 1]) + ba;
    static_cast<T*>(a.eta)[r] = from_f32<T>(a.lr * sigmoidf_acc(ye));
    static_cast<T*>(a.alpha)[r] = from_f32<T>(a.wd * sigmoidf_acc(ya));
  }
}

template <typename T>
bool vec_fits(const ProjArgs& p) {
  constexpr int VEC = 16 / sizeof(T);
  auto al = [](const void* q) { return q == nullptr || aligned16(q); };
  return p.D % VEC == 0 && p.D <= 8 * 64 * VEC && p.y_rs % VEC == 0 && p.out_rs % VEC == 0 &&
         (p.x == nullptr || p.x_rs % VEC == 0) && al(p.y) && al(p.x) && al(p.qw) && al(p.kw) && al(p.out[0]) &&
         al(p.out[1]) && al(p.out[2]);
}

template <typename T>
void launch_epilogue(const ProjArgs& p, hipStream_t st) {
  if (vec_fits<T>(p)) {
    constexpr int VEC = 16 / sizeof(T);
    const int kv = (p.D / VEC + 63) / 64;
    if (kv <= 1)
      hipLaunchKernelGGL((k_proj_epilogue_vec<T, 1>), dim3(p.rows), dim3(64), 0, st, p);
    else if (kv <= 2)
      hipLaunchKernelGGL((k_proj_epilogue_vec<T, 2>), dim3(p.rows), dim3(64), 0, st, p);
    else if (kv <= 4)
      hipLaunchKernelGGL((k_proj_epilogue_vec<T, 4>), dim3(p.rows), dim3(64), 0, st, p);
    else
      hipLaunchKernelGGL((k_proj_epilogue_vec<T, 8>), dim3(p.rows), dim3(64), 0, st, p);
    return;
  }
  if (p.D <= 4 * kThreads)
    hipLaunchKernelGGL((k_proj_epilogue<T, 4>), dim3(p.rows), dim3(kThreads), 0, st, p);
  else if (p.D <= 8 * kThreads)
    hipLaunchKernelGGL((k_proj_epilogue<T, 8>), dim3(p.rows), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((k_proj_epilogue<T, 16>), dim3(p.rows), dim3(kThreads), 0, st, p);
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_proj_epilogue(const uttt_proj_epilogue_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->rows >= 1 && a->rows <= 2147483647LL, "rows must be >= 1 (got %lld)", (long long)a->rows);
  UTTT_REQUIRE(a->d_model >= 1 && a->d_model <= kMaxPer * kThreads, "d_model must be in [1, %d] (got %lld)",
               kMaxPer * kThreads, (long long)a->d_model);
  UTTT_REQUIRE(a->act_dtype == UTTT_DTYPE_F32 || a->act_dtype == UTTT_DTYPE_BF16, "act_dtype must be F32 or BF16");
  UTTT_REQUIRE(a->y && a->q_weight && a->k_weight && a->q && a->k && a->v && a->eta && a->alpha,
               "pointers must be non-NULL");
  UTTT_REQUIRE(a->y_row_stride >= 3 * a->d_model + 2 && a->out_row_stride >= a->d_model,
               "row strides must cover a row");
  UTTT_REQUIRE(a->x == nullptr || a->x_row_stride >= a->d_model, "x row stride must cover a row");
  UTTT_REQUIRE(a->x == nullptr || a->x_eps > 0.f, "x_eps must be > 0 with a folded norm");
  ProjArgs p{};
  p.rows = (int)a->rows;
  p.D = (int)a->d_model;
  p.eps = a->eps;
  p.lr = a->inner_lr;
  p.wd = a->weight_decay;
  p.y = a->y;
  p.y_rs = a->y_row_stride;
  p.qw = a->q_weight;
  p.kw = a->k_weight;
  p.out[0] = a->q;
  p.out[1] = a->k;
  p.out[2] = a->v;
  p.out_rs = a->out_row_stride;
  p.eta = a->eta;
  p.alpha = a->alpha;
  p.x = a->x;
  p.x_rs = a->x_row_stride;
  p.x_eps = a->x_eps;
  p.ea_bias = a->eta_alpha_bias;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->act_dtype == UTTT_DTYPE_BF16)
    launch_epilogue<bf16>(p, st);
  else
    launch_epilogue<float>(p, st);
  return launch_status("uttt_proj_epilogue");
}
