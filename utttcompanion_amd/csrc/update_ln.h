// LayerNorm backward of the fast-weight reconstruction loss, shared by the single-chunk
// update (chunk_update.hip) and the layer chain (chunk_chain.hip).
// Per token t of row b: Z = sum of the split partials, Zh = LN(Z) (fp32 statistics),
// E = K + gamma Zh + beta - V, loss_t = 0.5 |E|^2 / s, dZh = (w_t / s) E gamma,
// dZ = rstd (dZh - mean(dZh) - Zh mean(dZh Zh)), w_t = eta_t m_t / max(1, sum m) or eta_t / C
// (reference: model/uttt_layer.py:357-389).
#pragma once

#include "uttt_device.h"

namespace uttt {
namespace {  // each translation unit that launches it owns its copy

constexpr int kMaxPerThread = 16;  // D <= 4096 with 256 threads

struct LnGradArgs {
  int B, C, D, nsplit, tok_pad, normalize;
  float eps;
  const float* zp;  // path-0 partials (nsplit, B, tok_pad, D)
  const void* k; int64_t k_rs;
  const void* v; int64_t v_rs;
  const void* eta; int64_t eta_rs;
  const float* mask; int64_t mask_rs;
  const float* ln_w;
  const float* ln_b;
  void* dz;     // act dtype (B, tok_pad, D)
  float* loss;  // (B, tok_pad): token loss times its mask value
};

// kPer features per thread (D <= 256 kPer); the split partials of a token are read
// 16 / kPer splits at a time so that many loads are in flight together.
template <typename T, int kPer>
__global__ void __launch_bounds__(kThreads) k_ln_grad(const LnGradArgs a) {
  __shared__ float red[4];
  const int t = blockIdx.x, b = blockIdx.y;
  T* dz = static_cast<T*>(a.dz) + ((int64_t)b * a.tok_pad + t) * a.D;
  if (t >= a.C) {
    for (int d = threadIdx.x; d < a.D; d += kThreads) dz[d] = from_f32<T>(0.f);
    if (threadIdx.x == 0) a.loss[b * a.tok_pad + t] = 0.f;
    return;
  }
  const T* kr = static_cast<const T*>(a.k) + (int64_t)b * a.k_rs + (int64_t)t * a.D;
  const T* vr = static_cast<const T*>(a.v) + (int64_t)b * a.v_rs + (int64_t)t * a.D;
  const float inv_d = 1.0f / (float)a.D;

  constexpr int kGroup = 16 / kPer;
  float z[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) z[i] = 0.f;
  for (int sp = 0; sp < a.nsplit; sp += kGroup) {
    float part[kGroup][kPer];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      const bool in = sp + g < a.nsplit;
      const float* src = a.zp + (((int64_t)(sp + g) * a.B + b) * a.tok_pad + t) * a.D;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int d = threadIdx.x + i * kThreads;
        part[g][i] = (in && d < a.D) ? src[d] : 0.f;
      }
    }
#pragma unroll
    for (int g = 0; g < kGroup; ++g)
#pragma unroll
      for (int i = 0; i < kPer; ++i) z[i] += part[g][i];
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) s += z[i];
  const float mean = block_sum(s, red) * inv_d;
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = threadIdx.x + i * kThreads;
    if (d < a.D) {
      const float c = z[i] - mean;
      s2 += c * c;
    }
  }
  const float var = block_sum(s2, red) * inv_d;
  const float rstd = 1.0f / sqrtf(var + a.eps);
  const float inv_scale = a.normalize ? inv_d : 1.0f;

  // z[] becomes z_hat, e[] the reconstruction error
  float e[kPer];
  float se = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = threadIdx.x + i * kThreads;
    e[i] = 0.f;
    if (d < a.D) {
      z[i] = (z[i] - mean) * rstd;
      const float vhat = to_f32(kr[d]) + (z[i] * a.ln_w[d] + a.ln_b[d]);
      e[i] = vhat - to_f32(vr[d]);
      se += e[i] * e[i];
    }
  }
  // the loss and the mask's token count in one reduction
  __shared__ float red2[8];
  const float* mr = a.mask != nullptr ? a.mask + (int64_t)b * a.mask_rs : nullptr;
  float msum = 0.f;  // the chunk's valid tokens (C may exceed the workgroup)
  if (mr != nullptr)
    for (int i = threadIdx.x; i < a.C; i += kThreads) msum += mr[i];
  float sums[2] = {se, msum};
  block_sums<2>(sums, red2);
  const float token_loss = 0.5f * sums[0] * inv_scale;

  const float eta_t = to_f32(static_cast<const T*>(a.eta)[(int64_t)b * a.eta_rs + t]);
  float weight, m_t = 1.f;
  if (mr != nullptr) {
    m_t = mr[t];
    weight = (eta_t * m_t) / fmaxf(sums[1], 1.0f);
  } else {
    weight = eta_t * (1.0f / (float)a.C);
  }
  const float coef = weight * inv_scale;

  float s3 = 0.f, s4 = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = threadIdx.x + i * kThreads;
    if (d < a.D) {
      e[i] = coef * e[i] * a.ln_w[d];  // dZ_hat
      s3 += e[i];
      s4 += e[i] * z[i];
    }
  }
  float moments[2] = {s3, s4};
  block_sums<2>(moments, red2);
  const float m1 = moments[0] * inv_d, m2 = moments[1] * inv_d;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = threadIdx.x + i * kThreads;
    if (d < a.D) dz[d] = from_f32<T>(rstd * (e[i] - m1 - z[i] * m2));
  }
  if (threadIdx.x == 0) a.loss[b * a.tok_pad + t] = a.mask != nullptr ? token_loss * m_t : token_loss;
}

// Launch k_ln_grad with the narrowest per-thread width that covers d_model.
template <typename T>
void launch_ln_grad(dim3 grid, hipStream_t st, const LnGradArgs& g) {
  if (g.D <= 4 * kThreads)
    hipLaunchKernelGGL((k_ln_grad<T, 4>), grid, dim3(kThreads), 0, st, g);
  else if (g.D <= 8 * kThreads)
    hipLaunchKernelGGL((k_ln_grad<T, 8>), grid, dim3(kThreads), 0, st, g);
  else
    hipLaunchKernelGGL((k_ln_grad<T, 16>), grid, dim3(kThreads), 0, st, g);
}

}  // namespace
}  // namespace uttt
