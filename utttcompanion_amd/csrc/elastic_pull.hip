// Slow-anchor elastic pull and drift norms of per-row fast weights (gfx950).
//   pull:  P = (1 - lambda) W + lambda W0;  with a ceiling r > 0:
//          s_b = min(1, r |W0| / |P_b - W0|)  (norms over all three matrices, +1e-8 inside sqrt)
//          W' = W0 + (P - W0) s_b            (reference model/uttt_layer.py:773-832)
//   drift: |W - W0|_F per matrix over all rows and |W0|_F per matrix (reference :834-874)
// HBM-bound streaming passes over the three (B, D, F) fp32 matrices; each row is split
// into `kBlocksPerRow` contiguous ranges whose partial sums go to a small workspace.
#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {

constexpr int kBlocksPerRow = 128;

struct PullArgs {
  int64_t per_mat;  // D * F
  float lam, ratio;
  const float* w[3];
  const float* w0[3];
  float* out[3];
  float* part;      // (B, kBlocksPerRow) sum of diff^2 ; then (kBlocksPerRow) sum of w0^2
  int B;
};

__device__ __forceinline__ void row_range(int64_t total, int blk, int64_t& lo, int64_t& hi) {
  const int64_t per = (total + kBlocksPerRow - 1) / kBlocksPerRow;
  lo = min(total, (int64_t)blk * per);
  hi = min(total, lo + per);
}

__device__ __forceinline__ float pulled(float w, float w0, float lam) {
#pragma clang fp contract(off)
  return (1.0f - lam) * w + lam * w0;
}

// grid (kBlocksPerRow, B): partial |P - W0|^2 per row, and |W0|^2 (row 0 blocks)
__global__ void __launch_bounds__(kThreads) k_pull_reduce(const PullArgs a) {
  __shared__ float red[4];
  const int blk = blockIdx.x, b = blockIdx.y;
  int64_t lo, hi;
  row_range(3 * a.per_mat, blk, lo, hi);
  float sd = 0.f, s0 = 0.f;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) {
    const int m = (int)(i / a.per_mat);
    const int64_t j = i - (int64_t)m * a.per_mat;
    const float w0 = a.w0[m][j];
    const float d = pulled(a.w[m][(int64_t)b * a.per_mat + j], w0, a.lam) - w0;
    sd += d * d;
    s0 += w0 * w0;
  }
  sd = block_sum(sd, red);
  s0 = block_sum(s0, red);
  if (threadIdx.x == 0) {
    a.part[(int64_t)b * kBlocksPerRow + blk] = sd;
    if (b == 0) a.part[(int64_t)a.B * kBlocksPerRow + blk] = s0;
  }
}

// grid (kBlocksPerRow, B)
__global__ void __launch_bounds__(kThreads) k_pull_apply(const PullArgs a) {
  __shared__ float scale_s;
  const int blk = blockIdx.x, b = blockIdx.y;
  if (a.ratio > 0.f && threadIdx.x < 64) {
    float sd = 0.f, s0 = 0.f;
    for (int i = threadIdx.x; i < kBlocksPerRow; i += 64) {
      sd += a.part[(int64_t)b * kBlocksPerRow + i];
      s0 += a.part[(int64_t)a.B * kBlocksPerRow + i];
    }
    sd = wave_sum(sd);
    s0 = wave_sum(s0);
    if (threadIdx.x == 0) {
      const float base = sqrtf(s0 + 1e-8f), drift = sqrtf(sd + 1e-8f);
      scale_s = fminf(a.ratio * base / drift, 1.0f);
    }
  }
  __syncthreads();
  int64_t lo, hi;
  row_range(3 * a.per_mat, blk, lo, hi);
  const bool capped = a.ratio > 0.f;
  const float sc = capped ? scale_s : 1.f;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) {
    const int m = (int)(i / a.per_mat);
    const int64_t j = i - (int64_t)m * a.per_mat;
    const int64_t off = (int64_t)b * a.per_mat + j;
    const float w0 = a.w0[m][j];
    const float p = pulled(a.w[m][off], w0, a.lam);
    float r;
    {
#pragma clang fp contract(off)
      r = capped ? w0 + (p - w0) * sc : p;
    }
    a.out[m][off] = r;
  }
}

// grid (kBlocksPerRow, B): partial sums of (W - W0)^2 per matrix; row 0 also W0^2 per matrix
__global__ void __launch_bounds__(kThreads) k_drift_reduce(const PullArgs a) {
  __shared__ float red[4];
  const int blk = blockIdx.x, b = blockIdx.y;
  int64_t lo, hi;
  row_range(3 * a.per_mat, blk, lo, hi);
  float sd[3] = {0.f, 0.f, 0.f}, s0[3] = {0.f, 0.f, 0.f};
  for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) {
    const int m = (int)(i / a.per_mat);
    const int64_t j = i - (int64_t)m * a.per_mat;
    const float w0 = a.w0[m][j];
    const float d = a.w[m][(int64_t)b * a.per_mat + j] - w0;
#pragma unroll
    for (int mm = 0; mm < 3; ++mm) {
      if (mm == m) {
        sd[mm] += d * d;
        s0[mm] += w0 * w0;
      }
    }
  }
  float* part = a.part + ((int64_t)b * kBlocksPerRow + blk) * 6;
#pragma unroll
  for (int mm = 0; mm < 3; ++mm) {
    const float x = block_sum(sd[mm], red);
    const float y = block_sum(s0[mm], red);
    if (threadIdx.x == 0) {
      part[mm] = x;
      part[3 + mm] = b == 0 ? y : 0.f;
    }
  }
}

// one workgroup: out[0..2] = sum_b sum (W - W0)^2 per matrix, out[3..5] = sum W0^2 per matrix
__global__ void __launch_bounds__(kThreads) k_drift_finalize(const float* part, int B, float* out) {
  __shared__ float red[4];
  for (int k = 0; k < 6; ++k) {
    float s = 0.f;
    for (int i = threadIdx.x; i < B * kBlocksPerRow; i += kThreads) s += part[(int64_t)i * 6 + k];
    s = block_sum(s, red);
    if (threadIdx.x == 0) out[k] = s;
  }
}

static int check_pull(int64_t B, int64_t D, int64_t F) {
  UTTT_REQUIRE(B >= 1 && B <= 65535, "batch must be in [1, 65535]");
  UTTT_REQUIRE(D >= 1 && F >= 1, "d_model and d_ff must be >= 1");
  return UTTT_OK;
}

}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_elastic_pull_workspace(int64_t batch) {
  return sizeof(float) * (size_t)(batch + 1) * kBlocksPerRow * 6;
}

extern "C" int uttt_elastic_pull(const uttt_elastic_pull_args* a, void* workspace, size_t workspace_bytes,
                                 uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  int rc = check_pull(a->batch, a->d_model, a->d_ff);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(a->w_up && a->w_gate && a->w_down && a->w0_up && a->w0_gate && a->w0_down &&
               a->out_up && a->out_gate && a->out_down, "pointers must be non-NULL");
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= uttt_elastic_pull_workspace(a->batch),
               "workspace too small");
  PullArgs p{};
  p.per_mat = a->d_model * a->d_ff;
  p.lam = a->anchor_lambda;
  p.ratio = a->max_drift_ratio;
  p.w[0] = a->w_up; p.w[1] = a->w_gate; p.w[2] = a->w_down;
  p.w0[0] = a->w0_up; p.w0[1] = a->w0_gate; p.w0[2] = a->w0_down;
  p.out[0] = a->out_up; p.out[1] = a->out_gate; p.out[2] = a->out_down;
  p.part = static_cast<float*>(workspace);
  p.B = (int)a->batch;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(kBlocksPerRow, (unsigned)a->batch);
  if (a->max_drift_ratio > 0.f) hipLaunchKernelGGL(k_pull_reduce, grid, dim3(kThreads), 0, st, p);
  hipLaunchKernelGGL(k_pull_apply, grid, dim3(kThreads), 0, st, p);
  return launch_status("uttt_elastic_pull");
}

extern "C" int uttt_fast_weight_drift(int64_t batch, int64_t d_model, int64_t d_ff, const float* w_up,
                                      const float* w_gate, const float* w_down, const float* w0_up,
                                      const float* w0_gate, const float* w0_down, float* out6, void* workspace,
                                      size_t workspace_bytes, uttt_stream_t stream) {
  int rc = check_pull(batch, d_model, d_ff);
  if (rc != UTTT_OK) return rc;
  UTTT_REQUIRE(w_up && w_gate && w_down && w0_up && w0_gate && w0_down && out6, "pointers must be non-NULL");
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= uttt_elastic_pull_workspace(batch), "workspace too small");
  PullArgs p{};
  p.per_mat = d_model * d_ff;
  p.w[0] = w_up; p.w[1] = w_gate; p.w[2] = w_down;
  p.w0[0] = w0_up; p.w0[1] = w0_gate; p.w0[2] = w0_down;
  p.part = static_cast<float*>(workspace);
  p.B = (int)batch;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_drift_reduce, dim3(kBlocksPerRow, (unsigned)batch), dim3(kThreads), 0, st, p);
  hipLaunchKernelGGL(k_drift_finalize, dim3(1), dim3(kThreads), 0, st, p.part, (int)batch, out6);
  return launch_status("uttt_fast_weight_drift");
}
