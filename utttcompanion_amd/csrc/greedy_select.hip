// Greedy token selection of a decode step, written for gfx950 (MI355X): per row of logits, the
// index of the largest value after the excluded ids (PAD / BOS / UNK) and the ids at or past the
// active-vocabulary limit are set to -inf.  Replaces the temperature-0 branch of the reference's
// sampling (model/uttt_model.py:1203-1221: float copy, three masked ids, the active-vocabulary
// mask, torch.argmax) with one launch that reads each logit once.
//
// argmax semantics follow torch.argmax: NaN counts as the largest value, ties go to the lowest
// index, and a row with every entry -inf gives 0.
#include <algorithm>

#include "uttt_device.h"
#include "uttt_host.h"

namespace uttt {
namespace {

struct SelectArgs {
  int vocab, limit;
  uint64_t low;  // excluded ids below 64, as a bit mask
  int n_high;    // excluded ids of 64 and above
  int high[8];
  const void* logits;
  int64_t rs;
  int64_t* out;
  int64_t* advance;
};

struct Best {
  float v;
  int i;
};

// a ranks before b
__device__ __forceinline__ bool ahead(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

__device__ __forceinline__ void take(Best& b, float v, int i) {
  if (ahead(v, i, b.v, b.i)) {
    b.v = v;
    b.i = i;
  }
}

constexpr int kSelThreads = 1024;
constexpr int kSelUnroll = 4;  // loads in flight per thread

__device__ __forceinline__ bool excluded(const SelectArgs& a, int i) {
  if (i >= a.limit) return true;
  if (i < 64) return (a.low >> i) & 1;
  bool m = false;
  for (int k = 0; k < a.n_high; ++k) m |= i == a.high[k];
  return m;
}

// VEC logits per load: 16 bytes where every row start is 16-byte aligned, else one.  One
// workgroup per row; each thread keeps kSelUnroll loads in flight.
template <typename T, int VEC>
__global__ void __launch_bounds__(kSelThreads) k_greedy_select(const SelectArgs a) {
  __shared__ float sv[kSelThreads / 64];
  __shared__ int si[kSelThreads / 64];
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  const int row = blockIdx.x;
  const T* x = static_cast<const T*>(a.logits) + (int64_t)row * a.rs;
  Best b{-INFINITY, 0x7fffffff};
  // the position to advance loads beside the logits, not after the reduction
  int64_t adv = 0;
  if (threadIdx.x == 0 && a.advance != nullptr) adv = a.advance[row];
  const int nvec = a.vocab / VEC;
  for (int c0 = threadIdx.x; c0 < nvec; c0 += kSelThreads * kSelUnroll) {
    vec_t v[kSelUnroll];
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int c = c0 + u * kSelThreads;
      if (c < nvec) v[u] = *reinterpret_cast<const vec_t*>(x + (int64_t)c * VEC);
    }
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int c = c0 + u * kSelThreads;
      if (c < nvec) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int i = c * VEC + e;
          take(b, excluded(a, i) ? -INFINITY : to_f32(v[u][e]), i);
        }
      }
    }
  }
  for (int i = nvec * VEC + threadIdx.x; i < a.vocab; i += kSelThreads)  // tail of a ragged vocabulary
    take(b, excluded(a, i) ? -INFINITY : to_f32(x[i]), i);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(b.v, off, 64);
    const int oi = __shfl_xor(b.i, off, 64);
    take(b, ov, oi);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = b.v;
    si[w] = b.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kSelThreads / 64; ++q) take(b, sv[q], si[q]);
    a.out[row] = (int64_t)b.i;
    if (a.advance != nullptr) a.advance[row] = adv + 1;
  }
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_greedy_select(const uttt_greedy_args* a, uttt_stream_t stream) {
  UTTT_REQUIRE(a != nullptr, "args is NULL");
  UTTT_REQUIRE(a->rows >= 1 && a->rows <= 65535, "rows must be in [1, 65535]");
  UTTT_REQUIRE(a->vocab >= 1 && a->vocab <= (1LL << 30), "vocab must be in [1, 2^30]");
  UTTT_REQUIRE(a->dtype == UTTT_DTYPE_BF16 || a->dtype == UTTT_DTYPE_F32, "logits must be bf16 or fp32");
  UTTT_REQUIRE(a->n_banned >= 0 && a->n_banned <= 8, "at most 8 excluded ids");
  for (int k = 0; k < a->n_banned; ++k) UTTT_REQUIRE(a->banned[k] >= 0, "excluded ids must be >= 0");
  UTTT_REQUIRE(a->logits != nullptr && a->out != nullptr, "logits and out must be non-NULL");
  UTTT_REQUIRE(a->row_stride >= a->vocab, "the row stride must cover vocab");
  SelectArgs s{};
  s.vocab = (int)a->vocab;
  for (int k = 0; k < a->n_banned; ++k) {
    if (a->banned[k] < 64)
      s.low |= uint64_t(1) << a->banned[k];
    else
      s.high[s.n_high++] = a->banned[k];
  }
  s.limit = (int)std::min<int64_t>(a->active_limit < 0 ? a->vocab : a->active_limit, a->vocab);
  s.logits = a->logits;
  s.rs = a->row_stride;
  s.out = a->out;
  s.advance = a->advance;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)a->rows);
  const bool bf = a->dtype == UTTT_DTYPE_BF16;
  const bool vec = aligned16(a->logits) && a->row_stride % (bf ? 8 : 4) == 0;
  if (bf && vec)
    hipLaunchKernelGGL((k_greedy_select<bf16, 8>), grid, dim3(kSelThreads), 0, st, s);
  else if (bf)
    hipLaunchKernelGGL((k_greedy_select<bf16, 1>), grid, dim3(kSelThreads), 0, st, s);
  else if (vec)
    hipLaunchKernelGGL((k_greedy_select<float, 4>), grid, dim3(kSelThreads), 0, st, s);
  else
    hipLaunchKernelGGL((k_greedy_select<float, 1>), grid, dim3(kSelThreads), 0, st, s);
  return launch_status("uttt_greedy_select");
}
