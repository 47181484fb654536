// Device-side building blocks shared by the uTTT HIP kernels (gfx950 / CDNA4).
//
// * 64-wide wavefronts; every kernel here runs 256-thread workgroups (4 waves).
// * Matrix products go through 32x32 MFMA wave tiles:
//     fp32 operands: v_mfma_f32_32x32x2f32   (K = 2 per instruction)
//     bf16 operands: v_mfma_f32_32x32x16_bf16 (K = 16 per instruction, gfx950)
//   Operand layout (lane l, r = l % 32, h = l / 32):
//     A (32 x K):   lane supplies A[r][k0 + h*KPL + j], j < KPL (KPL = 1 fp32, 8 bf16)
//     B (K x 32):   lane supplies B[k0 + h*KPL + j][r]
//   Result (32 x 32, 16 floats per lane): acc[i] = C[8*(i/4) + 4*h + (i%4)][r].
// * LDS operand tiles are stored "k-contiguous": A as [row][k], B as [col][k]
//   (i.e. B transposed), each row padded so lane reads spread over the banks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uttt {

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// ---------------------------------------------------------------------------
// MFMA traits
// ---------------------------------------------------------------------------
template <typename T> struct Mma;

template <> struct Mma<float> {
  static constexpr int kK = 2;     // K per instruction
  static constexpr int kPerLane = 1;
  static constexpr int kPad = 1;   // LDS row padding (elements)
  __device__ __forceinline__ static void step(f32x16& acc, const float* a_row, const float* b_row, int k0, int h) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a_row[k0 + h], b_row[k0 + h], acc, 0, 0, 0);
  }
};

template <> struct Mma<bf16> {
  static constexpr int kK = 16;
  static constexpr int kPerLane = 8;
  static constexpr int kPad = 8;   // keeps 16-byte alignment of every row
  __device__ __forceinline__ static void step(f32x16& acc, const bf16* a_row, const bf16* b_row, int k0, int h) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(a_row + k0 + h * 8);
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(b_row + k0 + h * 8);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  }
};

// acc(32x32) += A(32 x KT) * B(KT x 32); A at lds `a` ([32][lda]), B^T at `b` ([32][ldb]).
template <typename T, int KT>
__device__ __forceinline__ void wave_mma(f32x16& acc, const T* a, int lda, const T* b, int ldb) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const T* a_row = a + r * lda;
  const T* b_row = b + r * ldb;
#pragma unroll
  for (int k0 = 0; k0 < KT; k0 += Mma<T>::kK) Mma<T>::step(acc, a_row, b_row, k0, h);
}

__device__ __forceinline__ void zero(f32x16& acc) {
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
}

// Row / column of accumulator element i for this lane inside a 32x32 wave tile.
__device__ __forceinline__ int acc_row(int i) { return 8 * (i >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (i & 3); }
__device__ __forceinline__ int acc_col() { return threadIdx.x & 31; }

// ---------------------------------------------------------------------------
// LDS staging of 64 x KT operand tiles (256 threads cooperate)
// ---------------------------------------------------------------------------

// dst[row][k] = src[row * src_ld + k] for row < rows_valid (else 0), k < KT.
// Source element type S (float or bf16) converted to T.
template <typename T, typename S, int KT>
__device__ __forceinline__ void stage_rows(T* dst, int ldd, const S* src, int64_t src_ld, int rows_valid) {
  constexpr int kTotal = 64 * KT;
  for (int idx = threadIdx.x; idx < kTotal; idx += kThreads) {
    const int row = idx / KT, k = idx - row * KT;
    const float v = row < rows_valid ? to_f32(src[(int64_t)row * src_ld + k]) : 0.f;
    dst[row * ldd + k] = from_f32<T>(v);
  }
}

// Transposed staging: dst[col][k] = src[k * src_ld + col] for k < k_valid (else 0),
// col < 64.  Threads walk the source row-major so global reads coalesce.
template <typename T, typename S, int KT>
__device__ __forceinline__ void stage_cols(T* dst, int ldd, const S* src, int64_t src_ld, int k_valid) {
  constexpr int kTotal = 64 * KT;
  for (int idx = threadIdx.x; idx < kTotal; idx += kThreads) {
    const int k = idx >> 6, col = idx & 63;
    const float v = k < k_valid ? to_f32(src[(int64_t)k * src_ld + col]) : 0.f;
    dst[col * ldd + k] = from_f32<T>(v);
  }
}

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Sum over the 256-thread block; `scratch` holds >= 4 floats of LDS.  All threads get the sum.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

__device__ __forceinline__ float block_max(float v, float* scratch) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
}

__device__ __forceinline__ float sigmoidf_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace uttt
