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
  static constexpr int kPad = 4;   // LDS row padding (elements); keeps rows 16-byte aligned
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

// acc[2 rq + cq] (32x32 each) += A(rows 32 rq.., KT) * B(KT, cols 32 cq..): one wave takes a
// 64 x 64 tile, each A and B fragment read from LDS once per k step and used twice.
template <typename T, int KT>
__device__ __forceinline__ void wave_mma64(f32x16 (&acc)[4], const T* a, int lda, const T* b, int ldb) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const T* a0 = a + r * lda;
  const T* a1 = a + (32 + r) * lda;
  const T* b0 = b + r * ldb;
  const T* b1 = b + (32 + r) * ldb;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int k0 = 0; k0 < KT; k0 += 16) {
      const bf16x8 fa0 = *reinterpret_cast<const bf16x8*>(a0 + k0 + h * 8);
      const bf16x8 fa1 = *reinterpret_cast<const bf16x8*>(a1 + k0 + h * 8);
      const bf16x8 fb0 = *reinterpret_cast<const bf16x8*>(b0 + k0 + h * 8);
      const bf16x8 fb1 = *reinterpret_cast<const bf16x8*>(b1 + k0 + h * 8);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa0, fb0, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa0, fb1, acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa1, fb0, acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa1, fb1, acc[3], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int k0 = 0; k0 < KT; k0 += Mma<T>::kK) {
      Mma<T>::step(acc[0], a0, b0, k0, h);
      Mma<T>::step(acc[1], a0, b1, k0, h);
      Mma<T>::step(acc[2], a1, b0, k0, h);
      Mma<T>::step(acc[3], a1, b1, k0, h);
    }
  }
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
// Register-staged tiles with 16-byte global loads.  `load` issues every global read of
// a tile into registers (so a stage can be loaded while the previous one is consumed);
// `store` converts to the MFMA operand type and writes the LDS tile.  Sources must be
// 16-byte aligned with row strides that are multiples of 16 bytes.
// ---------------------------------------------------------------------------
template <typename S> struct Lanes16;
template <> struct Lanes16<float> {
  static constexpr int kVec = 4;
  __device__ __forceinline__ static float get(const uint4& v, int i) {
    return __uint_as_float(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
  }
};
template <> struct Lanes16<bf16> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float get(const uint4& v, int i) {
    const uint32_t w = i < 2 ? v.x : i < 4 ? v.y : i < 6 ? v.z : v.w;
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};

// store kVec source elements of one 16-byte chunk as T, contiguous at dst
template <typename S, typename T>
__device__ __forceinline__ void store_chunk(T* dst, const uint4& v) {
  if constexpr (sizeof(S) == sizeof(T)) {
    *reinterpret_cast<uint4*>(dst) = v;  // same type: raw copy (dst 16-byte aligned)
  } else {
#pragma unroll
    for (int i = 0; i < Lanes16<S>::kVec; ++i) dst[i] = from_f32<T>(Lanes16<S>::get(v, i));
  }
}

// 64 rows x KT columns, row-major source; LDS tile [row][k]
template <typename S, int KT>
struct RowStage {
  static constexpr int kVec = Lanes16<S>::kVec;
  static constexpr int kPerRow = KT / kVec;
  static constexpr int kN = 64 * kPerRow / kThreads;
  static_assert((64 * kPerRow) % kThreads == 0, "tile must split evenly over the workgroup");
  uint4 r[kN];

  __device__ __forceinline__ void load(const S* src, int64_t ld, int rows_valid) {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kPerRow, c = idx - row * kPerRow;
      r[j] = row < rows_valid ? *reinterpret_cast<const uint4*>(src + (int64_t)row * ld + c * kVec)
                              : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  template <typename T>
  __device__ __forceinline__ void store(T* dst, int ldd) const {
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int row = idx / kPerRow, c = idx - row * kPerRow;
      store_chunk<S, T>(dst + row * ldd + c * kVec, r[j]);
    }
  }
};

// KT source rows (k) x 64 columns; LDS tile transposed to [col][k].  One unit loads 8
// consecutive rows of one 16-byte column group and writes 8 consecutive k per column.
template <typename S, int KT>
struct ColStage {
  static constexpr int kVec = Lanes16<S>::kVec;
  static constexpr int kColGroups = 64 / kVec;
  static constexpr int kUnits = (KT / 8) * kColGroups;
  uint4 r[8];
  int unit;

  __device__ __forceinline__ void load(const S* src, int64_t ld, int k_valid, int u) {
    unit = u;
    if (u >= kUnits) return;
    const int kg = u / kColGroups, cg = u - kg * kColGroups;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = kg * 8 + i;
      r[i] = k < k_valid ? *reinterpret_cast<const uint4*>(src + (int64_t)k * ld + cg * kVec)
                         : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  template <typename T>
  __device__ __forceinline__ void store(T* dst, int ldd) const {
    if (unit >= kUnits) return;
    const int kg = unit / kColGroups, cg = unit - kg * kColGroups;
#pragma unroll
    for (int v = 0; v < kVec; ++v) {
      T* d = dst + (cg * kVec + v) * ldd + kg * 8;
      if constexpr (sizeof(T) == 2) {
        bf16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(Lanes16<S>::get(r[i], v));
        *reinterpret_cast<bf16x8*>(d) = o;
      } else {
        f32x4 o0, o1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o0[i] = Lanes16<S>::get(r[i], v);
          o1[i] = Lanes16<S>::get(r[i + 4], v);
        }
        *reinterpret_cast<f32x4*>(d) = o0;
        *reinterpret_cast<f32x4*>(d + 4) = o1;
      }
    }
  }
};

// bf16 KT x 64 tile transposed to [col][k] by 8 * KT / 8 units of 4 rows each (twice the
// units of ColStage, half the registers per thread): two such tiles occupy all 256 threads.
template <int KT>
struct ColStage4 {
  static constexpr int kColGroups = 8;  // 16-byte column groups of 8 bf16
  static constexpr int kUnits = (KT / 4) * kColGroups;
  uint4 r[4];
  int unit;

  __device__ __forceinline__ void load(const bf16* src, int64_t ld, int k_valid, int u) {
    unit = u;
    if (u >= kUnits) return;
    const int kg = u / kColGroups, cg = u - kg * kColGroups;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kg * 4 + i;
      r[i] = k < k_valid ? *reinterpret_cast<const uint4*>(src + (int64_t)k * ld + cg * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  // dst rows are 8-byte aligned (ldd a multiple of 4)
  __device__ __forceinline__ void store(bf16* dst, int ldd) const {
    if (unit >= kUnits) return;
    const int kg = unit / kColGroups, cg = unit - kg * kColGroups;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      // column v of the 4 rows: the 16-bit halves of word v / 2 of each row
      const int sh = (v & 1) * 16;
      const uint32_t w0 = (v < 2 ? r[0].x : v < 4 ? r[0].y : v < 6 ? r[0].z : r[0].w) >> sh;
      const uint32_t w1 = (v < 2 ? r[1].x : v < 4 ? r[1].y : v < 6 ? r[1].z : r[1].w) >> sh;
      const uint32_t w2 = (v < 2 ? r[2].x : v < 4 ? r[2].y : v < 6 ? r[2].z : r[2].w) >> sh;
      const uint32_t w3 = (v < 2 ? r[3].x : v < 4 ? r[3].y : v < 6 ? r[3].z : r[3].w) >> sh;
      uint2 o;
      o.x = (w0 & 0xffffu) | (w1 << 16);
      o.y = (w2 & 0xffffu) | (w3 << 16);
      *reinterpret_cast<uint2*>(dst + (cg * 8 + v) * ldd + kg * 4) = o;
    }
  }
};

// ---------------------------------------------------------------------------
// Buffer resources: one SGPR descriptor per array, 32-bit byte offsets per access; out-of-range
// loads return 0 and out-of-range stores are dropped.
// ---------------------------------------------------------------------------
constexpr int kBufferFlags = 0x00020000;  // raw 32-bit data format (CDNA buffer descriptor word 3)
constexpr int kNonTemporal = 2;           // cache policy of streaming accesses

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads and transposing LDS reads (gfx950)
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// buffer_load_dword{,x4} ... lds: lane i's `size` bytes land at the LDS address + i * size
// (the LDS address is wave-uniform); out-of-range lanes write zeros
__device__ void buffer_load_lds_raw(__amdgpu_buffer_rsrc_t rsrc, lds_void_ptr lds, int size, int voffset, int soffset,
                                    int offset, int aux) __asm("llvm.amdgcn.raw.ptr.buffer.load.lds");

// a 16-byte-per-lane direct-to-LDS load whose cache policy follows a wave-uniform choice: data
// streamed once (the state copies) goes non-temporal, so that it does not push out of L2 the
// slabs that the other tiles of a row re-read; everything else keeps the default policy
__device__ __forceinline__ void buffer_load_lds16(bool streamed, __amdgpu_buffer_rsrc_t rsrc, lds_void_ptr lds,
                                                  int voffset) {
  if (streamed)
    buffer_load_lds_raw(rsrc, lds, 16, voffset, 0, 0, kNonTemporal);
  else
    buffer_load_lds_raw(rsrc, lds, 16, voffset, 0, 0, 0);
}

// Whether a pass over the bf16 state copies of B rows (D x F each) streams them non-temporally:
// only when the two matrices a pass reads (4 B D F bytes) exceed 96 MiB, and only in passes whose
// copies no later pass of the chunk reads again (the snapshot products, the readout).  Smaller
// passes keep the default policy, and so do the down pass and the back pass at every size: the back
// pass re-reads the down pass's W_down / S_down copies, and finds them in the 256 MB infinity
// cache.  Measured: the hint on every pass took the config-2 prefill (50 MB per pass) from 59.9 to
// 62.4 ms; at config 3 (180 MB per pass) it took the prefill from 544 to 530 ms, and leaving the
// down pass out of it to 523 ms.
constexpr int64_t kStreamNtMinElems = 24LL << 20;
__device__ __forceinline__ bool stream_nt(int B, int D, int F) {
  return (int64_t)B * D * F > kStreamNtMinElems;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(p);  // the low half of a generic LDS address is its offset
}
__device__ __forceinline__ lds_void_ptr lds_ptr(uint32_t addr) { return (lds_void_ptr)(uintptr_t)addr; }

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives element (i & 3) of the 8 bytes
// that lane 4 e + (i >> 2) addresses, for e = 0..3.  With lane j of the group pointing at row
// r0 + j / 4, columns c0 + 4 (j % 4) .. + 3 of a row-major 16-bit matrix, lane i receives column
// c0 + i of rows r0 .. r0 + 3.  Issued as inline assembly so that the compiler adds no wait on
// outstanding direct-to-LDS loads; the caller waits for lgkmcnt before using the result.  It
// stays ordered with the barrier and wait builtins (all have side effects); no memory clobber,
// which would keep the compiler from reading uniform kernel data with scalar loads.
template <int OFF>
__device__ __forceinline__ i16x4 lds_read_tr16(uint32_t addr) {
  i16x4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// plain LDS reads issued the same way (waited for by the caller)
__device__ __forceinline__ f32x4 lds_read_b128(uint32_t addr) {
  f32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
template <int OFF>
__device__ __forceinline__ bf16x8 lds_read_bf16x8(uint32_t addr) {
  bf16x8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
__device__ __forceinline__ float lds_read_b32(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// ---------------------------------------------------------------------------
// Operands in LDS without register staging (bf16 activations): buffer loads with the lds bit
// write 1 KB per wave instruction (lane i at +16 i), and the MFMA reads them back, through
// transposing LDS reads for token-major slabs.  Both go around the compiler's wait tracking
// (explicit vmcnt / lgkmcnt waits), so a kernel counts its own loads per step.
//
// Token slab: 64 token rows of 128 bytes (64 bf16 columns); 16-byte piece p of row t sits in
// slot p ^ slab_swz(t), which keeps the transposing reads of four consecutive rows on distinct
// banks.  One load instruction covers a row group of 8 rows.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int slab_swz(int t) { return ((t >> 1) & 1) << 2; }

// source byte offset of this lane's piece in row group rg (row stride ld elements)
__device__ __forceinline__ int slab_src_off(int rg, int lane, int ld) {
  const int t = 8 * rg + (lane >> 3);
  return (t * ld + ((lane & 7) ^ slab_swz(t)) * 8) * 2;
}

// LDS address of this lane's first transposing read for MFMA operand columns cb .. cb + 31:
// lane (group g, j16) points at row 8 (g >> 1) + j16 / 4, columns cb + 16 (g & 1) + 4 (j16 % 4)
__device__ __forceinline__ uint32_t slab_tr_addr(uint32_t slab, int cb, int lane) {
  const int g = lane >> 4, j16 = lane & 15;
  const int t = 8 * (g >> 1) + (j16 >> 2);
  const int c = cb + 16 * (g & 1) + 4 * (j16 & 3);
  return slab + (uint32_t)(t * 128 + (((c >> 3) ^ slab_swz(t)) * 16) + (c & 7) * 2);
}

// the four K = 16 MFMA operand fragments of a slab (k step s = rows 16 s .., read r = + 4 r rows)
__device__ __forceinline__ void slab_frags(uint32_t addr, bf16x8 (&f)[4]) {
  i16x4 r[8];
  r[0] = lds_read_tr16<0>(addr);
  r[1] = lds_read_tr16<512>(addr);
  r[2] = lds_read_tr16<2048>(addr);
  r[3] = lds_read_tr16<2560>(addr);
  r[4] = lds_read_tr16<4096>(addr);
  r[5] = lds_read_tr16<4608>(addr);
  r[6] = lds_read_tr16<6144>(addr);
  r[7] = lds_read_tr16<6656>(addr);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    f[k] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(r[2 * k], r[2 * k + 1], 0, 1, 2, 3, 4, 5, 6, 7));
}

// s_waitcnt for "this wave's loads of all but the `ahead` (<= A) most recently issued steps",
// PER loads per wave and step
template <int PER, int A>
__device__ __forceinline__ void wait_steps(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      wait_vmcnt<PER * A>();
      return;
    }
    wait_steps<PER, A - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

// the reads above are invisible to the compiler's wait insertion: wait for them, tied to the
// fragments so that no use moves above the wait
__device__ __forceinline__ void lds_wait_frags(bf16x8 (&a)[4], bf16x8 (&b)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
}

// Row tile: 64 rows of 128 bytes holding 64 bf16 along k (an MFMA A operand read as is); 16-byte
// piece p of row t sits in slot p ^ row_swz(t), so the 16 rows one read instruction serves per
// cycle hit distinct banks.  One load instruction covers a row group of 8 rows.
__device__ __forceinline__ int row_swz(int t) { return (t >> 1) & 7; }

__device__ __forceinline__ int row_src_off(int rg, int lane, int ld) {
  const int t = 8 * rg + (lane >> 3);
  return (t * ld + ((lane & 7) ^ row_swz(t)) * 8) * 2;
}

// LDS address of this lane's A fragment of k step s for rows rb .. rb + 31
__device__ __forceinline__ uint32_t row_frag_addr(uint32_t tile, int rb, int lane, int s) {
  const int t = rb + (lane & 31), p = 2 * s + (lane >> 5);
  return tile + (uint32_t)(t * 128 + ((p ^ row_swz(t)) * 16));
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

// N block sums at once (one pair of barriers); each sum as block_sum would form it
template <int N>
__device__ __forceinline__ void block_sums(float (&v)[N], float* scratch /* 4 N floats */) {
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = wave_sum(v[k]);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k < N; ++k) scratch[4 * k + w] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = scratch[4 * k] + scratch[4 * k + 1] + scratch[4 * k + 2] + scratch[4 * k + 3];
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

// ---------------------------------------------------------------------------
// Tile placement over the XCDs
// ---------------------------------------------------------------------------
// Workgroup ids reach the 8 XCDs round-robin, and each XCD has its own L2.  xcd_contiguous lists
// a grid of exactly `total` workgroups so that XCD x takes the x-th contiguous eighth of the list
// (workgroup bid's position in it); the eighths differ by at most one workgroup.
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_contiguous(int bid, int total) {
  const int x = bid % kXcds, base = total / kXcds, extra = total % kXcds;
  return x * base + min(x, extra) + bid / kXcds;
}

// B rows of ntiles tiles each, where the tiles of a row share that row's activation slabs.  With
// 1, 2 or 4 rows, row b takes the 8 / B XCDs [8 b / B, 8 (b + 1) / B), which deal its tiles
// among themselves side by side (the grid padded to whole rounds of 8; the padding workgroups
// are not `valid` and return before any work), so a row's slabs reach 8 / B L2s and the XCDs of a
// row read neighbouring tiles at the same time.  Any other B: the tiles listed row by row and
// dealt in contiguous eighths (xcd_contiguous; the grid exactly B ntiles workgroups), so a row's
// tiles run on one or two XCDs and every XCD gets the same number of tiles within one.
// Measured against rows interleaved over every XCD (1-7 rows) and whole rows per XCD (8 or more):
// config 5 (1-16 rows per chunk step) 1.17-1.18 against 1.22-1.24 s, config 3 (4 rows) 520-521
// against 524 ms, config 2 (8 rows) within run-to-run; the contiguous split at 4 rows took the
// config-3 prefill to 551 ms.
struct RowTile {
  int b, tile;
  bool valid;
};

__device__ __forceinline__ RowTile row_tile(int bid, int B, int ntiles) {
  if (B < kXcds && kXcds % B == 0) {
    const int per = kXcds / B, x = bid % kXcds, tile = (bid / kXcds) * per + x % per;
    return {x / per, tile, tile < ntiles};
  }
  const int q = xcd_contiguous(bid, B * ntiles);
  return {q / ntiles, q % ntiles, true};
}

inline int row_tile_blocks(int B, int ntiles) {
  if (B < kXcds && kXcds % B == 0) return kXcds * ((ntiles + kXcds / B - 1) / (kXcds / B));
  return B * ntiles;
}

}  // namespace uttt
