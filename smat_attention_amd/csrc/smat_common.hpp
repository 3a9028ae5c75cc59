// Shared device helpers for the SMat HIP kernels (gfx950 / CDNA4).
//
// MFMA fragment convention used by every kernel in this library
// -------------------------------------------------------------
// All dense contractions use 16x16 output tiles held by one 64-lane wave.
// Lane l has  row16 = l & 15  and  grp = l >> 4  (0..3).
//
//   A fragment (16 x 32 block of an M x K operand): lane l holds the eight
//       values A[row16][kslot(grp, j)], j = 0..7.
//   B fragment (32 x 16 block of a K x N operand): lane l holds the eight
//       values B[kslot(grp, j)][row16], j = 0..7.
//   C tile (16 x 16, fp32): lane l holds C[4*grp + i][row16], i = 0..3.
//
// kslot(grp, j) is any bijection of (grp, j) onto the 32 k indices of the
// block, chosen by the kernel; A and B only have to agree on it, because the
// hardware contracts matching (lane group, element) slots of A and B.  With
// 16-bit inputs one fragment is one v_mfma_f32_16x16x32_{bf16,f16}; with fp32
// inputs it is eight v_mfma_f32_16x16x4_f32, element j feeding instruction j.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smat {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

enum DType { kBF16 = 0, kF16 = 1, kF32 = 2 };

template <typename In> struct Traits;
template <> struct Traits<bf16> {
  typedef bf16x8 frag;
  typedef bf16x4 half_frag;
  static constexpr bool split = true;    // fp32 operands go in as hi + lo
};
template <> struct Traits<f16> {
  typedef f16x8 frag;
  typedef f16x4 half_frag;
  static constexpr bool split = true;
};
template <> struct Traits<float> {
  typedef f32x8 frag;
  typedef float half_frag __attribute__((ext_vector_type(4)));
  static constexpr bool split = false;   // fp32 operands go in whole
};

__device__ __forceinline__ f32x4 mma(f32x4 c, bf16x8 a, bf16x8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f32x4 c, f16x8 a, f16x8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(f32x4 c, f32x8 a, f32x8 b) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }

template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

// hi/lo decomposition of an fp32 value into two 16-bit values with
// hi + lo == x to about 2^-17 relative: the second term carries the bits the
// first one rounded away, so In x fp32 products keep ~16 mantissa bits.
template <typename In>
__device__ __forceinline__ void split2(float x, In& hi, In& lo) {
  hi = from_f32<In>(x);
  lo = from_f32<In>(x - to_f32(hi));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Zero-initialised accumulator.
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Load 8 consecutive elements starting at p (16-bit: 16 B, fp32: 32 B) when the
// whole group is valid and aligned; element-wise with zero fill otherwise.
// `nvalid` counts how many of the 8 are in range (<= 0: none).
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag load8(const In* p, int nvalid, bool vec_ok) {
  typedef typename Traits<In>::frag F;
  F v;
  if (nvalid >= 8 && vec_ok) {
    v = *reinterpret_cast<const F*>(p);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (j < nvalid) ? p[j] : from_f32<In>(0.f);
  }
  return v;
}

}  // namespace smat
