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

// split2 of four values into half fragments.  For bf16 each pair of values
// takes one conversion for both hi parts (v_cvt_pk_bf16_f32) and reads them
// back as fp32 by shifting; the results are split2's, value by value.
template <typename In>
__device__ __forceinline__ void split4(const f32x4& x, typename Traits<In>::half_frag& hi,
                                       typename Traits<In>::half_frag& lo) {
  if constexpr (__is_same(In, bf16)) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x2 v = {x[2 * q], x[2 * q + 1]};
      const bf16x2 h = __builtin_convertvector(v, bf16x2);
      const unsigned u = __builtin_bit_cast(unsigned, h);
      const f32x2 back = {__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u)};
      const bf16x2 l = __builtin_convertvector(v - back, bf16x2);
      hi[2 * q] = h[0];
      hi[2 * q + 1] = h[1];
      lo[2 * q] = l[0];
      lo[2 * q + 1] = l[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      In h, l;
      split2<In>(x[i], h, l);
      hi[i] = h;
      lo[i] = l;
    }
  }
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

namespace smat {

// ---------------------------------------------------------------------------
// Staging a token-major tile into LDS transposed (feature-major), 8 x 8 at a
// time: a thread loads 8 token rows x 8 consecutive columns with 16-byte (or
// 32-byte for fp32) reads, transposes the 8 x 8 block in registers and writes
// 8 column runs of 8 tokens with 16-byte (32-byte) LDS stores.  This replaces
// per-element global loads and per-element transposed LDS writes.
// ---------------------------------------------------------------------------

template <typename In>
struct Tile8 {
  typename Traits<In>::frag row[8];   // row[t] = columns c0..c0+7 of token t
  unsigned live;                      // bit t: row t holds data (tile8_issue)
  int nv;                             // valid columns (tile8_issue)
};

// Split form of tile8_load<In, true> for prefetching: tile8_issue only starts
// the eight vector loads (nothing reads their results, so nothing waits for
// them); tile8_finish, called when the data is needed, zeroes padding rows and
// columns.  Same addresses, same bounds argument as tile8_load.
template <typename In>
__device__ __forceinline__ void tile8_issue(Tile8<In>& tl, const In* const* rowp, const In* safe,
                                            int c0, int ncols) {
  typedef typename Traits<In>::frag F;
  tl.nv = ncols - c0;
  tl.live = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const bool live = rowp[t] != nullptr && tl.nv > 0;
    tl.live |= live ? (1u << t) : 0u;
    tl.row[t] = *reinterpret_cast<const F*>(live ? rowp[t] + c0 : safe);
  }
}

template <typename In>
__device__ __forceinline__ void tile8_finish(Tile8<In>& tl) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const bool live = (tl.live >> t) & 1u;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      tl.row[t][j] = (live && j < tl.nv) ? tl.row[t][j] : from_f32<In>(0.f);
  }
}

// Load rows tok(0..7) x columns [c0, c0+8) of a row-major matrix; `rowp[t]` is
// the row start of token t (nullptr: a padding token, loaded as zeros).
// Columns >= ncols load as zeros.
//
// VEC (rows 16-byte aligned, row stride a multiple of 8 elements): branch-free.
// Every row is read with one 16-byte (fp32: 32-byte) load -- a padding row,
// or a tile starting at or past column ncols, from `safe` (the start of any
// valid row of the same matrix) -- and the padding rows and columns are then
// zeroed with selects.  A live read covers [c0, c0+8) with c0 < ncols and c0 a
// multiple of 8, so it ends at or before round_up(ncols, 8), which is at most
// the row stride because VEC is taken only for strides that are multiples of 8
// elements (rows_vec8_ok; for fp32 a stride of 4 mod 8 floats would not do):
// no read leaves its row, hence none leaves the allocation.  Branches around loads make the
// compiler wait for every outstanding load where they join, which would
// serialise the staging; this form keeps all eight loads in flight.
// !VEC: element-wise loads with zero fill.
template <typename In, bool VEC>
__device__ __forceinline__ void tile8_load(Tile8<In>& tl, const In* const* rowp, const In* safe,
                                           int c0, int ncols) {
  typedef typename Traits<In>::frag F;
  const int nv = ncols - c0;
  if constexpr (VEC) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // A tile wholly past the last column (nv <= 0) or a padding row reads
      // `safe` at column 0 instead: c0 + 8 may exceed the row stride there.
      const bool live = rowp[t] != nullptr && nv > 0;
      const In* src = live ? rowp[t] + c0 : safe;
      F v = *reinterpret_cast<const F*>(src);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (live && j < nv) ? v[j] : from_f32<In>(0.f);
      tl.row[t] = v;
    }
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        tl.row[t][j] = (rowp[t] != nullptr && j < nv) ? rowp[t][c0 + j] : from_f32<In>(0.f);
    }
  }
}

// Eight consecutive elements at p; elements j >= nvalid read as zero.  VEC as
// for tile8_load: one vector load from p when the row is valid, else from
// `safe`, then selects.
template <typename In, bool VEC>
__device__ __forceinline__ typename Traits<In>::frag load8v(const In* p, const In* safe,
                                                            int nvalid) {
  typedef typename Traits<In>::frag F;
  F v;
  if constexpr (VEC) {
    v = *reinterpret_cast<const F*>(nvalid > 0 ? p : safe);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (j < nvalid) ? v[j] : from_f32<In>(0.f);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (j < nvalid) ? p[j] : from_f32<In>(0.f);
  }
  return v;
}

// Write the transpose: dst[(c0 + j) * ld + t0 .. + 8] = column j of the tile.
template <typename In>
__device__ __forceinline__ void tile8_store_T(const Tile8<In>& tl, In* dst, int ld, int c0,
                                              int t0) {
  typedef typename Traits<In>::frag F;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    F col;
#pragma unroll
    for (int t = 0; t < 8; ++t) col[t] = tl.row[t][j];
    *reinterpret_cast<F*>(dst + (c0 + j) * ld + t0) = col;
  }
}

// Write the tile as is: dst[(t0 + t) * ld + c0 .. + 8] = row t.
template <typename In>
__device__ __forceinline__ void tile8_store(const Tile8<In>& tl, In* dst, int ld, int c0, int t0) {
  typedef typename Traits<In>::frag F;
#pragma unroll
  for (int t = 0; t < 8; ++t) *reinterpret_cast<F*>(dst + (t0 + t) * ld + c0) = tl.row[t];
}

}  // namespace smat

namespace smat {

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (vmcnt(0)), which would
// drain the prefetches the kernels keep in flight across a barrier; here the
// wave waits for its own LDS operations (lgkmcnt(0)) and then meets the
// others, which is all that LDS producer/consumer hand-offs need.  Global data
// loaded into registers is still waited for by the compiler at its first use.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until at most N vector memory operations of the wave are outstanding
// (loads and stores complete in the order they were issued).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One HBM -> LDS copy of 16 bytes a lane (global_load_lds_dwordx4: lane i
// writes bytes [16 i, 16 i + 16) from dst, a wave-uniform LDS address).
// UNTRACKED issues it from inline assembly, so the compiler does not know that
// an LDS write is in flight.  Tracked, every LDS read it cannot tell apart from
// the copy's target -- the transposing reads among them -- gets a compiler
// wait of vmcnt(0) in front, which drains the copies issued ahead and leaves
// nothing to overlap with the compute.  Untracked, the kernel's own vmcnt
// waits and barriers are what order each read after the copy it reads; loads
// the compiler does track must then not be pending across such a copy, or
// their compiler waits (counting only tracked loads) drain it as well.  m0
// (the LDS address) is saved and restored around the copy: the compiler
// reserves it and may keep a value of its own there.
template <bool UNTRACKED>
__device__ __forceinline__ void lds_dma16(const void* src, void* dst) {
  typedef __attribute__((address_space(3))) char lds_char;
  if constexpr (UNTRACKED) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_char*)(dst));
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(keep)
        : "v"(src), "s"(m0)
        : "memory");
  } else {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds_char*)(dst),
                                     16, 0, 0);
  }
}

}  // namespace smat
