// The feature map of src/smat/attention.py:82-106 as a device-side stage, shared
// by the stand-alone featurise kernel and the consumers that compute their
// features in place (scan, Gram sums, query):
//
//   Phi = map(Q W^T),  Psi = map(K W^T) * h,  Vb = [V, 1]
//   map = elu(.) + 1   (kind 0)   or   relu(.) + 1e-3   (kind 1)
//
// in the input dtype with torch's rounding steps: the product rounded to the
// dtype, elu rounded, + 1 rounded, the gate product rounded (fp32 math in
// between, as torch does for 16-bit tensors).
#pragma once

#include <type_traits>

#include "smat_common.hpp"

namespace smat {

// expm1(v) for v <= 0 in a few instructions: the degree-6 Taylor polynomial
// on (-0.25, 0] (truncation under 2e-8 relative there) and exp(v) - 1 below,
// where |expm1| > 0.22 and the hardware exp2 keeps the error under 1e-5
// relative.  Rounded to bf16, it equals the correctly rounded expm1 (and the
// fp32 libm expm1f) for every negative bf16 input -- an exhaustive check --
// at a fraction of expm1f's cost, which dominates the feature map's VALU time.
// Both forms are computed and one selected: no divergent branch, so the
// feature map's instructions interleave with the MFMAs around them.  (For
// v > 0 the exp2 form may be inf; callers select v there.)
__device__ __forceinline__ float expm1_neg(float v) {
  float r = 1.f / 720.f;
  r = fmaf(v, r, 1.f / 120.f);
  r = fmaf(v, r, 1.f / 24.f);
  r = fmaf(v, r, 1.f / 6.f);
  r = fmaf(v, r, 0.5f);
  r = fmaf(v, r, 1.f);
  const float near = v * r;
  const float far = __builtin_amdgcn_exp2f(v * 1.4426950408889634f) - 1.f;
  return v > -0.25f ? near : far;
}

// expm1 of a non-positive argument for input type In: the short form where the
// result is rounded to bf16 (where it is exact after rounding, above), libm's
// expm1f for fp16 (whose 11-bit significand the short form's 1e-5 error could
// round differently) and for fp32 (where nothing rounds afterwards).
template <typename In>
__device__ __forceinline__ float expm1_nonpos(float v) {
  if constexpr (std::is_same<In, bf16>::value) return expm1_neg(v);
  else return expm1f(v);
}

template <typename In, int KIND>
__device__ __forceinline__ float feature_map_k(float acc) {
  const float v = to_f32(from_f32<In>(acc));                 // torch's matmul output
  if constexpr (KIND == 0) {
    float e;
    if constexpr (std::is_same<In, bf16>::value) {
      const float m = expm1_neg(v);                            // computed for every lane
      e = to_f32(from_f32<In>(v > 0.f ? v : m));
    } else {
      e = to_f32(from_f32<In>(v > 0.f ? v : expm1_nonpos<In>(v)));
    }
    return to_f32(from_f32<In>(e + 1.0f));
  }
  return to_f32(from_f32<In>(fmaxf(v, 0.f) + 1e-3f));
}

template <typename In>
__device__ __forceinline__ float feature_map(float acc, int kind) {
  return kind == 0 ? feature_map_k<In, 0>(acc) : feature_map_k<In, 1>(acc);
}

// The feature map handed to a consumer kernel: W (128 x 128, features x d_qk,
// row-major, 16-byte aligned rows), the optional key gate h (nb, T) and kind.
struct FeatArgs {
  const void* W;
  const void* h;
  int64_t h_sb;
  int kind;
  // Where a Gram prepass that forms Psi also stores it, rows of 128 at row
  // stride 128 and sequence stride psi_sb (none when null).
  void* psi_out = nullptr;
  int64_t psi_sb = 0;
};

// Features [16 wf, 16 wf + 16) of W as MFMA A fragments over d_qk = 128: k-block
// kb holds k-slots 32 kb + 8 (lane / 16) + j, j < 8.  A per-wave constant.
template <typename In>
__device__ __forceinline__ void feat_w_load(typename Traits<In>::frag (&wa)[4], const In* W, int wf,
                                            int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const In* row = W + (int64_t)(16 * wf + r16) * 128;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    wa[kb] = *reinterpret_cast<const typename Traits<In>::frag*>(row + 32 * kb + 8 * g);
}

// Over NRT 16-row tiles starting at row tile rt0 of LDS tiles of 256-byte
// rows whose 16-byte chunk k of row t sits at slot k ^ swz(t): read the rows'
// 128 input values (X = Q or K) from src, form this wave's features
// C = W[16 wf .. +16] X^T on MFMA (lane (t, g) ends with features 16 wf + 4 g
// .. +3 of row t), then write map(C) (times gate[rt] for the lane's row of tile
// rt0 + rt when use_gate) into the row's feature chunk of dst.  In place
// (dst == src) every wave's reads must precede any write: the call then has a
// barrier between the two, which every wave of the workgroup must meet
// (inactive waves only meet it).  The caller places a barrier before the
// feature rows are read.  The MFMA sequence is the stand-alone kernel's
// (k-blocks 0..3 in order), so the features are bitwise the same.
template <typename In, int NRT, typename Swz>
__device__ __forceinline__ void feat_rows(const uint4* src, uint4* dst, int rt0, bool active,
                                          const typename Traits<In>::frag (&wa)[4], int wf,
                                          int kind, bool use_gate, const float (&gate)[NRT],
                                          int lane, Swz swz) {
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  const int r16 = lane & 15, g = lane >> 4;
  f32x4 acc[NRT];
  if (active) {
    Frag bx[NRT][4];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const int t = 16 * (rt0 + rt) + r16;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        bx[rt][kb] = *reinterpret_cast<const Frag*>(src + t * 16 + ((4 * kb + g) ^ swz(t)));
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      acc[rt] = zero4();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) acc[rt] = mma(acc[rt], wa[kb], bx[rt][kb]);
    }
  }
  if (dst == src) lds_barrier();                     // every wave has read its rows
  // one branch on the (uniform) kind around all of the rows' values
  auto put = [&](auto KC) {
    constexpr int KIND = decltype(KC)::value;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const int t = 16 * (rt0 + rt) + r16;
      Half hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y = feature_map_k<In, KIND>(acc[rt][i]);
        if (use_gate) y = to_f32(from_f32<In>(y * gate[rt]));
        hv[i] = from_f32<In>(y);
      }
      char* p = reinterpret_cast<char*>(dst + t * 16 + ((2 * wf + (g >> 1)) ^ swz(t)));
      *reinterpret_cast<Half*>(p + 8 * (g & 1)) = hv;
    }
  };
  if (active) {
    if (kind == 0)
      put(std::integral_constant<int, 0>{});
    else
      put(std::integral_constant<int, 1>{});
  }
}

// Columns 128..135 of [V, 1] for 64 rows (one 16-byte chunk a row): the ones
// column, then zeros.
template <typename In>
__device__ __forceinline__ void feat_ones_tile(uint4* chunks, int tid, int nthreads) {
  typedef typename Traits<In>::frag Frag;
  for (int t = tid; t < 64; t += nthreads) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = from_f32<In>(j == 0 ? 1.f : 0.f);
    *reinterpret_cast<Frag*>(chunks + t) = f;
  }
}

}  // namespace smat
