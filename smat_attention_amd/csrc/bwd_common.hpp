// Fragment helpers of the backward kernels at r = 64 features and p = 65
// value columns (head_dim 64 plus the ones column) on gfx950 MFMA
// (v_mfma_f32_16x16x32 for 16-bit inputs, 16x16x16 for the K = 16 tail over
// value columns 64..79, of which only 64 exists).
//
// LDS layouts: 16-bit tiles of 64 columns as rows of 128 bytes, 16-byte
// chunk k of row t at k ^ (t & 6) -- conflict-free for row-wise 16-byte reads
// (four phases of 16 lanes) and for the transposing ds_read_b64_tr_b16 (two
// phases of 32 lanes); fp32 tiles as rows of kS = 68 floats.
#pragma once

#include "smat_host.hpp"

namespace smat {

namespace cb {

// The (item, sequence) of this workgroup of a (nitems, nseq) grid, with all the
// items of a sequence on one XCD: workgroups are dispatched to the 8 XCDs
// round-robin by linear id, so XCD x takes sequences x, x + 8, ... in turn
// and the rows its items share (a token in several cells' or points' lists)
// are re-read from that XCD's L2 instead of from HBM.  Sequences past the
// last multiple of 8 keep the plain mapping.
__device__ __forceinline__ void xcd_item_seq(int& item, int64_t& seq) {
  const int64_t nitems = gridDim.x, nseq = gridDim.y;
  const int64_t lin = (int64_t)blockIdx.y * nitems + blockIdx.x;
  const int64_t full = (nseq / 8) * 8 * nitems;
  if (lin < full) {
    const int64_t k = lin >> 3;
    seq = (lin & 7) + 8 * (k / nitems);
    item = (int)(k % nitems);
  } else {
    seq = lin / nitems;
    item = (int)(lin % nitems);
  }
}

constexpr int kC = 128;          // tokens per chunk
constexpr int kR = 64;           // features
constexpr int kP = 65;           // value columns incl. the ones column
constexpr int kThreads = 512;
constexpr int kS = 68;           // fp32 LDS row stride (floats)
constexpr int kRowChunks = 8;    // 16-byte chunks per 16-bit row of 64
}  // namespace cb

__device__ __forceinline__ f32x4 mma_k16(f32x4 c, bf16x4 a, bf16x4 b) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a),
                                                   __builtin_bit_cast(s4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma_k16(f32x4 c, f16x4 a, f16x4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// 16-byte chunk slot of (row, chunk) in a 128-row x 128-byte tile.
__device__ __forceinline__ int cb_slot(int row, int k) { return row * cb::kRowChunks + (k ^ (row & 6)); }

template <typename In>
__device__ __forceinline__ typename Traits<In>::half_frag cb_tr(const uint4* tile, int row, int k,
                                                                int half) {
  typedef short short4v __attribute__((ext_vector_type(4)));
  const char* p = reinterpret_cast<const char*>(tile + cb_slot(row, k)) + 8 * half;
  short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v*)(__attribute__((address_space(3))) char*)(p));
  return __builtin_bit_cast(typename Traits<In>::half_frag, v);
}

// The A operand along tokens of a transposed 16-bit tile (Phi^T or Psi^T):
// lane (m = 16 ct + lane % 16, g) gets, as k-slot 4h + e, column m of token
// row 16 tile[h] + 4g + e.  Lane 4e + q of each sixteen addresses row
// 16 tile[h] + 4g + e, columns 16 ct + 4q .. +3.
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag cb_tr_pair(const uint4* tile, int t0, int t1,
                                                               int ct, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  const int k = 2 * ct + ((r16 & 3) >> 1), half = r16 & 1;
  const auto a = cb_tr<In>(tile, 16 * t0 + 4 * g + (r16 >> 2), k, half);
  const auto b = cb_tr<In>(tile, 16 * t1 + 4 * g + (r16 >> 2), k, half);
  typename Traits<In>::frag f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
  return f;
}

// Row-wise operand of a 16-bit tile: lane (row 16 tile + lane % 16, g) gets
// columns 32 kc + 8g .. +7.
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag cb_row(const uint4* tile, int tile_row, int kc,
                                                           int lane) {
  return *reinterpret_cast<const typename Traits<In>::frag*>(
      tile + cb_slot(16 * tile_row + (lane & 15), 4 * kc + (lane >> 4)));
}

// Row-wise operand of an fp32 LDS tile (rows of kS floats), split hi/lo:
// lane (row, g) gets columns 32 kc + 8g .. +7.
template <typename In>
__device__ __forceinline__ void cb_row32(const float* t, int row, int kc, int g,
                                         typename Traits<In>::frag& hi,
                                         typename Traits<In>::frag& lo) {
  const float4 a = *reinterpret_cast<const float4*>(t + row * cb::kS + 32 * kc + 8 * g);
  const float4 b = *reinterpret_cast<const float4*>(t + row * cb::kS + 32 * kc + 8 * g + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    In h, l;
    split2<In>(v[e], h, l);
    hi[e] = h;
    lo[e] = l;
  }
}

// The K = 16 tail over value columns 64..79 of an fp32 LDS tile: only column
// 64 exists, k-slot 0 of lane group 0.
template <typename In>
__device__ __forceinline__ void cb_tail32(const float* t, int row, int g,
                                          typename Traits<In>::half_frag& hi,
                                          typename Traits<In>::half_frag& lo) {
  const float v = g == 0 ? t[row * cb::kS + 64] : 0.f;
  In h, l;
  split2<In>(v, h, l);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = from_f32<In>(0.f);
    lo[e] = from_f32<In>(0.f);
  }
  hi[0] = h;
  lo[0] = l;
}

// hi/lo 16-bit B operand from two accumulator tiles (k-slot 4h + e <- tile h, entry e).
template <typename In>
__device__ __forceinline__ void cb_split_pair(const f32x4& a, const f32x4& b,
                                              typename Traits<In>::frag& hi,
                                              typename Traits<In>::frag& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    In h, l;
    split2<In>(a[e], h, l);
    hi[e] = h;
    lo[e] = l;
    split2<In>(b[e], h, l);
    hi[4 + e] = h;
    lo[4 + e] = l;
  }
}

// Stage one contiguous r x p fp32 matrix (16-byte aligned) in LDS rows of kS,
// all threads of the workgroup.
__device__ __forceinline__ void cb_stage_rp(float* s, const float* src) {
  using namespace cb;
  for (int f = threadIdx.x; f < (cb::kR * cb::kP) / 4; f += (int)blockDim.x) {
    const float4 v = reinterpret_cast<const float4*>(src)[f];
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * f + q;
      const int row = e / kP, col = e - row * kP;
      s[row * kS + col] = vv[q];
    }
  }
}

// Gradient rows leave as fp32 or rounded (to nearest even) to the inputs'
// 16-bit type.  Four consecutive values: one 16-byte store of floats, or one
// 8-byte store of 16-bit values (rows 16-byte aligned, the group at a column
// that is a multiple of 4).
__device__ __forceinline__ void store_grad4(float* p, const f32x4& v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <typename Out>
__device__ __forceinline__ void store_grad4(Out* p, const f32x4& v) {
  typename Traits<Out>::half_frag h;
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = from_f32<Out>(v[i]);
  *reinterpret_cast<typename Traits<Out>::half_frag*>(p) = h;
}
// The code of a gradient output type, as the host entry points take it.
template <typename Out> constexpr int out_code();
template <> constexpr int out_code<float>() { return SMAT_F32; }
template <> constexpr int out_code<bf16>() { return SMAT_BF16; }
template <> constexpr int out_code<f16>() { return SMAT_F16; }

// Sum over the four 16-lane groups of a wave (lanes r16, r16 + 16, +32, +48).
__device__ __forceinline__ float cb_sum_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// One step's gather: 32 entries, eight threads per entry (slot = tid / 8,
// sub = tid % 8).  A thread loads its entry's id once, then a 16-byte piece of
// the 64-wide 16-bit row (columns 8 sub .. +7) and every eighth element of the
// 65-wide row (columns sub + 8u).  Loads land in registers and the kernel
// writes them to LDS at the top of the step.  Issuing the next step's gather
// before the current step's products overlaps its two dependent latencies
// (entry id, then rows) with them.  The per-entry token, pair and dot
// partials are read after the step's last barrier, so they alternate
// between two buffers by step parity while the next step's rows are written.
template <typename In, typename Row65>
struct CbGather {
  static constexpr int kU = 9;                 // ceil(65 / 8)
  int tok, pair;
  bool ok;
  uint4 r64;
  Row65 r65[kU];
  // Entry ids are pair-major, pair * L + token (L tokens a sequence), so each
  // cell's list holds its pair-0 entries first.
  __device__ __forceinline__ void load(const int32_t* ent, int64_t s0, int64_t beg, int64_t end,
                                       int L, const In* rows64, int64_t st64, const Row65* rows65,
                                       int64_t st65, int tid) {
    const int slot = tid >> 3, sub = tid & 7;
    ok = s0 + slot < end;
    const int e = ent[ok ? s0 + slot : beg];
    pair = (int)((unsigned)e / (unsigned)L);
    tok = e - pair * L;
    r64 = *reinterpret_cast<const uint4*>(rows64 + (int64_t)tok * st64 + 8 * sub);
    const Row65* r = rows65 + (int64_t)tok * st65;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int col = sub + 8 * u;
      r65[u] = r[col < cb::kP ? col : 0];
    }
  }
};

}  // namespace smat
