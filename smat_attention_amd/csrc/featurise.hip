// Feature map and value packing, src/smat/attention.py:82-106:
//
//   Phi = map(Q W^T),  Psi = map(K W^T) * h,  Vb = [V, 1]
//   map = elu(.) + 1   ("elu1")   or   relu(.) + 1e-3   ("relu")
//
// in the input dtype with torch's rounding steps: the product rounded to the
// dtype, elu rounded, + 1 rounded, the gate product rounded (fp32 math in
// between, as torch does for 16-bit tensors).
//
// One wave computes a 16-row tile of X (Q or K) against all r features as
// C = W X^T on MFMA (W is the A operand from LDS, rows padded by 16 bytes so
// the sixteen feature rows a fragment reads fall in distinct banks; the X rows
// are the B operand, loaded straight from HBM as 16-byte rows).  Each lane
// then holds four consecutive features of one row and stores them as one
// 8-byte (16-bit types) or 16-byte (fp32) write.  The [V, 1] rows are copied
// by the same launch.  HBM-bound: 2 (T d_qk + T r) + T (d_v + p) elements per
// sequence.
#include <math.h>

#include "feat_map.hpp"
#include "smat_host.hpp"

namespace smat {

namespace ft {
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxDqk = 128;       // d_qk
constexpr int kMaxRank = 128;      // feature rank
}  // namespace ft

template <typename In>
__global__ __launch_bounds__(ft::kThreads) void featurise_kernel(
    const In* __restrict__ q, const In* __restrict__ k, const In* __restrict__ v,
    const In* __restrict__ W, const In* __restrict__ h, In* __restrict__ phi,
    In* __restrict__ psi, In* __restrict__ vb, int nb, int T, int dqk, int r, int dv, int kind,
    int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
    int64_t h_sb, int64_t o_sb, int64_t o_st, int64_t vb_sb, int64_t vb_st, int64_t ntiles,
    int vec) {
  // vec: bit 0 = Q/K rows and W 16-byte aligned (vector loads), bit 1 = Phi/Psi
  // rows aligned to four elements (one store per lane and tile), bit 2 = V and
  // Vb rows 16-byte aligned.
  using namespace ft;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Quad;
  constexpr int kE = 16 / (int)sizeof(In);                   // elements per 16 bytes
  constexpr int kWst = kMaxDqk + kE;                           // padded W row (elements)
  __shared__ __attribute__((aligned(16))) In w_lds[kMaxRank * kWst];

  // W (r x dqk) -> LDS, zero beyond r and dqk
  for (int i = threadIdx.x; i < kMaxRank * (kMaxDqk / kE); i += kThreads) {
    const int f = i / (kMaxDqk / kE), c = (i - f * (kMaxDqk / kE)) * kE;
    In tmp[kE];
    if ((vec & 1) && f < r && c + kE <= dqk) {
      *reinterpret_cast<uint4*>(tmp) = *reinterpret_cast<const uint4*>(W + (int64_t)f * dqk + c);
    } else {
#pragma unroll
      for (int e = 0; e < kE; ++e)
        tmp[e] = (f < r && c + e < dqk) ? W[(int64_t)f * dqk + c + e] : from_f32<In>(0.f);
    }
    *reinterpret_cast<uint4*>(w_lds + f * kWst + c) = *reinterpret_cast<const uint4*>(tmp);
  }
  __syncthreads();

  const int lane = lane_id();
  const int r16 = lane & 15, grp = lane >> 4;
  const int64_t tiles_per = (int64_t)nb * ((T + 15) / 16);
  const int nks = (dqk + 31) / 32;
  const int nft = (r + 15) / 16;
  const int64_t gwave = (int64_t)blockIdx.x * kWaves + wave_id();
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;

  for (int64_t tile = gwave; tile < ntiles; tile += nwaves) {
    const int which = (int)(tile / tiles_per);               // 0: Q, 1: K, 2: V
    const int64_t rem = tile - which * tiles_per;
    const int64_t b = rem / ((T + 15) / 16);
    const int t0 = (int)(rem - b * ((T + 15) / 16)) * 16;
    const int row = t0 + r16;
    const bool live = row < T;
    if ((which == 1 && !k) || (which == 2 && !v)) continue;   // wave-uniform
    if (which == 2) {
      // [V, 1]: lane r16 copies row t0 + r16 in chunks of kE, four lanes per row
      if (live) {
        const In* src = v + b * v_sb + (int64_t)row * v_st;
        In* dst = vb + b * vb_sb + (int64_t)row * vb_st;
        for (int c = grp; c * kE < dv + 1; c += 4) {
          if ((vec & 4) && (c + 1) * kE <= dv) {
            *reinterpret_cast<uint4*>(dst + c * kE) = *reinterpret_cast<const uint4*>(src + c * kE);
          } else {
#pragma unroll
            for (int e = 0; e < kE; ++e) {
              const int col = c * kE + e;
              if (col < dv) dst[col] = src[col];
              else if (col == dv) dst[col] = from_f32<In>(1.f);
            }
          }
        }
      }
      continue;
    }
    const In* X = (which == 0 ? q + b * q_sb : k + b * k_sb);
    const int64_t x_st = which == 0 ? q_st : k_st;
    // B operand: row r16 of the tile, k-slots 32 ks + 8 grp .. + 8
    Frag xb[kMaxDqk / 32];
    const In* xr = X + (int64_t)(live ? row : t0) * x_st;
#pragma unroll
    for (int ks = 0; ks < kMaxDqk / 32; ++ks) {
      if (ks < nks) {
        const int c0 = 32 * ks + 8 * grp;
        if ((vec & 1) && c0 + 8 <= dqk) {
          xb[ks] = *reinterpret_cast<const Frag*>(xr + c0);
          if (!live) xb[ks] = Frag{};
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            xb[ks][e] = (live && c0 + e < dqk) ? xr[c0 + e] : from_f32<In>(0.f);
        }
      }
    }
    float hv = 1.f;
    if (which == 1 && h) hv = live ? to_f32(h[b * h_sb + row]) : 0.f;
    In* O = (which == 0 ? phi : psi) + b * o_sb + (int64_t)row * o_st;
#pragma unroll 1
    for (int f = 0; f < nft; ++f) {
      f32x4 acc = zero4();
#pragma unroll
      for (int ks = 0; ks < kMaxDqk / 32; ++ks) {
        if (ks < nks) {
          Frag wa;
          const In* wp = w_lds + (16 * f + r16) * kWst + 32 * ks + 8 * grp;
#pragma unroll
          for (int e = 0; e < 8; ++e) wa[e] = wp[e];
          acc = mma(acc, wa, xb[ks]);
        }
      }
      if (live) {
        const int c0 = 16 * f + 4 * grp;
        Quad outv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float y = feature_map<In>(acc[i], kind);
          if (which == 1 && h) y = to_f32(from_f32<In>(y * hv));
          outv[i] = from_f32<In>(y);
        }
        if ((vec & 2) && c0 + 3 < r) {
          *reinterpret_cast<Quad*>(O + c0) = outv;
        } else if (c0 + 3 < r) {
#pragma unroll
          for (int i = 0; i < 4; ++i) O[c0 + i] = outv[i];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (c0 + i < r) O[c0 + i] = outv[i];
        }
      }
    }
  }
}

}  // namespace smat

extern "C" int smat_featurise(int dtype, const void* q, const void* k, const void* v,
                              const void* W, const void* h, void* phi, void* psi, void* vb,
                              int nb, int T, int d_qk, int r, int d_v, int kind, int64_t q_sb,
                              int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                              int64_t v_st, int64_t h_sb, int64_t o_sb, int64_t o_st,
                              int64_t vb_sb, int64_t vb_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(q && W && phi, SMAT_EINVAL, "smat_featurise: null pointer");
  SMAT_REQUIRE((!k || psi) && (!v || vb), SMAT_EINVAL, "smat_featurise: k given without psi, or v "
               "without vb");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && d_qk >= 1 && r >= 1 && d_v >= 0, SMAT_EINVAL,
               "smat_featurise: bad sizes");
  SMAT_REQUIRE(d_qk <= ft::kMaxDqk && r <= ft::kMaxRank, SMAT_EUNSUPPORTED,
               "smat_featurise: d_qk=%d r=%d beyond d_qk<=%d, r<=%d", d_qk, r, ft::kMaxDqk,
               ft::kMaxRank);
  SMAT_REQUIRE(kind == 0 || kind == 1, SMAT_EINVAL, "smat_featurise: kind must be 0 (elu1) or 1 "
               "(relu)");
  SMAT_REQUIRE(q_st >= d_qk && (!k || k_st >= d_qk) && (!v || (v_st >= d_v && vb_st > d_v)) &&
                   o_st >= r,
               SMAT_EINVAL, "smat_featurise: row stride too short");
  if (nb == 0 || T == 0) return SMAT_OK;
  const int64_t ntiles = 3 * (int64_t)nb * ((T + 15) / 16);
  const int64_t e16 = 16 / elem_bytes(dtype);
  if (!k) { k = q; k_sb = q_sb; k_st = q_st; psi = phi; }      // alignment checks only
  if (!v) { v = q; vb = phi; v_st = d_v; vb_st = d_v + 1; v_sb = vb_sb = 0; }
  const bool have_k = k != q || psi != phi, have_v = vb != phi;
  const int vec = ((aligned16(q) && aligned16(k) && aligned16(W) && q_st % e16 == 0 &&
                    k_st % e16 == 0 && q_sb % e16 == 0 && k_sb % e16 == 0 && d_qk % e16 == 0)
                       ? 1 : 0) |
                  ((((uintptr_t)phi | (uintptr_t)psi) % (4 * elem_bytes(dtype)) == 0 &&
                    o_st % 4 == 0 && o_sb % 4 == 0) ? 2 : 0) |
                  ((aligned16(v) && aligned16(vb) && v_st % e16 == 0 && v_sb % e16 == 0 &&
                    vb_st % e16 == 0 && vb_sb % e16 == 0) ? 4 : 0);
  int dev = 0, ncu = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t want = (ntiles + ft::kWaves - 1) / ft::kWaves;
  const unsigned grid = (unsigned)std::min<int64_t>(want, (int64_t)ncu * 8);
  hipStream_t st = (hipStream_t)stream;
  const void* kk = have_k ? k : nullptr;
  const void* vv = have_v ? v : nullptr;
#define SMAT_FT(T_)                                                                            \
  smat::launch(featurise_kernel<T_>, dim3(grid), dim3(ft::kThreads), 0, st, (const T_*)q, \
                     (const T_*)kk, (const T_*)vv, (const T_*)W, (const T_*)h, (T_*)phi, (T_*)psi, \
                     (T_*)vb, nb, T, d_qk, r, d_v, kind, q_sb, q_st, k_sb, k_st, v_sb, v_st,     \
                     h_sb, o_sb, o_st, vb_sb, vb_st, ntiles, vec)
  switch (dtype) {
    case SMAT_BF16: SMAT_FT(bf16); break;
    case SMAT_F16: SMAT_FT(f16); break;
    case SMAT_F32: SMAT_FT(float); break;
    default:
      set_error("smat_featurise: unknown dtype %d", dtype);
      return SMAT_EINVAL;
  }
#undef SMAT_FT
  return launch_status("smat_featurise");
}
