// Type-major query  Y[i] = Phi_rec[i] U_{i mod B}  -- the application of R
// (src/smat/attention.py:310-330).
//
// rho(i) = i mod B makes the rows of type h the stride-B progression
// h, h+B, h+2B, ...; one workgroup takes up to 64 of them (four 16-row tiles)
// and one hyperplane's U_h, so U_h is read from HBM exactly once per 64 rows.
// The four waves split U_h's column tiles (wave w: tiles w, w+4, w+8), which
// also means each U element is loaded by exactly one lane.  Phi rows are
// gathered straight into A fragments (8 consecutive features per lane).  U is
// fp32; for 16-bit inputs each U fragment is split into hi + lo 16-bit parts
// (two MFMAs, ~16 mantissa bits), for fp32 inputs it goes to fp32 MFMA whole.
#include "smat_host.hpp"

namespace smat {

namespace qy {
constexpr int kThreads = 256;
constexpr int kRowsPerWG = 64;
constexpr int kMT = kRowsPerWG / 16;
constexpr int kRK = 4;       // r <= 128
constexpr int kNCT = 9;      // p <= 144
constexpr int kCTPerWave = 3;
}  // namespace qy

template <typename In>
__global__ __launch_bounds__(qy::kThreads) void query_kernel(
    const In* __restrict__ phi, const float* __restrict__ U, float* __restrict__ Y, int T_R, int B,
    int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st, int nrb, int vec_q) {
  using namespace qy;
  typedef typename Traits<In>::frag Frag;
  const int h = blockIdx.x / nrb;
  const int rb = blockIdx.x - h * nrb;
  const int64_t b = blockIdx.y;
  const int lane = lane_id(), w = wave_id();
  const int row16 = lane & 15, grp = lane >> 4;
  const int rk = (r + 31) >> 5;
  const int nct = (p + 15) >> 4;
  // rows of type h: i = h + k*B, k < cnt
  const int cnt = (h < T_R) ? (T_R - h + B - 1) / B : 0;
  const int k0 = rb * kRowsPerWG;
  if (k0 >= cnt) return;
  const int nmt = min(kMT, (cnt - k0 + 15) / 16);

  const In* phib = phi + b * q_sb;
  const float* Uh = U + (b * B + h) * (int64_t)r * p;

  f32x4 acc[kMT][kCTPerWave];
#pragma unroll
  for (int t = 0; t < kMT; ++t)
#pragma unroll
    for (int j = 0; j < kCTPerWave; ++j) acc[t][j] = zero4();

#pragma unroll
  for (int kb = 0; kb < kRK; ++kb) {
    if (kb >= rk) continue;
    const int a0 = 32 * kb + 8 * grp;
    Frag pa[kMT];
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
      const int k = k0 + 16 * t + row16;
      const int nv = (t < nmt && k < cnt) ? min(8, r - a0) : 0;
      const int64_t i = (int64_t)h + (int64_t)k * B;
      pa[t] = load8<In>(phib + i * q_st + a0, nv, vec_q);
    }
#pragma unroll
    for (int j = 0; j < kCTPerWave; ++j) {
      const int ct = w + 4 * j;
      if (ct >= nct) continue;
      const int c = ct * 16 + row16;
      float u[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        u[e] = (c < p && a0 + e < r) ? Uh[(int64_t)(a0 + e) * p + c] : 0.f;
      if constexpr (Traits<In>::split) {
        Frag bh, bl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          In hh, ll;
          split2<In>(u[e], hh, ll);
          bh[e] = hh;
          bl[e] = ll;
        }
#pragma unroll
        for (int t = 0; t < kMT; ++t) {
          if (t >= nmt) continue;
          acc[t][j] = mma(acc[t][j], pa[t], bh);
          acc[t][j] = mma(acc[t][j], pa[t], bl);
        }
      } else {
        Frag bf;
#pragma unroll
        for (int e = 0; e < 8; ++e) bf[e] = u[e];
#pragma unroll
        for (int t = 0; t < kMT; ++t) {
          if (t >= nmt) continue;
          acc[t][j] = mma(acc[t][j], pa[t], bf);
        }
      }
    }
  }

  float* Yb = Y + b * y_sb;
#pragma unroll
  for (int t = 0; t < kMT; ++t) {
    if (t >= nmt) continue;
#pragma unroll
    for (int j = 0; j < kCTPerWave; ++j) {
      const int ct = w + 4 * j;
      if (ct >= nct) continue;
      const int c = ct * 16 + row16;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int k = k0 + 16 * t + 4 * grp + i4;
        if (k < cnt && c < p) Yb[((int64_t)h + (int64_t)k * B) * y_st + c] = acc[t][j][i4];
      }
    }
  }
}

template <typename In>
static int launch_query(const void* phi, const float* U, float* Y, int nb, int T_R, int B, int r,
                        int p, int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st,
                        hipStream_t stream) {
  const int maxcnt = (T_R + B - 1) / B;
  const int nrb = (maxcnt + qy::kRowsPerWG - 1) / qy::kRowsPerWG;
  const int64_t gx = (int64_t)B * nrb;
  if (gx >= (1ll << 31)) {
    set_error("smat_query: problem too large");
    return SMAT_EUNSUPPORTED;
  }
  const int vq = rows_vec_ok(phi, q_sb, q_st, sizeof(In));
  hipLaunchKernelGGL(query_kernel<In>, dim3((unsigned)gx, (unsigned)nb), dim3(qy::kThreads), 0,
                     stream, (const In*)phi, U, Y, T_R, B, r, p, q_sb, q_st, y_sb, y_st, nrb, vq);
  return launch_status("smat_query");
}

int query_dispatch(int dtype, const void* phi, const float* U, float* Y, int nb, int T_R, int B,
                   int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st,
                   hipStream_t stream) {
  if (nb == 0 || T_R == 0 || B == 0) return SMAT_OK;
  switch (dtype) {
    case SMAT_BF16:
      return launch_query<bf16>(phi, U, Y, nb, T_R, B, r, p, q_sb, q_st, y_sb, y_st, stream);
    case SMAT_F16:
      return launch_query<f16>(phi, U, Y, nb, T_R, B, r, p, q_sb, q_st, y_sb, y_st, stream);
    case SMAT_F32:
      return launch_query<float>(phi, U, Y, nb, T_R, B, r, p, q_sb, q_st, y_sb, y_st, stream);
  }
  set_error("smat_query: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}

}  // namespace smat

extern "C" int smat_query(int dtype, const void* phi_rec, const float* U, float* Y, int nb,
                          int T_R, int B, int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb,
                          int64_t y_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi_rec && U && Y, SMAT_EINVAL, "smat_query: null pointer");
  SMAT_REQUIRE(nb >= 0 && T_R >= 0 && B >= 1, SMAT_EINVAL, "smat_query: bad sizes");
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_query: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && y_st >= p, SMAT_EINVAL, "smat_query: row stride too short");
  return query_dispatch(dtype, phi_rec, U, Y, nb, T_R, B, r, p, q_sb, q_st, y_sb, y_st,
                        (hipStream_t)stream);
}
