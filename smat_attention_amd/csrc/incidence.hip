// Incidence  U_h = sum_{x in H_h} F_x  -- the application of C
// (src/smat/attention.py:239-285; the Triton kernel it replaces is
// src/smat/kernels/triton_fwd.py:162-216).
//
// Pure gather-reduce over fp32 rows of rp = r*p floats.  The design target is
// that every F element crosses HBM once even though each point lies on D
// hyperplanes (D = q+1 for d = 3) and is therefore read D times:
//
//   * work is cut into (batch, element slice) GROUPS; a group's F panel is
//     N0 x kSlice floats (1.7 MB at N0 = 1681) and fits one XCD's 4 MB L2;
//   * workgroups are dispatched round-robin over the 8 XCDs (workgroup L runs
//     on XCD L mod 8), so the flat id is remapped to give each XCD a
//     contiguous run of groups: all the hyperplanes of a group then read the
//     panel from the same L2;
//   * one wave per hyperplane and slice; each lane owns 4 consecutive floats
//     (16-byte loads) and sums its deg rows in registers, in the row order of
//     the table, exactly like the reference's fp32 accumulation.
#include "smat_host.hpp"

namespace smat {

namespace inc {
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSlice = 256;               // floats per wave per hyperplane (64 lanes x 4)
constexpr int kPlanesPerWave = 2;
constexpr int kPlanesPerWG = kWaves * kPlanesPerWave;
constexpr int kXCD = 8;
}  // namespace inc

template <typename Idx, bool Vec>
__global__ __launch_bounds__(inc::kThreads) void incidence_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const Idx* __restrict__ idx,
    const int64_t* __restrict__ indptr, int deg, float* __restrict__ U, int nb, int N0, int B,
    int64_t rp, int nslices, int nhg, int64_t total_wg, int64_t per_xcd) {
  using namespace inc;
  // XCD-aware remap: flat id L runs on XCD L % 8; give XCD x the work items
  // [x * per_xcd, (x+1) * per_xcd).
  const int64_t L = blockIdx.x;
  const int64_t work = (L % kXCD) * per_xcd + L / kXCD;
  if (work >= total_wg) return;
  const int64_t group = work / nhg;          // (b, slice)
  const int hg = (int)(work - group * nhg);
  const int64_t b = group / nslices;
  const int slice = (int)(group - b * nslices);

  const int lane = lane_id(), w = wave_id();
  const int64_t e0 = (int64_t)slice * kSlice + 4 * lane;
  const float* Fb = F + b * (int64_t)N0 * rp;
  const float* Fgb = Fg ? Fg + b * rp : nullptr;
  float* Ub = U + b * (int64_t)B * rp;

#pragma unroll
  for (int k = 0; k < kPlanesPerWave; ++k) {
    const int h = hg * kPlanesPerWG + w * kPlanesPerWave + k;
    if (h >= B) break;
    int64_t lo, hi;
    if (indptr) {
      lo = indptr[h];
      hi = indptr[h + 1];
    } else {
      lo = (int64_t)h * deg;
      hi = lo + deg;
    }
    if (Vec) {
      if (e0 < rp) {   // rp % 4 == 0 on this path, so the 4 floats are in range
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int64_t t = lo; t < hi; ++t) {
          const int64_t x = (int64_t)idx[t];
          const float4 v = *reinterpret_cast<const float4*>(Fb + x * rp + e0);
          acc.x += v.x;
          acc.y += v.y;
          acc.z += v.z;
          acc.w += v.w;
        }
        if (Fgb) {
          const float4 v = *reinterpret_cast<const float4*>(Fgb + e0);
          acc.x += v.x;
          acc.y += v.y;
          acc.z += v.z;
          acc.w += v.w;
        }
        *reinterpret_cast<float4*>(Ub + (int64_t)h * rp + e0) = acc;
      }
    } else {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int64_t t = lo; t < hi; ++t) {
        const int64_t x = (int64_t)idx[t];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (e0 + j < rp) acc[j] += Fb[x * rp + e0 + j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (e0 + j < rp) {
          float v = acc[j];
          if (Fgb) v += Fgb[e0 + j];
          Ub[(int64_t)h * rp + e0 + j] = v;
        }
      }
    }
  }
}

int incidence_dispatch(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                       const int64_t* indptr, int deg, float* U, int nb, int N0, int B, int64_t rp,
                       hipStream_t stream) {
  using namespace inc;
  if (nb == 0 || B == 0 || rp == 0) return SMAT_OK;
  const int nslices = (int)((rp + kSlice - 1) / kSlice);
  const int nhg = (B + kPlanesPerWG - 1) / kPlanesPerWG;
  const int64_t total = (int64_t)nb * nslices * nhg;
  const int64_t per_xcd = (total + kXCD - 1) / kXCD;
  const int64_t grid = per_xcd * kXCD;
  if (grid >= (1ll << 31)) {
    set_error("smat_incidence: problem too large (%lld workgroups)", (long long)grid);
    return SMAT_EUNSUPPORTED;
  }
  const bool vec = (rp % 4 == 0) && aligned16(F) && aligned16(U) && (!F_glob || aligned16(F_glob));
#define SMAT_INC_LAUNCH(IDX, VEC)                                                              \
  hipLaunchKernelGGL((incidence_kernel<IDX, VEC>), dim3((unsigned)grid), dim3(kThreads), 0,    \
                     stream, F, F_glob, (const IDX*)idx, indptr, deg, U, nb, N0, B, rp,        \
                     nslices, nhg, total, per_xcd)
  if (idx_is_64) {
    if (vec) SMAT_INC_LAUNCH(int64_t, true); else SMAT_INC_LAUNCH(int64_t, false);
  } else {
    if (vec) SMAT_INC_LAUNCH(int32_t, true); else SMAT_INC_LAUNCH(int32_t, false);
  }
#undef SMAT_INC_LAUNCH
  return launch_status("smat_incidence");
}

}  // namespace smat

extern "C" int smat_incidence(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                              const int64_t* indptr, int deg, float* U, int nb, int N0, int B,
                              int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && idx && U, SMAT_EINVAL, "smat_incidence: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && B >= 0 && rp >= 0, SMAT_EINVAL, "smat_incidence: bad sizes");
  SMAT_REQUIRE(indptr || deg >= 0, SMAT_EINVAL, "smat_incidence: need indptr or deg >= 0");
  return incidence_dispatch(F, F_glob, idx, idx_is_64, indptr, deg, U, nb, N0, B, rp,
                            (hipStream_t)stream);
}
