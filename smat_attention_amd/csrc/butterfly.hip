// Power-of-two butterflies over the profile axis of pooled tables, and the
// complement used by the subtractive schedule:
//
//   zeta  (Z_k F)_a = sum_{x subset of a} F_x          (src/smat/attention.py:369-384)
//   walsh U = (tot + H F) / 2, H the Walsh matrix      (src/smat/attention.py:288-307)
//         -- the endpoint mask's incidence C[h, a] = 1{popcount(h & a) even}
//   complement  U_h <- U_h - sum_x F_x                 (src/smat/attention.py:458-482,
//         negated: the query of the result is -Y_ex, added where the
//         reference subtracts)
//
// F is (nb, N, rp) fp32, N = 2^k.  The butterflies work on slices of E
// floats of every profile held in LDS: one workgroup stages its N x E panel,
// runs the k stages in place (a barrier between stages) and writes the
// panel back -- HBM is crossed once in each direction.  Panels too large for
// LDS run one global pass per stage instead.  Stage j pairs x and x | 2^j
// (bit j of x clear), as the reference's reshape (N / 2^{j+1}, 2, 2^j) does.
#include <stdlib.h>

#include "smat_host.hpp"

namespace smat {

namespace bfy {
constexpr int kThreads = 1024;
constexpr int kLdsBudget = 150 * 1024;
}  // namespace bfy

__device__ __forceinline__ void bf_pair(float4& a, float4& b, int mode) {
  if (mode == 0) {                      // zeta: b += a
    b.x += a.x;
    b.y += a.y;
    b.z += a.z;
    b.w += a.w;
  } else {                              // walsh: (a, b) <- (a + b, a - b)
    const float4 s = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    const float4 d = make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w);
    a = s;
    b = d;
  }
}

// One workgroup per (batch, slice of E = 4*Q floats); mode 0 zeta, 1 walsh.
template <int Q>
__global__ __launch_bounds__(bfy::kThreads) void butterfly_lds_kernel(
    const float* __restrict__ X, float* __restrict__ Y, int N, int logN, int64_t rp,
    int nslices, int mode) {
  extern __shared__ float4 pan[];
  const int64_t b = blockIdx.x / nslices;
  const int slice = (int)(blockIdx.x - b * nslices);
  const int64_t e0 = (int64_t)slice * 4 * Q;
  const float* Xb = X + b * (int64_t)N * rp + e0;
  float* Yb = Y + b * (int64_t)N * rp + e0;
  for (int i = threadIdx.x; i < N * Q; i += bfy::kThreads) {
    const int x = i / Q, k = i - x * Q;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + 4 * k < rp) v = *reinterpret_cast<const float4*>(Xb + (int64_t)x * rp + 4 * k);
    pan[i] = v;
  }
  __syncthreads();
  const int half = N >> 1;
  for (int j = 0; j < logN; ++j) {
    const int lo = 1 << j;
    for (int i = threadIdx.x; i < half * Q; i += bfy::kThreads) {
      const int pr = i / Q, k = i - pr * Q;
      const int x = ((pr >> j) << (j + 1)) | (pr & (lo - 1));     // bit j clear
      float4 a = pan[x * Q + k], c = pan[(x | lo) * Q + k];
      bf_pair(a, c, mode);
      pan[x * Q + k] = a;
      pan[(x | lo) * Q + k] = c;
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < N * Q; i += bfy::kThreads) {
    const int x = i / Q, k = i - x * Q;
    if (e0 + 4 * k >= rp) continue;
    float4 v = pan[i];
    if (mode == 1) {                    // U_h = (H F)_0 / 2 + (H F)_h / 2
      const float4 t = pan[k];
      v = make_float4(0.5f * (t.x + v.x), 0.5f * (t.y + v.y), 0.5f * (t.z + v.z),
                      0.5f * (t.w + v.w));
    }
    *reinterpret_cast<float4*>(Yb + (int64_t)x * rp + 4 * k) = v;
  }
}

// Global fallback: one stage over all pairs, in place on Y (float4 elements).
__global__ __launch_bounds__(256) void butterfly_pass_kernel(float* __restrict__ Y, int N, int j,
                                                             int64_t rp4, int64_t npairs,
                                                             int mode) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= npairs) return;
  const int64_t e = i % rp4;
  const int64_t rest = i / rp4;
  const int64_t pr = rest % (N >> 1);
  const int64_t b = rest / (N >> 1);
  const int64_t lo = 1ll << j;
  const int64_t x = ((pr >> j) << (j + 1)) | (pr & (lo - 1));
  float4* Yb = reinterpret_cast<float4*>(Y) + b * N * rp4;
  float4 a = Yb[x * rp4 + e], c = Yb[(x | lo) * rp4 + e];
  bf_pair(a, c, mode);
  Yb[x * rp4 + e] = a;
  Yb[(x | lo) * rp4 + e] = c;
}

// Walsh fallback finish: U_h = ((H F)_0 + (H F)_h) / 2, h >= 1 first, then h = 0.
__global__ __launch_bounds__(256) void walsh_finish_kernel(float* __restrict__ Y, int N,
                                                           int64_t rp4, int64_t total, int row0) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t e = i % rp4;
  const int64_t rest = i / rp4;
  const int64_t h = row0 ? 0 : 1 + rest % (N - 1);
  const int64_t b = row0 ? rest : rest / (N - 1);
  float4* Yb = reinterpret_cast<float4*>(Y) + b * N * rp4;
  const float4 t = Yb[e];
  float4 v = Yb[h * rp4 + e];
  v = make_float4(0.5f * (t.x + v.x), 0.5f * (t.y + v.y), 0.5f * (t.z + v.z),
                  0.5f * (t.w + v.w));
  Yb[h * rp4 + e] = v;
}

static int butterfly_dispatch(const float* X, float* Y, int nb, int N, int64_t rp, int mode,
                              hipStream_t stream, const char* who) {
  if (nb == 0 || N == 0 || rp == 0) return SMAT_OK;
  int logN = 0;
  while ((1 << logN) < N) ++logN;
  if ((1 << logN) != N) {
    set_error("%s: N=%d is not a power of two", who, N);
    return SMAT_EINVAL;
  }
  if (rp % 4 || !aligned16(X) || !aligned16(Y)) {
    set_error("%s: needs rp %% 4 == 0 and 16-byte aligned tables (rp=%lld)", who, (long long)rp);
    return SMAT_EUNSUPPORTED;
  }
  for (int Q : {4, 2, 1}) {
    const size_t smem = (size_t)N * Q * 16;
    if (smem > (size_t)bfy::kLdsBudget) continue;
    const int nslices = (int)((rp + 4 * Q - 1) / (4 * Q));
    const int64_t grid = (int64_t)nb * nslices;
    if (grid >= (1ll << 31)) break;
#define SMAT_BFY(QQ)                                                                           \
  {                                                                                            \
    auto kern = butterfly_lds_kernel<QQ>;                                                      \
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                              bfy::kLdsBudget);                                                \
    smat::launch(kern, dim3((unsigned)grid), dim3(bfy::kThreads), smem, stream, X, Y, N, \
                       logN, rp, nslices, mode);                                               \
  }
    if (Q == 4) SMAT_BFY(4) else if (Q == 2) SMAT_BFY(2) else SMAT_BFY(1)
#undef SMAT_BFY
    return launch_status(who);
  }
  // global passes (large N): copy X to Y, then one launch per stage
  if (X != Y) {
    hipError_t e = hipMemcpyAsync(Y, X, (size_t)nb * N * rp * 4, hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) {
      set_error("%s: copy failed: %s", who, hipGetErrorString(e));
      return SMAT_ELAUNCH;
    }
  }
  const int64_t rp4 = rp / 4;
  const int64_t npairs = (int64_t)nb * (N / 2) * rp4;
  for (int j = 0; j < logN; ++j) {
    smat::launch(butterfly_pass_kernel, dim3((unsigned)((npairs + 255) / 256)), dim3(256), 0,
                       stream, Y, N, j, rp4, npairs, mode);
  }
  if (mode == 1) {
    const int64_t t1 = (int64_t)nb * (N - 1) * rp4;
    if (t1 > 0)
      smat::launch(walsh_finish_kernel, dim3((unsigned)((t1 + 255) / 256)), dim3(256), 0,
                         stream, Y, N, rp4, t1, 0);
    const int64_t t0 = (int64_t)nb * rp4;
    smat::launch(walsh_finish_kernel, dim3((unsigned)((t0 + 255) / 256)), dim3(256), 0,
                       stream, Y, N, rp4, t0, 1);
  }
  return launch_status(who);
}

// U_h -= sum_x F_x: one thread per (batch, float4 of rp); sums F over x, then
// updates every row type.
__global__ __launch_bounds__(256) void complement_kernel(const float* __restrict__ F,
                                                         float* __restrict__ U, int N0, int B,
                                                         int64_t rp4, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t e = i % rp4;
  const int64_t b = i / rp4;
  const float4* Fb = reinterpret_cast<const float4*>(F) + b * N0 * rp4 + e;
  float4* Ub = reinterpret_cast<float4*>(U) + b * B * rp4 + e;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int x = 0; x < N0; ++x) {
    const float4 v = Fb[(int64_t)x * rp4];
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  for (int h = 0; h < B; ++h) {
    float4 u = Ub[(int64_t)h * rp4];
    u.x -= s.x;
    u.y -= s.y;
    u.z -= s.z;
    u.w -= s.w;
    Ub[(int64_t)h * rp4] = u;
  }
}

}  // namespace smat

extern "C" int smat_zeta(const float* F, float* Z, int nb, int N, int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && Z, SMAT_EINVAL, "smat_zeta: null pointer");
  SMAT_REQUIRE(nb >= 0 && N >= 0 && rp >= 0, SMAT_EINVAL, "smat_zeta: bad sizes");
  return butterfly_dispatch(F, Z, nb, N, rp, 0, (hipStream_t)stream, "smat_zeta");
}

extern "C" int smat_walsh(const float* F, float* U, int nb, int N, int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && U, SMAT_EINVAL, "smat_walsh: null pointer");
  SMAT_REQUIRE(nb >= 0 && N >= 0 && rp >= 0, SMAT_EINVAL, "smat_walsh: bad sizes");
  return butterfly_dispatch(F, U, nb, N, rp, 1, (hipStream_t)stream, "smat_walsh");
}

extern "C" int smat_incidence_complement(const float* F, float* U, int nb, int N0, int B,
                                         int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && U, SMAT_EINVAL, "smat_incidence_complement: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 0 && B >= 0 && rp >= 0, SMAT_EINVAL,
               "smat_incidence_complement: bad sizes");
  SMAT_REQUIRE(rp % 4 == 0 && aligned16(F) && aligned16(U), SMAT_EUNSUPPORTED,
               "smat_incidence_complement: needs rp %% 4 == 0 and aligned tables");
  const int64_t rp4 = rp / 4;
  const int64_t total = (int64_t)nb * rp4;
  if (total == 0 || B == 0) return SMAT_OK;
  smat::launch(complement_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, F, U, N0, B, rp4, total);
  return launch_status("smat_incidence_complement");
}
