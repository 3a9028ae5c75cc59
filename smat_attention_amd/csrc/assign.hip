// Content hash of a content-addressed assignment (src/smat/assign.py:246-276,
// the hard path): for every token row u (d_model values) and head h,
//
//   z_k  = (LN(u) . Wn[h, k]) * gamma[h, k] + b[h, k]      k < dim
//   s_k  = clamp(q * Phi_N(z_k), 0, q - 1e-4)               Phi_N(z) = erfc(-z/sqrt 2)/2
//   cell = sum_k floor(s_k) * q^(dim-1-k)
//
// LN is LayerNorm without affine (biased variance, eps 1e-5), Wn the unit
// rows W / max(|W|, 1e-6).  One wave per token row: the row is read once,
// its mean and variance reduced across the wave (two passes over the row in
// registers), then every (head, coordinate) dot product.  s is returned too:
// the straight-through weights and the load-balance term use its fraction.
// Output layout follows the reference's (nb*h, L, .) head-major reshape.
#include "smat_host.hpp"

namespace smat {

namespace ah {
constexpr int kThreads = 256;
constexpr int kMaxDM = 2048;        // d_model: at most 32 values per lane
constexpr int kMaxHD = 64;          // heads * dim
}  // namespace ah

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename T>
__global__ __launch_bounds__(ah::kThreads) void cell_hash_kernel(
    const T* __restrict__ u, const float* __restrict__ Wn, const float* __restrict__ gamma,
    const float* __restrict__ bias, float* __restrict__ s_out, int64_t* __restrict__ cells,
    int nb, int L, int dm, int nh, int dim, int q, int64_t u_sb, int64_t u_st) {
  constexpr int kPer = ah::kMaxDM / 64;
  const int64_t row = (int64_t)blockIdx.x * (ah::kThreads / 64) + wave_id();
  const int lane = lane_id();
  if (row >= (int64_t)nb * L) return;
  const int64_t bi = row / L;
  const int li = (int)(row - bi * L);
  const T* ur = u + bi * u_sb + (int64_t)li * u_st;
  float x[kPer];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int m = lane + 64 * j;
    x[j] = m < dm ? (float)ur[m] : 0.f;
    sum += x[j];
  }
  const float mean = wave_sum(sum) / (float)dm;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int m = lane + 64 * j;
    const float d = m < dm ? x[j] - mean : 0.f;
    sq += d * d;
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)dm + 1e-5f);
#pragma unroll
  for (int j = 0; j < kPer; ++j) x[j] = (x[j] - mean) * rstd;

  for (int h = 0; h < nh; ++h) {
    int64_t cell = 0;
    for (int k = 0; k < dim; ++k) {
      const float* w = Wn + ((int64_t)h * dim + k) * dm;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int m = lane + 64 * j;
        if (m < dm) acc += x[j] * w[m];
      }
      const float z = wave_sum(acc) * gamma[h * dim + k] + bias[h * dim + k];
      float s = 0.5f * erfcf(-z * 0.70710678118654752f) * (float)q;
      s = fminf(fmaxf(s, 0.f), (float)q - 1e-4f);
      cell = cell * q + (int64_t)floorf(s);
      if (lane == 0) s_out[(((int64_t)bi * nh + h) * L + li) * dim + k] = s;
    }
    if (lane == 0) cells[((int64_t)bi * nh + h) * L + li] = cell;
  }
}

}  // namespace smat

extern "C" int smat_cell_hash(int dtype, const void* u, const float* Wn, const float* gamma,
                              const float* bias, float* s_out, int64_t* cells, int nb, int L,
                              int dm, int nh, int dim, int q, int64_t u_sb, int64_t u_st,
                              void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(u && Wn && gamma && bias && s_out && cells, SMAT_EINVAL,
               "smat_cell_hash: null pointer");
  SMAT_REQUIRE(nb >= 0 && L >= 0 && dm >= 1 && dm <= ah::kMaxDM && nh >= 1 && dim >= 1 &&
                   nh * dim <= ah::kMaxHD && q >= 2,
               SMAT_EUNSUPPORTED, "smat_cell_hash: sizes beyond d_model<=%d, heads*dim<=%d",
               ah::kMaxDM, ah::kMaxHD);
  SMAT_REQUIRE(u_st >= dm, SMAT_EINVAL, "smat_cell_hash: row stride too short");
  const int64_t rows = (int64_t)nb * L;
  if (rows == 0) return SMAT_OK;
  const int64_t grid = (rows + ah::kThreads / 64 - 1) / (ah::kThreads / 64);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SMAT_F32:
      hipLaunchKernelGGL(cell_hash_kernel<float>, dim3((unsigned)grid), dim3(ah::kThreads), 0, st,
                         (const float*)u, Wn, gamma, bias, s_out, cells, nb, L, dm, nh, dim, q,
                         u_sb, u_st);
      break;
    case SMAT_BF16:
      hipLaunchKernelGGL(cell_hash_kernel<bf16>, dim3((unsigned)grid), dim3(ah::kThreads), 0, st,
                         (const bf16*)u, Wn, gamma, bias, s_out, cells, nb, L, dm, nh, dim, q,
                         u_sb, u_st);
      break;
    case SMAT_F16:
      hipLaunchKernelGGL(cell_hash_kernel<f16>, dim3((unsigned)grid), dim3(ah::kThreads), 0, st,
                         (const f16*)u, Wn, gamma, bias, s_out, cells, nb, L, dm, nh, dim, q,
                         u_sb, u_st);
      break;
    default:
      set_error("smat_cell_hash: unknown dtype %d", dtype);
      return SMAT_EINVAL;
  }
  return launch_status("smat_cell_hash");
}
