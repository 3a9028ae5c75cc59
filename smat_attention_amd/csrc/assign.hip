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
constexpr int kMaxOcc = 4096;       // dim * q: the occupancy bins of one (sequence, head)
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
      cell = cell * q + (int64_t)fminf(floorf(s), (float)(q - 1));
      if (lane == 0) s_out[(((int64_t)bi * nh + h) * L + li) * dim + k] = s;
    }
    if (lane == 0) cells[((int64_t)bi * nh + h) * L + li] = cell;
  }
}

// The (cell, weight) pairs of the training path at anneal = 1
// (src/smat/assign.py:257-317), from the projections z (nb, L, nh*dim) that
// autograd computed: s_k = clamp(q Phi_N(z_k), 0, q - 1e-4), the low bin
// lo_k = floor(s_k), the high bin min(lo_k + 1, q - 1) and the fraction
// f_k = s_k - lo_k.  Pair p of a token takes the high bin in coordinate k
// when bit k of p is set (the reference's concatenation order), so
// idx[p] = sum_k bin_k(p) q^(dim-1-k) and the chosen cell is idx[0].  A planted
// token (plant[l] >= 0) gets that cell for every pair.  The soft occupancy
// occ[k][bin] sums 1 - f_k at the low bin and f_k at the high bin over the
// sequence's L tokens, planted ones included.  One workgroup per
// (sequence, head); the occupancy is accumulated with LDS atomics, so the
// order of each bin's sum is not fixed (as the reference's scatter_add).
__global__ __launch_bounds__(ah::kThreads) void hash_pairs_kernel(
    const float* __restrict__ z, const int64_t* __restrict__ plant, float* __restrict__ s_out,
    int64_t* __restrict__ cells, int64_t* __restrict__ idx, float* __restrict__ occ, int L,
    int nh, int dim, int q) {
  __shared__ float socc[ah::kMaxOcc];
  const int bh = blockIdx.x;
  const int bi = bh / nh, h = bh - bi * nh;
  const int hd = nh * dim, K = 1 << dim;
  for (int i = threadIdx.x; i < dim * q; i += ah::kThreads) socc[i] = 0.f;
  __syncthreads();
  for (int li = threadIdx.x; li < L; li += ah::kThreads) {
    const float* zr = z + ((int64_t)bi * L + li) * hd + h * dim;
    const int64_t t = (int64_t)bh * L + li;
    int lo[8], hi[8];
    int64_t cell = 0;
    for (int k = 0; k < dim; ++k) {
      float sv = 0.5f * erfcf(-zr[k] * 0.70710678118654752f) * (float)q;
      sv = fminf(fmaxf(sv, 0.f), (float)q - 1e-4f);
      const float fl = fminf(floorf(sv), (float)(q - 1));   // q - 1e-4 rounds to q past q ~ 1700
      const float f = sv - fl;
      lo[k] = (int)fl;
      hi[k] = lo[k] + 1 < q ? lo[k] + 1 : q - 1;
      s_out[t * dim + k] = sv;
      atomicAdd(&socc[k * q + lo[k]], 1.f - f);
      atomicAdd(&socc[k * q + hi[k]], f);
      cell = cell * q + lo[k];
    }
    const int64_t pc = plant ? plant[li] : -1;
    cells[t] = pc >= 0 ? pc : cell;
    for (int pr = 0; pr < K; ++pr) {
      int64_t c = 0;
      for (int k = 0; k < dim; ++k) c = c * q + (((pr >> k) & 1) ? hi[k] : lo[k]);
      idx[t * K + pr] = pc >= 0 ? pc : c;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < dim * q; i += ah::kThreads) occ[(int64_t)bh * dim * q + i] = socc[i];
}

// Backward of the pairs: the gradient of z from the pairs' weights dw
// (nb*nh, L, 2^dim) and the occupancy's docc (nb*nh, dim, q), either null.
// The forward weights are the one-hot of pair 0; pair p's weight is the
// product over k of 1 + (1 - f_k) - sg(1 - f_k) (low bin) or f_k - sg(f_k)
// (high bin), so its derivative by f_k is -1 at p = 0, +1 at p = 2^k and 0
// elsewhere.  Planted tokens have fixed weights (no dw term) but still count
// in the occupancy.  With d s / d z = q phi(z) inside the clamp's range:
//
//   dz_k = q phi(z_k) [0 <= q Phi_N(z_k) <= q - 1e-4]
//          * (dw[2^k] - dw[0] + docc[k][hi_k] - docc[k][lo_k])
//
// One thread per (token, head).
__global__ __launch_bounds__(ah::kThreads) void hash_pairs_bwd_kernel(
    const float* __restrict__ z, const float* __restrict__ s_fwd, const int64_t* __restrict__ plant,
    const float* __restrict__ dw, const float* __restrict__ docc, float* __restrict__ dz, int nb,
    int L, int nh, int dim, int q) {
  const int64_t n = (int64_t)nb * L * nh;
  const int hd = nh * dim, K = 1 << dim;
  for (int64_t i = (int64_t)blockIdx.x * ah::kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * ah::kThreads) {
    const int64_t row = i / nh;                       // bi * L + li
    const int h = (int)(i - row * nh);
    const int64_t bi = row / L;
    const int li = (int)(row - bi * L);
    const int64_t bh = bi * nh + h;
    const int64_t t = bh * L + li;
    const bool fixed = plant && plant[li] >= 0;
    for (int k = 0; k < dim; ++k) {
      const float zk = z[row * hd + h * dim + k];
      const float sraw = 0.5f * erfcf(-zk * 0.70710678118654752f) * (float)q;
      float df = 0.f;
      if (dw && !fixed) df += dw[t * K + (1 << k)] - dw[t * K];
      if (docc) {
        const float sv = s_fwd[t * dim + k];
        const int lo = (int)fminf(floorf(sv), (float)(q - 1));
        const int hi = lo + 1 < q ? lo + 1 : q - 1;
        const float* dr = docc + (bh * dim + k) * q;
        df += dr[hi] - dr[lo];
      }
      const bool inside = sraw >= 0.f && sraw <= (float)q - 1e-4f;
      dz[row * hd + h * dim + k] =
          inside ? df * (float)q * 0.39894228040143268f * expf(-0.5f * zk * zk) : 0.f;
    }
  }
}

}  // namespace smat

extern "C" int smat_hash_pairs(const float* z, const int64_t* plant, float* s_out, int64_t* cells,
                               int64_t* idx, float* occ, int nb, int L, int nh, int dim, int q,
                               void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(z && s_out && cells && idx && occ, SMAT_EINVAL, "smat_hash_pairs: null pointer");
  SMAT_REQUIRE(nb >= 0 && L >= 0 && nh >= 1 && dim >= 1 && dim <= 8 && q >= 2 &&
                   dim * q <= ah::kMaxOcc && nh * dim <= ah::kMaxHD,
               SMAT_EUNSUPPORTED, "smat_hash_pairs: sizes beyond dim<=8, dim*q<=%d, heads*dim<=%d",
               ah::kMaxOcc, ah::kMaxHD);
  if (nb == 0) return SMAT_OK;
  hipLaunchKernelGGL(hash_pairs_kernel, dim3((unsigned)(nb * nh)), dim3(ah::kThreads), 0,
                     (hipStream_t)stream, z, plant, s_out, cells, idx, occ, L, nh, dim, q);
  return launch_status("smat_hash_pairs");
}

extern "C" int smat_hash_pairs_backward(const float* z, const float* s_fwd, const int64_t* plant,
                                        const float* dw, const float* docc, float* dz, int nb,
                                        int L, int nh, int dim, int q, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(z && s_fwd && dz, SMAT_EINVAL, "smat_hash_pairs_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && L >= 0 && nh >= 1 && dim >= 1 && dim <= 8 && q >= 2 &&
                   nh * dim <= ah::kMaxHD,
               SMAT_EUNSUPPORTED, "smat_hash_pairs_backward: sizes beyond dim<=8, heads*dim<=%d",
               ah::kMaxHD);
  const int64_t n = (int64_t)nb * L * nh;
  if (n == 0) return SMAT_OK;
  const int64_t need = (n + ah::kThreads - 1) / ah::kThreads;
  const unsigned grid = (unsigned)(need < 4096 ? need : 4096);
  hipLaunchKernelGGL(hash_pairs_bwd_kernel, dim3(grid), dim3(ah::kThreads), 0, (hipStream_t)stream,
                     z, s_fwd, plant, dw, docc, dz, nb, L, nh, dim, q);
  return launch_status("smat_hash_pairs_backward");
}

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
