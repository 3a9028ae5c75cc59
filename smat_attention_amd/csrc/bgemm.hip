// Strided batched GEMM with fp32 MFMA, for the backward pass of the schedule:
//
//   C[i] (M x N)  =  A[i] (M x K) . B[i] (K x N)        (beta = 0)
//   C[i]         +=  A[i] . B[i]                        (beta = 1)
//
// with an optional causal mask on C (keep m >= n, or m <= n).  Every operand
// is addressed by a row stride and a column stride (so a transpose is only a
// swap of strides) and a two-level batch index i = (i1, i2), each level with
// its own stride -- enough to express per-chunk, per-row-type and per-profile
// products on the (nb, T, .) activations without copies.  Inputs may be bf16,
// fp16 or fp32; they are widened to fp32 when staged, and the products run on
// v_mfma_f32_16x16x4_f32, so results are fp32 products summed in fp32.
//
// Tiling: a 256-thread workgroup computes a 64 x kBN block of C.  kBN = 64:
// wave w owns the 32 x 32 quarter (w >> 1, w & 1) as 2 x 2 MFMA tiles.
// kBN = 80, for N just past a multiple of 64 (p = 65, 129: value columns plus
// the ones column): wave w owns rows 16w .. 16w + 15 across five column tiles,
// so N = 65 takes one block instead of two.  K advances 32 at a time through
// LDS (A as [m][k], B as [n][k]).
#include "smat_host.hpp"

namespace smat {

namespace bg {
constexpr int kThreads = 256;
constexpr int kBM = 64, kBK = 32;
constexpr int kPad = kBK + 4;        // LDS row length (floats)
}  // namespace bg

struct GemmArgs {
  int M, N, K, n2;
  int64_t a1, a2, am, ak;   // A: batch strides, row (m) stride, column (k) stride
  int64_t b1, b2, bk, bn;   // B: batch strides, row (k) stride, column (n) stride
  int64_t c1, c2, cm, cn;   // C
  int beta, mask;           // mask: 0 none, 1 keep m >= n, 2 keep m <= n
};

template <typename TA, typename TB, int kBN>
__global__ __launch_bounds__(bg::kThreads) void bgemm_kernel(const TA* __restrict__ A,
                                                             const TB* __restrict__ B,
                                                             float* __restrict__ Cm, GemmArgs g) {
  using namespace bg;
  static_assert(kBN == 64 || kBN == 80, "column block of 64 or 80");
  constexpr int kWC = kBN == 64 ? 2 : 1;            // waves across the columns
  constexpr int kTM = kBN == 64 ? 2 : 1;            // 16-row MFMA tiles per wave
  constexpr int kTN = kBN == 64 ? 2 : 5;            // 16-column MFMA tiles per wave
  __shared__ __attribute__((aligned(16))) float sA[kBM * kPad];
  __shared__ __attribute__((aligned(16))) float sB[kBN * kPad];

  const int bi = blockIdx.z;
  const int i1 = bi / g.n2, i2 = bi - i1 * g.n2;
  const TA* Ab = A + i1 * g.a1 + i2 * g.a2;
  const TB* Bb = B + i1 * g.b1 + i2 * g.b2;
  float* Cb = Cm + i1 * g.c1 + i2 * g.c2;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int lane = lane_id(), w = wave_id();
  const int row16 = lane & 15, grp = lane >> 4;
  const int wm = (w / kWC) * 16 * kTM, wn = (w % kWC) * 16 * kTN;

  // a masked block contributes nothing: skip its products (the store still
  // writes zeros where beta = 0)
  bool skip = false;
  if (g.mask == 1 && n0 > m0 + kBM - 1) skip = true;
  if (g.mask == 2 && m0 > n0 + kBN - 1) skip = true;

  f32x4 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) acc[i][j] = zero4();

  if (!skip) {
    // the next K step's elements are loaded into registers while the current
    // step is multiplied (element idx = tid + e kThreads of each tile)
    constexpr int kPA = kBM * kBK / kThreads, kPB = kBN * kBK / kThreads;   // 8; 8 or 10
    float ra[kPA], rb[kPB];
    auto load = [&](int k0) {
#pragma unroll
      for (int e = 0; e < kPA; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        const int mm = idx / kBK, kk = idx - mm * kBK;
        const int m = m0 + mm, k = k0 + kk;
        ra[e] = (m < g.M && k < g.K) ? to_f32(Ab[(int64_t)m * g.am + (int64_t)k * g.ak]) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < kPB; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        const int nn = idx / kBK, kk = idx - nn * kBK;
        const int n = n0 + nn, k = k0 + kk;
        rb[e] = (n < g.N && k < g.K) ? to_f32(Bb[(int64_t)k * g.bk + (int64_t)n * g.bn]) : 0.f;
      }
    };
    load(0);
    for (int k0 = 0; k0 < g.K; k0 += kBK) {
      if (k0 > 0) __syncthreads();       // the previous step's readers are done
#pragma unroll
      for (int e = 0; e < kPA; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        sA[(idx / kBK) * kPad + idx % kBK] = ra[e];
      }
#pragma unroll
      for (int e = 0; e < kPB; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        sB[(idx / kBK) * kPad + idx % kBK] = rb[e];
      }
      __syncthreads();
      if (k0 + kBK < g.K) load(k0 + kBK);
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
        f32x8 a;
        const float* ap = sA + (wm + 16 * i + row16) * kPad + 8 * grp;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = ap[e];
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          f32x8 bv;
          const float* bp = sB + (wn + 16 * j + row16) * kPad + 8 * grp;
#pragma unroll
          for (int e = 0; e < 8; ++e) bv[e] = bp[e];
          acc[i][j] = mma(acc[i][j], a, bv);
        }
      }
    }
  }

#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int n = n0 + wn + 16 * j + row16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm + 16 * i + 4 * grp + e;
        if (m < g.M && n < g.N) {
          float v = acc[i][j][e];
          if ((g.mask == 1 && n > m) || (g.mask == 2 && m > n)) v = 0.f;
          float* cp = Cb + (int64_t)m * g.cm + (int64_t)n * g.cn;
          *cp = g.beta ? *cp + v : v;
        }
      }
    }
  }
}

template <typename TA, typename TB>
static int launch_bgemm(const void* A, const void* B, float* C, int n1, const GemmArgs& g,
                        hipStream_t stream) {
  // the column block that pads N least (ties: 64)
  const int64_t pad64 = (int64_t)(g.N + 63) / 64 * 64, pad80 = (int64_t)(g.N + 79) / 80 * 80;
  const int bn = pad80 < pad64 ? 80 : 64;
  dim3 grid((unsigned)((g.N + bn - 1) / bn), (unsigned)((g.M + bg::kBM - 1) / bg::kBM),
            (unsigned)(n1 * g.n2));
  if (bn == 80)
    hipLaunchKernelGGL((bgemm_kernel<TA, TB, 80>), grid, dim3(bg::kThreads), 0, stream,
                       (const TA*)A, (const TB*)B, C, g);
  else
    hipLaunchKernelGGL((bgemm_kernel<TA, TB, 64>), grid, dim3(bg::kThreads), 0, stream,
                       (const TA*)A, (const TB*)B, C, g);
  return launch_status("smat_bgemm");
}

template <typename TA>
static int bgemm_b(int tb, const void* A, const void* B, float* C, int n1, const GemmArgs& g,
                   hipStream_t s) {
  switch (tb) {
    case SMAT_BF16: return launch_bgemm<TA, bf16>(A, B, C, n1, g, s);
    case SMAT_F16: return launch_bgemm<TA, f16>(A, B, C, n1, g, s);
    case SMAT_F32: return launch_bgemm<TA, float>(A, B, C, n1, g, s);
  }
  set_error("smat_bgemm: unknown dtype of B %d", tb);
  return SMAT_EINVAL;
}

}  // namespace smat

extern "C" int smat_bgemm(int dtype_a, int dtype_b, const void* A, const void* B, float* C, int M,
                          int N, int K, int n1, int n2, int64_t a1, int64_t a2, int64_t am,
                          int64_t ak, int64_t b1, int64_t b2, int64_t bk, int64_t bn, int64_t c1,
                          int64_t c2, int64_t cm, int64_t cn, int beta, int mask, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(A && B && C, SMAT_EINVAL, "smat_bgemm: null pointer");
  SMAT_REQUIRE(M >= 0 && N >= 0 && K >= 0 && n1 >= 0 && n2 >= 1, SMAT_EINVAL,
               "smat_bgemm: bad sizes");
  SMAT_REQUIRE((int64_t)n1 * n2 < 65536, SMAT_EUNSUPPORTED,
               "smat_bgemm: %lld batches exceed 65535", (long long)n1 * n2);
  SMAT_REQUIRE(mask >= 0 && mask <= 2 && (beta == 0 || beta == 1), SMAT_EINVAL,
               "smat_bgemm: mask must be 0..2 and beta 0 or 1");
  if (M == 0 || N == 0 || n1 == 0) return SMAT_OK;
  GemmArgs g{M, N, K, n2, a1, a2, am, ak, b1, b2, bk, bn, c1, c2, cm, cn, beta, mask};
  hipStream_t s = (hipStream_t)stream;
  switch (dtype_a) {
    case SMAT_BF16: return bgemm_b<bf16>(dtype_b, A, B, C, n1, g, s);
    case SMAT_F16: return bgemm_b<f16>(dtype_b, A, B, C, n1, g, s);
    case SMAT_F32: return bgemm_b<float>(dtype_b, A, B, C, n1, g, s);
  }
  set_error("smat_bgemm: unknown dtype of A %d", dtype_a);
  return SMAT_EINVAL;
}
