// One cached-decode step for a batch of sequences (SmatDecoder.step,
// src/smat/attention.py:522-528):
//   S' = S + psi vb^T;   o = phi (S' + U[step mod B]);   out = o[:p-1] / o[p-1]
//
// A bandwidth kernel: per sequence it reads S and U_h (r*p fp32 each) and
// writes S' once.  Workgroups own 32-column groups of one sequence; 8 thread
// rows split the features and reduce through LDS.  Every group also needs the
// normaliser column, which only one group advances, so the state is
// double-buffered (S in, S' out): no group ever reads a column another group
// has already advanced.
#include "smat_host.hpp"

namespace smat {

namespace dc {
constexpr int kThreads = 256;
constexpr int kCols = 32;
constexpr int kParts = kThreads / kCols;   // 8 feature partitions
}  // namespace dc

template <typename In>
__global__ __launch_bounds__(dc::kThreads) void decode_step_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ S_in, float* __restrict__ S_out, const float* __restrict__ U,
    float* __restrict__ out, float* __restrict__ o_full, int B, int r, int p, int64_t step,
    int64_t q_sb, int64_t k_sb, int64_t v_sb) {
  using namespace dc;
  __shared__ float sphi[kMaxR], spsi[kMaxR], svb[kMaxP];
  __shared__ float red[kParts][kCols + 1];
  __shared__ float den_s;
  __shared__ float wsum[kThreads / 64];

  const int64_t b = blockIdx.y;
  const int c0 = blockIdx.x * kCols;
  const int tid = threadIdx.x;
  const int cl = tid % kCols, part = tid / kCols;
  const int h = (int)(step % B);

  if (tid < r) {
    sphi[tid] = to_f32(phi[b * q_sb + tid]);
    spsi[tid] = to_f32(psi[b * k_sb + tid]);
  }
  if (tid < p) svb[tid] = to_f32(vb[b * v_sb + tid]);
  __syncthreads();

  const int64_t rp = (int64_t)r * p;
  const float* Sb = S_in + b * rp;
  float* Sob = S_out + b * rp;
  const float* Ub = U + (b * B + h) * rp;

  const int c = c0 + cl;
  float acc = 0.f;
  if (c < p) {
    const float vc = svb[c];
    for (int a = part; a < r; a += kParts) {
      const int64_t o = (int64_t)a * p + c;
      const float s = Sb[o] + spsi[a] * vc;
      Sob[o] = s;
      acc += sphi[a] * (s + Ub[o]);
    }
  }
  red[part][cl] = acc;
  __syncthreads();

  // The normaliser o[p-1], computed the same way by every column group (so
  // all groups divide by the same value) from the incoming state.
  {
    float v = 0.f;
    for (int a = tid; a < r; a += kThreads) {
      const int64_t o = (int64_t)a * p + (p - 1);
      v += sphi[a] * ((Sb[o] + spsi[a] * svb[p - 1]) + Ub[o]);
    }
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
    if ((tid & 63) == 0) wsum[tid >> 6] = v;
    __syncthreads();
    if (tid == 0) {
      float t = 0.f;
      for (int i = 0; i < kThreads / 64; ++i) t += wsum[i];
      den_s = t;
    }
  }
  __syncthreads();

  if (tid < kCols && c0 + tid < p) {
    float o = 0.f;
    for (int i = 0; i < kParts; ++i) o += red[i][tid];
    const int cc = c0 + tid;
    if (o_full) o_full[b * p + cc] = o;
    if (cc < p - 1) out[b * (p - 1) + cc] = o / den_s;
  }
}

template <typename In>
static int launch_decode(const void* phi, const void* psi, const void* vb, const float* S_in,
                         float* S_out, const float* U, float* out, float* o_full, int nb, int B,
                         int r, int p, int64_t step, int64_t q_sb, int64_t k_sb, int64_t v_sb,
                         hipStream_t stream) {
  dim3 grid((unsigned)((p + dc::kCols - 1) / dc::kCols), (unsigned)nb);
  hipLaunchKernelGGL(decode_step_kernel<In>, grid, dim3(dc::kThreads), 0, stream, (const In*)phi,
                     (const In*)psi, (const In*)vb, S_in, S_out, U, out, o_full, B, r, p, step,
                     q_sb, k_sb, v_sb);
  return launch_status("smat_decode_step");
}

}  // namespace smat

extern "C" int smat_decode_step(int dtype, const void* phi_t, const void* psi_t, const void* vb_t,
                                const float* S_in, float* S_out, const float* U, float* out,
                                float* o_full, int nb, int B, int r, int p, int64_t step,
                                int64_t q_sb, int64_t k_sb, int64_t v_sb, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi_t && psi_t && vb_t && S_in && S_out && U && out, SMAT_EINVAL,
               "smat_decode_step: null pointer");
  SMAT_REQUIRE(S_in != S_out, SMAT_EINVAL, "smat_decode_step: S_in and S_out must differ");
  SMAT_REQUIRE(nb >= 0 && B >= 1 && step >= 0 && p >= 2, SMAT_EINVAL,
               "smat_decode_step: bad sizes (B=%d p=%d step=%lld)", B, p, (long long)step);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_decode_step: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  if (nb == 0) return SMAT_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SMAT_BF16:
      return launch_decode<bf16>(phi_t, psi_t, vb_t, S_in, S_out, U, out, o_full, nb, B, r, p,
                                 step, q_sb, k_sb, v_sb, st);
    case SMAT_F16:
      return launch_decode<f16>(phi_t, psi_t, vb_t, S_in, S_out, U, out, o_full, nb, B, r, p,
                                step, q_sb, k_sb, v_sb, st);
    case SMAT_F32:
      return launch_decode<float>(phi_t, psi_t, vb_t, S_in, S_out, U, out, o_full, nb, B, r, p,
                                  step, q_sb, k_sb, v_sb, st);
  }
  set_error("smat_decode_step: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}
