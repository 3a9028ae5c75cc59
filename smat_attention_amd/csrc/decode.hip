// One cached-decode step for a batch of sequences (SmatDecoder.step,
// src/smat/attention.py:522-528):
//   S' = S + psi vb^T;   o = phi (S' + U[step mod B]);   out = o[:p-1] / o[p-1]
//
// A bandwidth kernel: per sequence it reads S and U_h (r*p fp32 each) and
// writes S' once.  The state is double-buffered (S in, S' out) so a step never
// reads what it writes; the caller swaps the buffers.
#include "smat_host.hpp"

namespace smat {

namespace dc {
constexpr int kThreads = 1024;
constexpr int kCols = 144;                // p <= 144 columns, one thread column each
constexpr int kParts = kThreads / kCols;  // 7 feature partitions (1008 threads busy)
constexpr int kRows = (kMaxR + kParts - 1) / kParts;   // rows per thread, at most 19
}  // namespace dc

// One workgroup per sequence: thread (part, c) owns column c of the rows
// a = part, part + 7, ... (at most 19, all loaded up front); it advances S
// there (S_out = S_in + psi vb^T) and
// accumulates phi_a (S_out + U_h)[a][c].  The 7 partial sums of each column
// meet in LDS, which also hands every column the normaliser o[p-1] -- one read
// of S, U_h and one write of S per sequence, nothing recomputed.
template <typename In>
__global__ __launch_bounds__(dc::kThreads) void decode_step_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ S_in, float* __restrict__ S_out, const float* __restrict__ U,
    float* __restrict__ out, float* __restrict__ o_full, int B, int r, int p, int64_t step,
    int64_t q_sb, int64_t k_sb, int64_t v_sb) {
  using namespace dc;
  __shared__ float sphi[kMaxR], spsi[kMaxR], svb[kMaxP];
  __shared__ float red[kParts][kCols];

  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int c = tid % kCols, part = tid / kCols;
  const int h = (int)(step % B);

  const int64_t rp = (int64_t)r * p;
  const float* Sb = S_in + b * rp;
  float* Sob = S_out + b * rp;
  const float* Ub = U + (b * B + h) * rp;
  const bool mine = part < kParts && c < p;

  // every row of this thread (at most kRows) is loaded before phi, psi and vb
  // are staged: the state and the step's inputs are in flight together, one
  // memory latency per step instead of two.  U_h is read with non-temporal
  // loads (a type row comes back only B steps later); S is read again next
  // step and may stay in the caches.
  float sv[kRows], uv[kRows];
  if (mine) {
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const int a = part + u * kParts;
      if (a < r) {
        const int64_t o = (int64_t)a * p + c;
        sv[u] = Sb[o];
        uv[u] = __builtin_nontemporal_load(Ub + o);
      }
    }
  }
  if (tid < r) {
    sphi[tid] = to_f32(phi[b * q_sb + tid]);
    spsi[tid] = to_f32(psi[b * k_sb + tid]);
  }
  if (tid < p) svb[tid] = to_f32(vb[b * v_sb + tid]);
  __syncthreads();

  float acc = 0.f;
  if (mine) {
    const float vc = svb[c];
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const int a = part + u * kParts;
      if (a < r) {
        const float s = sv[u] + spsi[a] * vc;
        Sob[(int64_t)a * p + c] = s;
        acc += sphi[a] * (s + uv[u]);
      }
    }
  }
  if (part < kParts) red[part][c] = acc;
  __syncthreads();

  if (tid < p) {
    float o = 0.f, den = 0.f;
#pragma unroll
    for (int i = 0; i < kParts; ++i) {
      o += red[i][tid];
      den += red[i][p - 1];
    }
    if (o_full) o_full[b * p + tid] = o;
    if (tid < p - 1) out[b * (p - 1) + tid] = o / den;
  }
}

template <typename In>
static int launch_decode(const void* phi, const void* psi, const void* vb, const float* S_in,
                         float* S_out, const float* U, float* out, float* o_full, int nb, int B,
                         int r, int p, int64_t step, int64_t q_sb, int64_t k_sb, int64_t v_sb,
                         hipStream_t stream) {
  hipLaunchKernelGGL(decode_step_kernel<In>, dim3((unsigned)nb), dim3(dc::kThreads), 0, stream,
                     (const In*)phi, (const In*)psi, (const In*)vb, S_in, S_out, U, out, o_full,
                     B, r, p, step, q_sb, k_sb, v_sb);
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
