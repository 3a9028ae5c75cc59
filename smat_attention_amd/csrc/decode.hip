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
}  // namespace dc

// One sequence is split by value columns over nsplit workgroups (blockIdx.y):
// workgroup s owns columns [s cw, s cw + cw) of the p - 1 value columns, cw =
// ceil((p - 1) / nsplit), and also the normaliser column p - 1, which every
// workgroup needs for its division (only s = 0 writes it back).  Within a
// workgroup, thread (part, cl) owns local column cl of the rows a = part,
// part + kParts, ... (at most kRows, all loaded up front); it advances S there
// (S_out = S_in + psi vb^T) and accumulates phi_a (S_out + U_h)[a][c].  The
// kParts partial sums of each column meet in LDS, which also hands every
// column the normaliser -- S and U_h are read once and S written once, the
// normaliser column aside.
template <typename In, int kCols>
__global__ __launch_bounds__(dc::kThreads) void decode_step_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ S_in, float* __restrict__ S_out, const float* __restrict__ U,
    float* __restrict__ out, float* __restrict__ o_full, int B, int r, int p, int64_t step,
    int64_t q_sb, int64_t k_sb, int64_t v_sb) {
  using namespace dc;
  constexpr int kParts = kThreads / kCols;                 // feature partitions
  constexpr int kRows = (kMaxR + kParts - 1) / kParts;     // rows per thread
  __shared__ float sphi[kThreads], spsi[kThreads], svb[kThreads];   // one slot per thread
  __shared__ float red[kParts][kCols];

  const int64_t b = blockIdx.x;
  const int sp = blockIdx.y, nsplit = gridDim.y;
  const int tid = threadIdx.x;
  const int cl = tid % kCols, part = tid / kCols;
  const int h = (int)(step % B);
  const int cw = (p - 1 + nsplit - 1) / nsplit;            // value columns per workgroup
  const int cbeg = sp * cw;
  const int ncw = max(0, min(p - 1, cbeg + cw) - cbeg);    // this one's (ncw < kCols)
  const int c = cl < ncw ? cbeg + cl : p - 1;              // cl = ncw: the normaliser
  const bool mine = part < kParts && cl <= ncw;
  const bool writes = cl < ncw || sp == 0;                 // S and o_full of column c

  const int64_t rp = (int64_t)r * p;
  const float* Sb = S_in + b * rp;
  float* Sob = S_out + b * rp;
  const float* Ub = U + (b * B + h) * rp;

  // Loads, in issue order: this step's phi, psi and vb entry, then every row
  // of this thread (at most kRows of S and of U_h).  All are unconditional
  // (clamped indices), so each thread has a fixed count in flight, and loads
  // retire in order: the barrier that publishes phi, psi and vb waits for the
  // first three only, and each row below waits for its own pair while the
  // rest stream in -- the stores of S' start as the first rows land.  U_h is
  // read with non-temporal loads (a type row comes back only B steps later);
  // S is read again next step and may stay in the caches.
  const float fphi = to_f32(phi[b * q_sb + min(tid, r - 1)]);
  const float fpsi = to_f32(psi[b * k_sb + min(tid, r - 1)]);
  const float fvb = to_f32(vb[b * v_sb + min(tid, p - 1)]);
  __builtin_amdgcn_sched_barrier(0);   // ... issued before the rows
  float sv[kRows], uv[kRows];
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    const int64_t o = (int64_t)min(part + u * kParts, r - 1) * p + c;    // c < p always
    sv[u] = Sb[o];
    uv[u] = __builtin_nontemporal_load(Ub + o);
  }
  __builtin_amdgcn_sched_barrier(0);   // the rows are issued before the barrier below
  // unconditional stores: a branch here would let the compiler sink the
  // three loads below the rows (entries past r and p are never read)
  sphi[tid] = fphi;
  spsi[tid] = fpsi;
  svb[tid] = fvb;
  __syncthreads();

  // branch-free but for the store, so the row loads stay ahead of the
  // barrier (a branch around their uses would let the compiler sink them)
  float acc = 0.f;
  const float vc = svb[c];
#pragma unroll
  for (int u = 0; u < kRows; ++u) {
    const int a = part + u * kParts;
    const int ac = min(a, r - 1);
    const bool ok = mine && a < r;
    const float s = sv[u] + spsi[ac] * vc;
    if (ok && writes) Sob[(int64_t)a * p + c] = s;
    acc += ok ? sphi[ac] * (s + uv[u]) : 0.f;
  }
  if (part < kParts) red[part][cl] = acc;
  __syncthreads();

  if (tid <= ncw) {
    float o = 0.f, den = 0.f;
#pragma unroll
    for (int i = 0; i < kParts; ++i) {
      o += red[i][tid];
      den += red[i][ncw];
    }
    const int cc = tid < ncw ? cbeg + tid : p - 1;
    if (o_full && (tid < ncw || sp == 0)) o_full[b * p + cc] = o;
    if (tid < ncw) out[b * (p - 1) + cc] = o / den;
  }
}

// Column split: the fewest workgroups per sequence (1, 2 or 4) that give at
// least 256 workgroups, one per CU, so a small batch still streams S and U_h
// through every CU.
static int decode_split(int nb) {
  int ns = 1;
  while (ns < 4 && (int64_t)nb * ns < 256) ns <<= 1;
  return ns;
}

template <typename In>
static int launch_decode(const void* phi, const void* psi, const void* vb, const float* S_in,
                         float* S_out, const float* U, float* out, float* o_full, int nb, int B,
                         int r, int p, int64_t step, int64_t q_sb, int64_t k_sb, int64_t v_sb,
                         hipStream_t stream) {
  const int ns = decode_split(nb);
  const dim3 grid((unsigned)nb, (unsigned)ns);
  // local columns: ceil((p - 1) / ns) value columns and the normaliser, with
  // p <= 144: at most 144, 73 and 37
  if (ns == 1)
    hipLaunchKernelGGL((decode_step_kernel<In, 144>), grid, dim3(dc::kThreads), 0, stream,
                       (const In*)phi, (const In*)psi, (const In*)vb, S_in, S_out, U, out, o_full,
                       B, r, p, step, q_sb, k_sb, v_sb);
  else if (ns == 2)
    hipLaunchKernelGGL((decode_step_kernel<In, 80>), grid, dim3(dc::kThreads), 0, stream,
                       (const In*)phi, (const In*)psi, (const In*)vb, S_in, S_out, U, out, o_full,
                       B, r, p, step, q_sb, k_sb, v_sb);
  else
    hipLaunchKernelGGL((decode_step_kernel<In, 48>), grid, dim3(dc::kThreads), 0, stream,
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
