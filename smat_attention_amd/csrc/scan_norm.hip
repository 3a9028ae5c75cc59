// Bandwidth kernels around the chunk pass:
//   * the segmented shifted exclusive scan of chunk summaries
//     (src/smat/attention.py:163-179);
//   * the final normalisation H[..., :-1] / H[..., -1:] with the long-range
//     term added for recent rows and the optional output gate
//     (src/smat/attention.py:446-453).
#include "smat_host.hpp"

namespace smat {

// One thread per state element; it walks its segment's chunks in order, so
// Sin[c] is the running sum BEFORE adding D[c] (a shifted scan: D[c] never
// reaches its own Sin[c], and no subtraction ever happens).
__global__ __launch_bounds__(256) void segment_scan_kernel(const float* __restrict__ D,
                                                           float* __restrict__ Sin, int nc,
                                                           int nc0, int64_t rp) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  const int seg = blockIdx.z;
  if (e >= rp) return;
  const int c_lo = seg == 0 ? 0 : nc0;
  const int c_hi = seg == 0 ? nc0 : nc;
  const float* Db = D + b * nc * rp + e;
  float* Sb = Sin + b * nc * rp + e;
  // eight loads in flight per thread, then their eight running sums (same
  // order of additions as one at a time)
  float run = 0.f;
  int c = c_lo;
  for (; c + 8 <= c_hi; c += 8) {
    float d[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) d[u] = Db[(int64_t)(c + u) * rp];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      Sb[(int64_t)(c + u) * rp] = run;
      run += d[u];
    }
  }
  for (; c < c_hi; ++c) {
    const float d = Db[(int64_t)c * rp];
    Sb[(int64_t)c * rp] = run;
    run += d;
  }
}

// The decayed recurrence over chunks (src/smat/model.py:71-80):
//   Sin[c] = the state entering chunk c;  S <- aC[c] S + D[c];  S = 0 at c = nc0.
__global__ __launch_bounds__(256) void decay_scan_kernel(const float* __restrict__ D,
                                                         const float* __restrict__ aC,
                                                         float* __restrict__ Sin, int nc, int nc0,
                                                         int64_t rp) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (e >= rp) return;
  const float* Db = D + b * nc * rp + e;
  const float* ab = aC + b * nc;
  float* Sb = Sin + b * nc * rp + e;
  float run = 0.f;
  for (int c = 0; c < nc; ++c) {
    if (c == nc0) run = 0.f;
    Sb[(int64_t)c * rp] = run;
    run = ab[c] * run + Db[(int64_t)c * rp];
  }
}

// Its gradient, walking the chunks backwards (the reset at nc0 stops the flow):
//   g = 0;  for c = nc-1 .. 0:  gn = (c + 1 == nc0) ? 0 : g;  dD[c] = gn;
//                               g = dSin[c] + aC[c] gn
// dD[c] is the gradient of the summary D[c] (that of the state after chunk c).
__global__ __launch_bounds__(256) void decay_scan_rev_kernel(const float* __restrict__ dSin,
                                                             const float* __restrict__ aC,
                                                             float* __restrict__ dD, int nc,
                                                             int nc0, int64_t rp) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (e >= rp) return;
  const float* gb = dSin + b * nc * rp + e;
  const float* ab = aC + b * nc;
  float* db = dD + b * nc * rp + e;
  float g = 0.f;
  for (int c = nc - 1; c >= 0; --c) {
    const float gn = (c + 1 == nc0) ? 0.f : g;
    db[(int64_t)c * rp] = gn;
    g = gb[(int64_t)c * rp] + ab[c] * gn;
  }
}

// The mirror image for the backward pass: Sout[c] = sum of D[c'] over the
// later chunks c' > c of the same segment (the state flowing backwards).
__global__ __launch_bounds__(256) void segment_scan_rev_kernel(const float* __restrict__ D,
                                                               float* __restrict__ Sout, int nc,
                                                               int nc0, int64_t rp) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  const int seg = blockIdx.z;
  if (e >= rp) return;
  const int c_lo = seg == 0 ? 0 : nc0;
  const int c_hi = seg == 0 ? nc0 : nc;
  const float* Db = D + b * nc * rp + e;
  float* Sb = Sout + b * nc * rp + e;
  float run = 0.f;
  for (int c = c_hi - 1; c >= c_lo; --c) {
    const float d = Db[(int64_t)c * rp];
    Sb[(int64_t)c * rp] = run;
    run += d;
  }
}

// Rows of the normalisation: sixteen lanes a row, four rows a wave, sixteen
// a workgroup; lane l of a row's group takes columns l, l + 16, ... (each
// load coalesced over the group).
namespace nrm {
constexpr int kLanes = 16;
constexpr int kRows = 256 / kLanes;
}  // namespace nrm

// Backward of out = N[:, :p-1] / den * g, where N = H + [0; Y] (the Y rows
// added from row n on; Y may be null) and den is N[:, p-1], floored at eps
// when kFloor (the layer's clamp_min):
//   dN_c = dout_c g / den (c < p-1),
//   dN_{p-1} = -sum_c dN_c N_c / den (0 where the floor is active),
//   dg = sum_c dout_c N_c / den.
// dN is the gradient of H and, from row n on, of Y as well.
template <bool kFloor, typename Din>
__global__ __launch_bounds__(256) void normalise_bwd_kernel(
    const Din* __restrict__ dout, const float* __restrict__ H, const float* __restrict__ Y,
    const float* __restrict__ g, float* __restrict__ dH, float* __restrict__ dg, int T, int n,
    int p, float eps, int64_t o_sb, int64_t o_st, int64_t h_sb, int64_t h_st, int64_t y_sb,
    int64_t y_st, int64_t d_sb, int64_t d_st, int64_t g_sb) {
  const int64_t row = (int64_t)blockIdx.x * nrm::kRows + (threadIdx.x >> 4);
  const int64_t b = blockIdx.y;
  const int l = threadIdx.x & (nrm::kLanes - 1);
  if (row >= T) return;                              // whole 16-lane groups
  const float* h = H + b * h_sb + row * h_st;
  const float* y = (Y != nullptr && row >= n) ? Y + b * y_sb + (row - n) * y_st : nullptr;
  const Din* d = dout + b * o_sb + row * o_st;
  float* dh = dH + b * d_sb + row * d_st;
  const float den_raw = y ? h[p - 1] + y[p - 1] : h[p - 1];
  const float den = kFloor ? fmaxf(den_raw, eps) : den_raw;
  const float inv = 1.f / den;
  const float gate = g ? g[b * g_sb + row] : 1.f;
  float sh = 0.f, sg = 0.f;
#pragma unroll 4
  for (int c = l; c < p - 1; c += nrm::kLanes) {
    const float o = (y ? h[c] + y[c] : h[c]) * inv;
    const float dv = to_f32(d[c]);
    const float dc = dv * gate * inv;
    dh[c] = dc;
    sh += dc * o;
    sg += dv * o;
  }
#pragma unroll
  for (int off = nrm::kLanes / 2; off > 0; off >>= 1) {
    sh += __shfl_xor(sh, off, nrm::kLanes);
    sg += __shfl_xor(sg, off, nrm::kLanes);
  }
  if (l == 0) {
    dh[p - 1] = (kFloor && !(den_raw >= eps)) ? 0.f : -sh;
    if (dg) dg[b * T + row] = sg;
  }
}

int segment_scan_dispatch(const float* D, float* Sin, int nb, int nc, int nc0, int64_t rp,
                          hipStream_t stream) {
  if (nb == 0 || nc == 0 || rp == 0) return SMAT_OK;
  // nc0 == 0 or nc0 == nc: one segment.  Segment 1 is [nc0, nc).
  dim3 grid((unsigned)((rp + 255) / 256), (unsigned)nb, 2);
  smat::launch(segment_scan_kernel, grid, dim3(256), 0, stream, D, Sin, nc, nc0, rp);
  return launch_status("smat_segment_scan");
}

// Sixteen lanes per output row: the normaliser is read once, every column
// divided; with kFloor (eps >= 0 at dispatch) the normaliser is floored at
// eps first.
template <bool kFloor, typename Out>
__global__ __launch_bounds__(256) void normalise_kernel(
    const float* __restrict__ H, const float* __restrict__ Y, const float* __restrict__ g,
    Out* __restrict__ out, int T, int n, int p, float eps, int64_t h_sb, int64_t h_st,
    int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st, int64_t g_sb) {
  const int64_t row = (int64_t)blockIdx.x * nrm::kRows + (threadIdx.x >> 4);
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & (nrm::kLanes - 1);
  if (row >= T) return;
  const float* h = H + b * h_sb + row * h_st;
  const float* y = (Y != nullptr && row >= n) ? Y + b * y_sb + (row - n) * y_st : nullptr;
  float den = h[p - 1];
  if (y) den += y[p - 1];
  if (kFloor) den = fmaxf(den, eps);
  const float gate = g ? g[b * g_sb + row] : 1.f;
  Out* o = out + b * o_sb + row * o_st;
#pragma unroll 4
  for (int c = lane; c < p - 1; c += nrm::kLanes) {
    float num = h[c];
    if (y) num += y[c];
    float v = num / den;
    if (g) v *= gate;
    o[c] = from_f32<Out>(v);
  }
}

template <typename Out>
static int launch_normalise(const float* H, const float* Y, const float* g, Out* out, int nb, int T,
                            int n, int p, int64_t h_sb, int64_t h_st, int64_t y_sb, int64_t y_st,
                            int64_t o_sb, int64_t o_st, int64_t g_sb, hipStream_t stream,
                            float eps) {
  if (nb == 0 || T == 0) return SMAT_OK;
  dim3 grid((unsigned)((T + nrm::kRows - 1) / nrm::kRows), (unsigned)nb);
  if (eps >= 0.f)
    smat::launch((normalise_kernel<true, Out>), grid, dim3(256), 0, stream, H, Y, g, out, T,
                       n, p, eps, h_sb, h_st, y_sb, y_st, o_sb, o_st, g_sb);
  else
    smat::launch((normalise_kernel<false, Out>), grid, dim3(256), 0, stream, H, Y, g, out, T,
                       n, p, 0.f, h_sb, h_st, y_sb, y_st, o_sb, o_st, g_sb);
  return launch_status("smat_normalise");
}

int normalise_dispatch(const float* H, const float* Y, const float* g, float* out, int nb, int T,
                       int n, int p, int64_t h_sb, int64_t h_st, int64_t y_sb, int64_t y_st,
                       int64_t o_sb, int64_t o_st, int64_t g_sb, hipStream_t stream,
                       float eps) {
  return launch_normalise<float>(H, Y, g, out, nb, T, n, p, h_sb, h_st, y_sb, y_st, o_sb, o_st,
                                 g_sb, stream, eps);
}

template <typename Din>
static int launch_normalise_bwd(const Din* dout, const float* H, const float* Y, const float* g,
                                float* dH, float* dg, int nb, int T, int n, int p, float eps,
                                int64_t o_sb, int64_t o_st, int64_t h_sb, int64_t h_st,
                                int64_t y_sb, int64_t y_st, int64_t d_sb, int64_t d_st,
                                int64_t g_sb, hipStream_t stream) {
  if (nb == 0 || T == 0) return SMAT_OK;
  dim3 grid((unsigned)((T + nrm::kRows - 1) / nrm::kRows), (unsigned)nb);
  if (eps >= 0.f)
    smat::launch((normalise_bwd_kernel<true, Din>), grid, dim3(256), 0, stream, dout, H, Y,
                       g, dH, dg, T, n, p, eps, o_sb, o_st, h_sb, h_st, y_sb, y_st, d_sb, d_st,
                       g_sb);
  else
    smat::launch((normalise_bwd_kernel<false, Din>), grid, dim3(256), 0, stream, dout, H, Y,
                       g, dH, dg, T, n, p, 0.f, o_sb, o_st, h_sb, h_st, y_sb, y_st, d_sb, d_st,
                       g_sb);
  return launch_status("smat_normalise_backward");
}

}  // namespace smat

extern "C" int smat_decay_scan(const float* D, const float* aC, float* Sin, int nb, int nc,
                               int nc0, int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(D && aC && Sin && D != Sin, SMAT_EINVAL, "smat_decay_scan: null or aliased D/Sin");
  SMAT_REQUIRE(nb >= 0 && nb < 65536 && nc >= 0 && rp >= 0, SMAT_EINVAL,
               "smat_decay_scan: bad sizes");
  if (nb == 0 || nc == 0 || rp == 0) return SMAT_OK;
  dim3 grid((unsigned)((rp + 255) / 256), (unsigned)nb);
  smat::launch(decay_scan_kernel, grid, dim3(256), 0, (hipStream_t)stream, D, aC, Sin, nc,
                     nc0, rp);
  return launch_status("smat_decay_scan");
}

extern "C" int smat_decay_scan_reverse(const float* dSin, const float* aC, float* dD, int nb,
                                       int nc, int nc0, int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(dSin && aC && dD && dSin != dD, SMAT_EINVAL,
               "smat_decay_scan_reverse: null or aliased dSin/dD");
  SMAT_REQUIRE(nb >= 0 && nb < 65536 && nc >= 0 && rp >= 0, SMAT_EINVAL,
               "smat_decay_scan_reverse: bad sizes");
  if (nb == 0 || nc == 0 || rp == 0) return SMAT_OK;
  dim3 grid((unsigned)((rp + 255) / 256), (unsigned)nb);
  smat::launch(decay_scan_rev_kernel, grid, dim3(256), 0, (hipStream_t)stream, dSin, aC,
                     dD, nc, nc0, rp);
  return launch_status("smat_decay_scan_reverse");
}

extern "C" int smat_segment_scan(const float* D, float* Sin, int nb, int nc, int nc0, int64_t rp,
                                 void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(D && Sin && D != Sin, SMAT_EINVAL, "smat_segment_scan: null or aliased D/Sin");
  SMAT_REQUIRE(nb >= 0 && nc >= 0 && nc0 >= 0 && nc0 <= nc && rp >= 0, SMAT_EINVAL,
               "smat_segment_scan: need 0 <= nc0 <= nc (nc=%d nc0=%d)", nc, nc0);
  return segment_scan_dispatch(D, Sin, nb, nc, nc0, rp, (hipStream_t)stream);
}

extern "C" int smat_normalise(const float* H, const float* Y, const float* g, float* out, int nb,
                              int T, int n, int p, int64_t h_sb, int64_t h_st, int64_t y_sb,
                              int64_t y_st, int64_t o_sb, int64_t o_st, int64_t g_sb,
                              void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(H && out, SMAT_EINVAL, "smat_normalise: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && n >= 0 && n <= T && p >= 2, SMAT_EINVAL,
               "smat_normalise: bad sizes (T=%d n=%d p=%d)", T, n, p);
  SMAT_REQUIRE(h_st >= p && o_st >= p - 1, SMAT_EINVAL, "smat_normalise: row stride too short");
  return normalise_dispatch(H, Y, g, out, nb, T, n, p, h_sb, h_st, y_sb, y_st, o_sb, o_st, g_sb,
                            (hipStream_t)stream, -1.f);
}

extern "C" int smat_segment_scan_reverse(const float* D, float* Sout, int nb, int nc, int nc0,
                                         int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(D && Sout && D != Sout, SMAT_EINVAL,
               "smat_segment_scan_reverse: null or aliased D/Sout");
  SMAT_REQUIRE(nb >= 0 && nc >= 0 && nc0 >= 0 && nc0 <= nc && rp >= 0, SMAT_EINVAL,
               "smat_segment_scan_reverse: need 0 <= nc0 <= nc (nc=%d nc0=%d)", nc, nc0);
  if (nb == 0 || nc == 0 || rp == 0) return SMAT_OK;
  dim3 grid((unsigned)((rp + 255) / 256), (unsigned)nb, 2);
  smat::launch(segment_scan_rev_kernel, grid, dim3(256), 0, (hipStream_t)stream, D, Sout, nc,
                     nc0, rp);
  return launch_status("smat_segment_scan_reverse");
}

extern "C" int smat_normalise_backward(const float* dout, const float* H, const float* g,
                                       float* dH, float* dg, int nb, int T, int p, int64_t o_sb,
                                       int64_t o_st, int64_t h_sb, int64_t h_st, int64_t d_sb,
                                       int64_t d_st, int64_t g_sb, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(dout && H && dH, SMAT_EINVAL, "smat_normalise_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && p >= 2 && h_st >= p && d_st >= p && o_st >= p - 1,
               SMAT_EINVAL, "smat_normalise_backward: bad sizes");
  return launch_normalise_bwd<float>(dout, H, nullptr, g, dH, dg, nb, T, 0, p, -1.f, o_sb, o_st,
                                     h_sb, h_st, 0, 0, d_sb, d_st, g_sb, (hipStream_t)stream);
}

extern "C" int smat_combine_normalise(int out_dtype, const float* H, const float* Y, void* out,
                                      int nb, int T, int n, int p, float eps, int64_t h_sb,
                                      int64_t h_st, int64_t y_sb, int64_t y_st, int64_t o_sb,
                                      int64_t o_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(H && out, SMAT_EINVAL, "smat_combine_normalise: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && n >= 0 && n <= T && p >= 2 && eps >= 0.f, SMAT_EINVAL,
               "smat_combine_normalise: bad sizes (T=%d n=%d p=%d) or eps < 0", T, n, p);
  SMAT_REQUIRE(h_st >= p && o_st >= p - 1 && (!Y || y_st >= p), SMAT_EINVAL,
               "smat_combine_normalise: row stride too short");
  hipStream_t st = (hipStream_t)stream;
  switch (out_dtype) {
    case SMAT_F32:
      return launch_normalise<float>(H, Y, nullptr, (float*)out, nb, T, n, p, h_sb, h_st, y_sb,
                                     y_st, o_sb, o_st, 0, st, eps);
    case SMAT_BF16:
      return launch_normalise<bf16>(H, Y, nullptr, (bf16*)out, nb, T, n, p, h_sb, h_st, y_sb, y_st,
                                    o_sb, o_st, 0, st, eps);
    case SMAT_F16:
      return launch_normalise<f16>(H, Y, nullptr, (f16*)out, nb, T, n, p, h_sb, h_st, y_sb, y_st,
                                   o_sb, o_st, 0, st, eps);
  }
  set_error("smat_combine_normalise: unknown dtype %d", out_dtype);
  return SMAT_EINVAL;
}

extern "C" int smat_combine_normalise_backward(int dout_dtype, const void* dout, const float* H,
                                               const float* Y, float* dH, int nb, int T, int n,
                                               int p, float eps, int64_t o_sb, int64_t o_st,
                                               int64_t h_sb, int64_t h_st, int64_t y_sb,
                                               int64_t y_st, int64_t d_sb, int64_t d_st,
                                               void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(dout && H && dH, SMAT_EINVAL, "smat_combine_normalise_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && n >= 0 && n <= T && p >= 2 && eps >= 0.f && h_st >= p &&
                   d_st >= p && o_st >= p - 1 && (!Y || y_st >= p),
               SMAT_EINVAL, "smat_combine_normalise_backward: bad sizes");
  hipStream_t st = (hipStream_t)stream;
  switch (dout_dtype) {
    case SMAT_F32:
      return launch_normalise_bwd<float>((const float*)dout, H, Y, nullptr, dH, nullptr, nb, T, n,
                                         p, eps, o_sb, o_st, h_sb, h_st, y_sb, y_st, d_sb, d_st, 0,
                                         st);
    case SMAT_BF16:
      return launch_normalise_bwd<bf16>((const bf16*)dout, H, Y, nullptr, dH, nullptr, nb, T, n, p,
                                        eps, o_sb, o_st, h_sb, h_st, y_sb, y_st, d_sb, d_st, 0, st);
    case SMAT_F16:
      return launch_normalise_bwd<f16>((const f16*)dout, H, Y, nullptr, dH, nullptr, nb, T, n, p,
                                       eps, o_sb, o_st, h_sb, h_st, y_sb, y_st, d_sb, d_st, 0, st);
  }
  set_error("smat_combine_normalise_backward: unknown dtype %d", dout_dtype);
  return SMAT_EINVAL;
}
