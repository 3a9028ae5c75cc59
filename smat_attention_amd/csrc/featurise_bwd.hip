// Backward of the feature map (src/smat/attention.py:82-106) for one map at
// d_qk = r = 64 with 16-bit inputs -- the training shape:
//
//   y = x W^T (fp32),  g = G * m'(y) (* h),  dx = g W,  dW += g^T x,
//   dh = sum_f G * m(y)          (the gated key map only)
//
// with m(y) = elu(y) + 1, m'(y) = 1 (y > 0) or e^y (kind 0), or m(y) =
// relu(y) + 1e-3, m'(y) = [y > 0] (kind 1); G is the upstream gradient of the
// map's output (dPhi, or dPsi before the gate).  Persistent workgroups of four
// waves stage W once and walk 64-token tiles: x, G (and h) through LDS, the
// next tile's rows in flight while the current tile is multiplied.  Wave w:
//
//   * forms y^T for its 16 tokens (A = W rows, B = x rows; lane (t, g) holds
//     features 4g + i of each feature tile), applies m' and the gate, and
//     feeds the two-tile pairs, split hi/lo, as the B operand of
//     dx^T = W^T g^T (A = W^T by transposing reads); lane (t, g) ends with
//     dx[t][16 dt + 4g .. +3];
//   * forms y for feature tile w over the tile's 64 tokens (A = x rows,
//     B = W rows; lane (f, g) holds tokens 4g + i) and adds
//     dW^T = x^T g (A = x^T by transposing reads) to its accumulators.
//
// The per-workgroup dW partials go to a buffer that a second launch sums.
// y is fp32 from exact 16-bit products; g is split hi/lo (~2^-17) against
// the exact 16-bit W and x.
#include <math.h>

#include "bwd_common.hpp"

namespace smat {

namespace fb {
constexpr int kThreads = 256;
constexpr int kTile = 64;          // tokens a tile
constexpr int kD = 64;             // d_qk = r
}  // namespace fb

template <typename In>
__global__ __launch_bounds__(fb::kThreads) void featurise_bwd_kernel(
    const In* __restrict__ x, const In* __restrict__ G, const In* __restrict__ W,
    const In* __restrict__ h, In* __restrict__ dx, float* __restrict__ dWp, In* __restrict__ dh,
    int T, int kind, int64_t ntiles, int64_t x_sb, int64_t x_st, int64_t g_sb, int64_t g_st,
    int64_t h_sb, int64_t o_sb, int64_t o_st, int64_t dh_sb) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 sW[fb::kD * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sX[fb::kTile * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sG[fb::kTile * kRowChunks];
  __shared__ float sH[fb::kTile];
  const int tid = threadIdx.x;
  for (int i = tid; i < fb::kD * kRowChunks; i += fb::kThreads)
    sW[cb_slot(i >> 3, i & 7)] = reinterpret_cast<const uint4*>(W)[i];

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  const int tiles_per_seq = (T + fb::kTile - 1) / fb::kTile;
  f32x4 accW[4];                                     // dW^T[d = 16 dt + 4g + i][f = 16w + r16]
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) accW[dt] = zero4();

  auto dmap = [&](float y) {
    return kind == 0 ? (y > 0.f ? 1.f : expf(y)) : (y > 0.f ? 1.f : 0.f);
  };
  auto fmap = [&](float y) {
    return kind == 0 ? (y > 0.f ? y : expm1f(y)) + 1.f : fmaxf(y, 0.f) + 1e-3f;
  };

  // x and G rows of a tile (16-byte chunks; rows past T are zero) and the
  // gate: the next tile's are loaded into registers while the current one
  // is multiplied, and written to LDS at the top of the next iteration
  constexpr int kChunks = fb::kTile * kRowChunks / fb::kThreads;    // 2 a thread
  uint4 px[kChunks], pg[kChunks];
  float ph = 1.f;
  auto issue = [&](int64_t tile) {
    const int64_t b = tile / tiles_per_seq;
    const int t0 = (int)(tile - b * tiles_per_seq) * fb::kTile;
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int i = tid + fb::kThreads * u;
      const int row = i >> 3, k = i & 7;
      const bool ok = t0 + row < T;
      const int64_t t = ok ? t0 + row : t0;
      px[u] = *reinterpret_cast<const uint4*>(x + b * x_sb + t * x_st + 8 * k);
      pg[u] = *reinterpret_cast<const uint4*>(G + b * g_sb + t * g_st + 8 * k);
      if (!ok) px[u] = pg[u] = make_uint4(0, 0, 0, 0);
    }
    if (tid < fb::kTile) {
      const bool ok = t0 + tid < T;
      ph = h && ok ? to_f32(h[b * h_sb + t0 + tid]) : 1.f;
    }
  };
  if ((int64_t)blockIdx.x < ntiles) issue(blockIdx.x);
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t b = tile / tiles_per_seq;
    const int t0 = (int)(tile - b * tiles_per_seq) * fb::kTile;
    __syncthreads();                                 // W staged / the last tile's readers done
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int i = tid + fb::kThreads * u;
      sX[cb_slot(i >> 3, i & 7)] = px[u];
      sG[cb_slot(i >> 3, i & 7)] = pg[u];
    }
    if (tid < fb::kTile) sH[tid] = ph;
    __syncthreads();
    if (tile + gridDim.x < ntiles) issue(tile + gridDim.x);

    // ---- dx and dh for tokens 16w .. 16w+15 of the tile -------------------
    {
      const int trow = 16 * w + r16;
      const float hv = sH[trow];
      f32x4 gq[4];
      float dhs = 0.f;
#pragma unroll
      for (int ft = 0; ft < 4; ++ft) {
        f32x4 y = zero4();
#pragma unroll
        for (int kd = 0; kd < 2; ++kd)
          y = mma(y, cb_row<In>(sW, ft, kd, lane), cb_row<In>(sX, w, kd, lane));
        // lane (t, g) holds y[t][16 ft + 4g + i]; G at the same features
        const Half gv = *reinterpret_cast<const Half*>(
            reinterpret_cast<const char*>(sG + cb_slot(trow, 2 * ft + (g >> 1))) + 8 * (g & 1));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gi = to_f32(gv[i]);
          if (h) dhs += gi * fmap(y[i]);
          gq[ft][i] = gi * hv * dmap(y[i]);
        }
      }
      if (h) {
        dhs += __shfl_xor(dhs, 16);
        dhs += __shfl_xor(dhs, 32);
        if (g == 0 && t0 + trow < T) dh[b * dh_sb + t0 + trow] = from_f32<In>(dhs);
      }
      f32x4 ax[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) ax[dt] = zero4();
#pragma unroll
      for (int fp = 0; fp < 2; ++fp) {
        Frag bh, bl;
        cb_split_pair<In>(gq[2 * fp], gq[2 * fp + 1], bh, bl);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const Frag wa = cb_tr_pair<In>(sW, 2 * fp, 2 * fp + 1, dt, lane);
          ax[dt] = mma(ax[dt], wa, bh);
          ax[dt] = mma(ax[dt], wa, bl);
        }
      }
      if (t0 + trow < T) {
        In* o = dx + b * o_sb + (int64_t)(t0 + trow) * o_st;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          Half v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = from_f32<In>(ax[dt][i]);
          *reinterpret_cast<Half*>(o + 16 * dt + 4 * g) = v;
        }
      }
    }

    // ---- dW for features 16w .. 16w+15 over the tile's 64 tokens -----------
    {
      const int frow = 16 * w + r16;
      f32x4 gt[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        f32x4 y = zero4();
#pragma unroll
        for (int kd = 0; kd < 2; ++kd)
          y = mma(y, cb_row<In>(sX, tt, kd, lane), cb_row<In>(sW, w, kd, lane));
        // lane (f, g) holds y[t = 16 tt + 4g + i][f]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * tt + 4 * g + i;
          const In gv = reinterpret_cast<const In*>(sG + cb_slot(t, frow >> 3))[frow & 7];
          gt[tt][i] = to_f32(gv) * sH[t] * dmap(y[i]);
        }
      }
#pragma unroll
      for (int tp = 0; tp < 2; ++tp) {
        Frag bh, bl;
        cb_split_pair<In>(gt[2 * tp], gt[2 * tp + 1], bh, bl);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const Frag xa = cb_tr_pair<In>(sX, 2 * tp, 2 * tp + 1, dt, lane);
          accW[dt] = mma(accW[dt], xa, bh);
          accW[dt] = mma(accW[dt], xa, bl);
        }
      }
    }
  }
  // partial dW of this workgroup: dWp[block][f][d], lane (f, g) holds d = 16 dt + 4g + i
  float* o = dWp + (int64_t)blockIdx.x * fb::kD * fb::kD + (16 * w + r16) * fb::kD;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    *reinterpret_cast<float4*>(o + 16 * dt + 4 * g) =
        make_float4(accW[dt][0], accW[dt][1], accW[dt][2], accW[dt][3]);
}

// dW[i] = (sum over parts of dWp[part][i]) (+ dW[i] when accumulating), fp32.
// A workgroup owns 64 consecutive i (one coalesced 256-byte run per part);
// its 16 waves take parts w, w + 16, ... with four independent loads in
// flight, and the 16 partial sums meet in LDS, in a fixed order.
__global__ __launch_bounds__(1024) void featurise_dw_reduce_kernel(const float* __restrict__ dWp,
                                                                   float* __restrict__ dW,
                                                                   int nparts, int n, int beta) {
  __shared__ float red[16][64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (i < n) {
    int p = w;
    for (; p + 48 < nparts; p += 64) {
      const float a = dWp[(int64_t)p * n + i], b = dWp[(int64_t)(p + 16) * n + i];
      const float c = dWp[(int64_t)(p + 32) * n + i], d = dWp[(int64_t)(p + 48) * n + i];
      s += (a + b) + (c + d);
    }
    for (; p < nparts; p += 16) s += dWp[(int64_t)p * n + i];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && i < n) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += red[k][lane];
    dW[i] = beta ? dW[i] + t : t;
  }
}

}  // namespace smat

extern "C" int64_t smat_featurise_backward_parts(int nb, int T) {
  using namespace smat;
  if (nb <= 0 || T <= 0) return 0;
  const int64_t ntiles = (int64_t)nb * ((T + fb::kTile - 1) / fb::kTile);
  // as many workgroups as the device holds at once (each walks its tiles)
  int dev = 0, ncu = 256, per_cu = 0;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, featurise_bwd_kernel<bf16>,
                                                   fb::kThreads, 0) != hipSuccess || per_cu < 1)
    per_cu = 2;
  const int64_t cap = (int64_t)ncu * per_cu;
  return ntiles < cap ? ntiles : cap;
}

extern "C" int smat_featurise_backward(int dtype, const void* x, const void* G, const void* W,
                                       const void* h, void* dx, float* dWp, float* dW, void* dh,
                                       int nb, int T, int d_qk, int r, int kind, int beta,
                                       int64_t x_sb, int64_t x_st, int64_t g_sb, int64_t g_st,
                                       int64_t h_sb, int64_t o_sb, int64_t o_st, int64_t dh_sb,
                                       void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(x && G && W && dx && dWp && dW && (!h || dh), SMAT_EINVAL,
               "smat_featurise_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && (kind == 0 || kind == 1) && (beta == 0 || beta == 1),
               SMAT_EINVAL, "smat_featurise_backward: bad sizes, kind or beta");
  SMAT_REQUIRE((dtype == SMAT_BF16 || dtype == SMAT_F16) && d_qk == fb::kD && r == fb::kD,
               SMAT_EUNSUPPORTED,
               "smat_featurise_backward: needs dtype bf16/f16 and d_qk = r = 64 (got %d, %d, %d)",
               dtype, d_qk, r);
  SMAT_REQUIRE(rows_vec_ok(x, x_sb, x_st, 2) && rows_vec_ok(G, g_sb, g_st, 2) && aligned16(W) &&
                   (o_st % 4 == 0) && (o_sb % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(dx) & 7) == 0 && aligned16(dWp),
               SMAT_EINVAL, "smat_featurise_backward: rows must be 16-byte aligned");
  const int64_t parts = smat_featurise_backward_parts(nb, T);
  hipStream_t st = (hipStream_t)stream;
  if (parts > 0) {
    const int64_t ntiles = (int64_t)nb * ((T + fb::kTile - 1) / fb::kTile);
    const dim3 grid((unsigned)parts);
    if (dtype == SMAT_BF16)
      hipLaunchKernelGGL(featurise_bwd_kernel<bf16>, grid, dim3(fb::kThreads), 0, st,
                         (const bf16*)x, (const bf16*)G, (const bf16*)W, (const bf16*)h,
                         (bf16*)dx, dWp, (bf16*)dh, T, kind, ntiles, x_sb, x_st, g_sb, g_st, h_sb,
                         o_sb, o_st, dh_sb);
    else
      hipLaunchKernelGGL(featurise_bwd_kernel<f16>, grid, dim3(fb::kThreads), 0, st,
                         (const f16*)x, (const f16*)G, (const f16*)W, (const f16*)h, (f16*)dx,
                         dWp, (f16*)dh, T, kind, ntiles, x_sb, x_st, g_sb, g_st, h_sb, o_sb, o_st,
                         dh_sb);
    int rc = launch_status("smat_featurise_backward");
    if (rc != SMAT_OK) return rc;
  }
  const int n = fb::kD * fb::kD;
  hipLaunchKernelGGL(featurise_dw_reduce_kernel, dim3((n + 63) / 64), dim3(1024), 0, st, dWp, dW,
                     (int)parts, n, beta);
  return launch_status("smat_featurise_backward");
}
