// Backward of the pooled long-range branch at the training shape (16-bit
// inputs, r = 64 features, p = 65 value columns).  The forward (attention.py:
// 196-330) pools F_x = sum_{j in profile x} Psi_j^T Vb_j, sums U_h =
// sum_{x in H_h} F_x (+ F_glob), and adds Y_i = Phi_i U_{h(i)} to recent row
// i, h(i) = (i - n) mod B.  Given dY = dH on the recent rows:
//
//   smat_lr_dphi        dPhi_i += dY_i U_h^T                     per row type h
//   smat_lr_dfeat       dF_x = sum_{h : x in H_h} sum_{i in R_h} Phi_i^T dY_i
//                       (dU_h = sum_{i in R_h} Phi_i^T dY_i, then C^T dU, in
//                       one pass: dU never reaches HBM); the global channel's
//                       dF_glob = sum over every recent row
//   smat_pool_backward  dPsi_j += Vb_j dF_x^T,  dVb_j += Psi_j dF_x
//                       per profile x, dF_x read once for both
//
// Each launch streams one r x p fp32 matrix per item (U_h, dF_x) against the
// few token rows of that item -- bandwidth kernels whose waves mostly wait
// on their loads: the list gram and the pool backward cap their registers
// so five workgroups share a CU (a few spilled values; 245 -> 232 and
// 171 -> 163 us at C4 d = 3).  The products run on bf16
// MFMA with fp32 operands split hi/lo, except the query's dPhi (fp32 MFMA, see
// there).  The reference differentiates
// the query and incidence with torch and fuses the pool backward in
// src/smat/kernels/triton_bwd.py:203-237 ("dF_x loaded once"); the
// incidence backward there is the forward kernel over C^T (:262-276).
#include "bwd_common.hpp"

namespace smat {

namespace lr {
constexpr int kThreads = 256;       // four waves; wave w owns 16-wide tile w
constexpr int kRP = cb::kR * cb::kP;   // 4160 floats per r x p matrix
constexpr int kStep = 32;           // tokens per K step of the list gram
}  // namespace lr

// ---------------------------------------------------------------------------
// dPhi[n + h + kB] += dY[n + h + kB] U_h^T, one workgroup per (h, sequence).
// Wave w forms feature tile w of the transposed product, dPhi^T = U_h dY^T:
// A = U_h rows (LDS, loaded once), B = dY^T from the token rows, 16 at a time;
// lane (row, g) ends with dPhi[row][16w + 4g .. +3].
//
// This product runs on fp32 MFMA (v_mfma_f32_16x16x4_f32, k = 4j + g for
// frag element j): its sum over value columns cancels the normaliser column
// against the values (the quotient rule of the final division), and U_h holds
// large pooled sums, so hi/lo 16-bit operands (~2^-16) would leave an error
// of order 1e-3 of the result.
// ---------------------------------------------------------------------------
template <typename In>
__global__ __launch_bounds__(lr::kThreads) void lr_dphi_kernel(
    const float* __restrict__ dH, const float* __restrict__ U, float* __restrict__ dPhi,
    int T_R, int B, int n, int64_t h_sb, int64_t h_st, int64_t u_sb, int64_t d_sb,
    int64_t d_st, int accumulate) {
  using namespace cb;
  __shared__ __attribute__((aligned(16))) float sU[kR * kS];
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int cnt = h < T_R ? (T_R - h + B - 1) / B : 0;
  if (cnt == 0) return;                              // uniform over the workgroup
  cb_stage_rp(sU, U + b * u_sb + (int64_t)h * lr::kRP);
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  const int arow = 16 * w + r16;
  f32x8 ua[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int j = 0; j < 8; ++j) ua[kc][j] = sU[arow * kS + 32 * kc + 4 * j + g];
  const float ut = g == 0 ? sU[arow * kS + 64] : 0.f;   // column 64: k-slot 0 of the tail

  const float* dHb = dH + b * h_sb;
  float* dPb = dPhi + b * d_sb;
  for (int rt = 0; 16 * rt < cnt; ++rt) {
    const int k = 16 * rt + r16;
    const bool ok = k < cnt;
    const int64_t row = n + h + (int64_t)(ok ? k : 0) * B;
    const float* y = dHb + row * h_st;
    f32x4 acc = zero4();
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      f32x8 yb;
#pragma unroll
      for (int j = 0; j < 8; ++j) yb[j] = ok ? y[32 * kc + 4 * j + g] : 0.f;
      acc = mma(acc, ua[kc], yb);
    }
    const float yt = ok && g == 0 ? y[64] : 0.f;
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ut, yt, acc, 0, 0, 0);
    if (ok) {
      float4* o = reinterpret_cast<float4*>(dPb + row * d_st + 16 * w + 4 * g);
      float4 cur = accumulate ? *o : make_float4(0.f, 0.f, 0.f, 0.f);
      cur.x += acc[0];
      cur.y += acc[1];
      cur.z += acc[2];
      cur.w += acc[3];
      *o = cur;
    }
  }
}

// ---------------------------------------------------------------------------
// dF[x] = sum over the token list of item x of Phi_t^T dY_t, one workgroup
// per (item, sequence): 32 tokens a step are gathered into LDS (Phi rows
// swizzled, dY rows of kS floats; eight threads a token, the next step's
// gather in flight during the products), then D[a][c] += Phi^T dY with
// A = Phi^T by transposing reads (k-slot 8g + e = token slot) and B = dY
// columns split hi/lo.  Wave w owns value-column tile w for all four feature
// tiles; wave 0 also tile 4 (column 64).
// ---------------------------------------------------------------------------
template <typename In>
__global__ __launch_bounds__(lr::kThreads, 5) void lr_dfeat_kernel(
    const In* __restrict__ phi, const float* __restrict__ dH, const int32_t* __restrict__ tptr,
    const int32_t* __restrict__ tok, float* __restrict__ dF, int64_t q_sb, int64_t q_st,
    int64_t h_sb, int64_t h_st, int64_t f_sb) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 sPh[lr::kStep * kRowChunks];
  __shared__ __attribute__((aligned(16))) float sY[lr::kStep * kS];
  int x;
  int64_t b;
  xcd_item_seq(x, b);
  const int tid = threadIdx.x;
  const int64_t beg = tptr[x], end = tptr[x + 1];
  const In* phib = phi + b * q_sb;
  const float* dHb = dH + b * h_sb;
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;

  f32x4 acc[4], acc4[4];
#pragma unroll
  for (int at = 0; at < 4; ++at) {
    acc[at] = zero4();
    acc4[at] = zero4();
  }
  CbGather<In, float> ga;
  // plain token ids: an L above every id decodes each as (pair 0, token id)
  constexpr int kNoPair = 0x7fffffff;
  if (beg < end) ga.load(tok, beg, beg, end, kNoPair, phib, q_st, dHb, h_st, tid);
  for (int64_t s0 = beg; s0 < end; s0 += lr::kStep) {
    if (s0 > beg) __syncthreads();                   // the last step's readers are done
    {
      const int slot = tid >> 3, sub = tid & 7;
      sPh[cb_slot(slot, sub)] = ga.ok ? ga.r64 : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < CbGather<In, float>::kU; ++u) {
        const int col = sub + 8 * u;
        if (col < kP) sY[slot * kS + col] = ga.ok ? ga.r65[u] : 0.f;
      }
    }
    __syncthreads();
    if (s0 + lr::kStep < end)
      ga.load(tok, s0 + lr::kStep, beg, end, kNoPair, phib, q_st, dHb, h_st, tid);

    // B = dY (k = token slot 8g + e, n = column c)
    auto bfrag = [&](int ct, Frag& hi, Frag& lo) {
      const int col = 16 * ct + r16;
      const bool okc = col < kP;
      const int cc = okc ? col : 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = okc ? sY[(8 * g + e) * kS + cc] : 0.f;
        In hh, ll;
        split2<In>(v, hh, ll);
        hi[e] = hh;
        lo[e] = ll;
      }
    };
    Frag bh, bl;
    bfrag(w, bh, bl);
#pragma unroll
    for (int at = 0; at < 4; ++at) {
      // A = Phi^T: lane (a = 16 at + r16, g), k-slot 4h + e = token slot
      // 8g + 4h + e; lane 4e + q addresses slot 8g + 4h + e, columns
      // 16 at + 4q .. +3
      const int k = 2 * at + ((r16 & 3) >> 1), half = r16 & 1;
      const Half lo4 = cb_tr<In>(sPh, 8 * g + (r16 >> 2), k, half);
      const Half hi4 = cb_tr<In>(sPh, 8 * g + 4 + (r16 >> 2), k, half);
      Frag pa;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pa[e] = lo4[e];
        pa[4 + e] = hi4[e];
      }
      acc[at] = mma(acc[at], pa, bh);
      acc[at] = mma(acc[at], pa, bl);
      if (w == 0) {
        Frag b4h, b4l;
        bfrag(4, b4h, b4l);
        acc4[at] = mma(acc4[at], pa, b4h);
        acc4[at] = mma(acc4[at], pa, b4l);
      }
    }
  }
  // lane (c = 16 w + r16, g) holds dF[16 at + 4g + e][c]
  float* out = dF + b * f_sb + (int64_t)x * lr::kRP;
#pragma unroll
  for (int at = 0; at < 4; ++at)
#pragma unroll
    for (int e = 0; e < 4; ++e) out[(16 * at + 4 * g + e) * kP + 16 * w + r16] = acc[at][e];
  if (w == 0 && r16 == 0) {
#pragma unroll
    for (int at = 0; at < 4; ++at)
#pragma unroll
      for (int e = 0; e < 4; ++e) out[(16 * at + 4 * g + e) * kP + 64] = acc4[at][e];
  }
}

// ---------------------------------------------------------------------------
// Pool backward, one workgroup per (profile x, sequence): profile x < N0
// holds tokens n_P + x + s N0 < n; item N0 (the global channel, when n_P > 0)
// holds tokens 0 .. n_P - 1 with dF row N0 = dF_glob.  dF_x is staged once;
// wave w forms
//   dPsi^T tile w = dF_x Vb^T       (A = dF rows, B = Vb rows)
//   dVb^T  tile w = dF_x^T Psi^T    (A = dF columns, B = Psi rows)
// (wave 0 also column tile 4) for the tokens, 16 at a time, and adds them in.
// ---------------------------------------------------------------------------
template <typename In>
__global__ __launch_bounds__(lr::kThreads, 5) void lr_pool_bwd_kernel(
    const In* __restrict__ psi, const In* __restrict__ vb, const float* __restrict__ dF,
    float* __restrict__ dPsi, float* __restrict__ dVb, int N0, int n, int n_P, int64_t k_sb,
    int64_t k_st, int64_t v_sb, int64_t v_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
    int64_t e_sb, int64_t e_st, int accumulate) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) float sF[kR * kS];
  int x;
  int64_t b;
  xcd_item_seq(x, b);
  const int64_t start = x < N0 ? (int64_t)n_P + x : 0;
  const int64_t stride = x < N0 ? N0 : 1;
  const int nX = n - n_P;
  const int cnt = x < N0 ? (x < nX ? (nX - x + N0 - 1) / N0 : 0) : n_P;
  if (cnt == 0) return;                              // uniform over the workgroup
  cb_stage_rp(sF, dF + b * f_sb + (int64_t)x * lr::kRP);
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  // dPsi: A = dF rows a = 16w + r16 (hi/lo), columns 32 kc + 8g + e and 64
  Frag fh[2], fl[2];
  Half fth, ftl;
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) cb_row32<In>(sF, 16 * w + r16, kc, g, fh[kc], fl[kc]);
  cb_tail32<In>(sF, 16 * w + r16, g, fth, ftl);
  // dVb: A = dF^T rows c (value column), k = feature 32 ka + 8g + e
  auto colfrag = [&](int ct, Frag (&hi)[2], Frag (&lo)[2]) {
    const int col = 16 * ct + r16;
    const bool okc = col < kP;
    const int cc = okc ? col : 0;
#pragma unroll
    for (int ka = 0; ka < 2; ++ka)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = okc ? sF[(32 * ka + 8 * g + e) * kS + cc] : 0.f;
        In hh, ll;
        split2<In>(v, hh, ll);
        hi[ka][e] = hh;
        lo[ka][e] = ll;
      }
  };
  Frag ch[2], cl[2], c4h[2], c4l[2];
  colfrag(w, ch, cl);
  if (w == 0) colfrag(4, c4h, c4l);

  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;
  float* dPb = dPsi + b * d_sb;
  float* dVbb = dVb + b * e_sb;
  for (int rt = 0; 16 * rt < cnt; ++rt) {
    const int k = 16 * rt + r16;
    const bool ok = k < cnt;
    const int64_t j = start + (int64_t)(ok ? k : 0) * stride;
    // B operands along this lane's token row j
    Frag vf[2], pf[2];
    Half vt;
    const In* vrow = vbb + j * v_st;
    const In* prow = psib + j * k_st;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const Frag pv = *reinterpret_cast<const Frag*>(prow + 32 * kc + 8 * g);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vf[kc][e] = ok ? vrow[32 * kc + 8 * g + e] : from_f32<In>(0.f);
        pf[kc][e] = ok ? pv[e] : from_f32<In>(0.f);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) vt[e] = from_f32<In>(0.f);
    if (ok && g == 0) vt[0] = vrow[64];

    f32x4 ap = zero4(), av = zero4(), av4 = zero4();
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      ap = mma(ap, fh[kc], vf[kc]);
      ap = mma(ap, fl[kc], vf[kc]);
      av = mma(av, ch[kc], pf[kc]);
      av = mma(av, cl[kc], pf[kc]);
      if (w == 0) {
        av4 = mma(av4, c4h[kc], pf[kc]);
        av4 = mma(av4, c4l[kc], pf[kc]);
      }
    }
    ap = mma_k16(ap, fth, vt);
    ap = mma_k16(ap, ftl, vt);
    if (ok) {
      // lane (j, g): dPsi[j][16w + 4g + e], dVb[j][16w + 4g + e] (and dVb[j][64])
      float4* o = reinterpret_cast<float4*>(dPb + j * d_st + 16 * w + 4 * g);
      float4 cur = accumulate ? *o : make_float4(0.f, 0.f, 0.f, 0.f);
      cur.x += ap[0];
      cur.y += ap[1];
      cur.z += ap[2];
      cur.w += ap[3];
      *o = cur;
      float* ov = dVbb + j * e_st + 16 * w + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = (accumulate ? ov[e] : 0.f) + av[e];
      if (w == 0 && g == 0) dVbb[j * e_st + 64] = (accumulate ? dVbb[j * e_st + 64] : 0.f) + av4[0];
    }
  }
}

static bool lr_shape_ok(int dtype, int r, int p) {
  return (dtype == SMAT_BF16 || dtype == SMAT_F16) && r == cb::kR && p == cb::kP;
}

}  // namespace smat

extern "C" int smat_lr_dphi(int dtype, const float* dH, const float* U, float* dPhi, int nb,
                            int T_R, int B, int n, int r, int p, int64_t h_sb, int64_t h_st,
                            int64_t u_sb, int64_t d_sb, int64_t d_st, int accumulate,
                            void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(dH && U && dPhi, SMAT_EINVAL, "smat_lr_dphi: null pointer");
  SMAT_REQUIRE(nb >= 0 && T_R >= 0 && B >= 1 && n >= 0, SMAT_EINVAL, "smat_lr_dphi: bad sizes");
  SMAT_REQUIRE(lr_shape_ok(dtype, r, p), SMAT_EUNSUPPORTED,
               "smat_lr_dphi: needs dtype bf16/f16, r=64, p=65 (got %d, %d, %d)", dtype, r, p);
  SMAT_REQUIRE(aligned16(U) && u_sb % 4 == 0 && rows_vec_ok(dPhi, d_sb, d_st, 4) &&
                   h_st >= p && d_st >= r,
               SMAT_EINVAL, "smat_lr_dphi: U and dPhi rows must be 16-byte aligned");
  SMAT_REQUIRE(B < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED, "smat_lr_dphi: grid too large");
  if (nb == 0 || T_R == 0) return SMAT_OK;
  const dim3 grid((unsigned)B, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SMAT_BF16)
    hipLaunchKernelGGL(lr_dphi_kernel<bf16>, grid, dim3(lr::kThreads), 0, st, dH, U, dPhi, T_R, B,
                       n, h_sb, h_st, u_sb, d_sb, d_st, accumulate);
  else
    hipLaunchKernelGGL(lr_dphi_kernel<f16>, grid, dim3(lr::kThreads), 0, st, dH, U, dPhi, T_R, B,
                       n, h_sb, h_st, u_sb, d_sb, d_st, accumulate);
  return launch_status("smat_lr_dphi");
}

extern "C" int smat_lr_dfeat(int dtype, const void* phi, const float* dH, const int32_t* tptr,
                             const int32_t* tok, float* dF, int nb, int nitems, int r, int p,
                             int64_t q_sb, int64_t q_st, int64_t h_sb, int64_t h_st, int64_t f_sb,
                             void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && dH && tptr && tok && dF, SMAT_EINVAL, "smat_lr_dfeat: null pointer");
  SMAT_REQUIRE(nb >= 0 && nitems >= 0, SMAT_EINVAL, "smat_lr_dfeat: bad sizes");
  SMAT_REQUIRE(lr_shape_ok(dtype, r, p), SMAT_EUNSUPPORTED,
               "smat_lr_dfeat: needs dtype bf16/f16, r=64, p=65 (got %d, %d, %d)", dtype, r, p);
  SMAT_REQUIRE(rows_vec_ok(phi, q_sb, q_st, 2) && h_st >= p && f_sb >= (int64_t)nitems * r * p,
               SMAT_EINVAL, "smat_lr_dfeat: Phi rows must be 16-byte aligned");
  SMAT_REQUIRE(nitems < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_lr_dfeat: grid too large");
  if (nb == 0 || nitems == 0) return SMAT_OK;
  const dim3 grid((unsigned)nitems, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SMAT_BF16)
    hipLaunchKernelGGL(lr_dfeat_kernel<bf16>, grid, dim3(lr::kThreads), 0, st, (const bf16*)phi,
                       dH, tptr, tok, dF, q_sb, q_st, h_sb, h_st, f_sb);
  else
    hipLaunchKernelGGL(lr_dfeat_kernel<f16>, grid, dim3(lr::kThreads), 0, st, (const f16*)phi,
                       dH, tptr, tok, dF, q_sb, q_st, h_sb, h_st, f_sb);
  return launch_status("smat_lr_dfeat");
}

extern "C" int smat_pool_backward(int dtype, const void* psi, const void* vb, const float* dF,
                                  float* dPsi, float* dVb, int nb, int N0, int n, int n_P, int r,
                                  int p, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                                  int64_t f_sb, int64_t d_sb, int64_t d_st, int64_t e_sb,
                                  int64_t e_st, int accumulate, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && dF && dPsi && dVb, SMAT_EINVAL, "smat_pool_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && n_P >= 0 && n >= n_P, SMAT_EINVAL,
               "smat_pool_backward: bad sizes");
  SMAT_REQUIRE(lr_shape_ok(dtype, r, p), SMAT_EUNSUPPORTED,
               "smat_pool_backward: needs dtype bf16/f16, r=64, p=65 (got %d, %d, %d)", dtype, r,
               p);
  SMAT_REQUIRE(rows_vec_ok(psi, k_sb, k_st, 2) && rows_vec_ok(dPsi, d_sb, d_st, 4) &&
                   aligned16(dF) && f_sb % 4 == 0 && v_st >= p && e_st >= p && d_st >= r,
               SMAT_EINVAL, "smat_pool_backward: Psi, dPsi and dF must be 16-byte aligned");
  const int nitems = N0 + (n_P > 0 ? 1 : 0);
  SMAT_REQUIRE(nitems < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_pool_backward: grid too large");
  if (nb == 0) return SMAT_OK;
  const dim3 grid((unsigned)nitems, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SMAT_BF16)
    hipLaunchKernelGGL(lr_pool_bwd_kernel<bf16>, grid, dim3(lr::kThreads), 0, st,
                       (const bf16*)psi, (const bf16*)vb, dF, dPsi, dVb, N0, n, n_P, k_sb, k_st,
                       v_sb, v_st, f_sb, d_sb, d_st, e_sb, e_st, accumulate);
  else
    hipLaunchKernelGGL(lr_pool_bwd_kernel<f16>, grid, dim3(lr::kThreads), 0, st, (const f16*)psi,
                       (const f16*)vb, dF, dPsi, dVb, N0, n, n_P, k_sb, k_st, v_sb, v_st, f_sb,
                       d_sb, d_st, e_sb, e_st, accumulate);
  return launch_status("smat_pool_backward");
}
