// Gradients of the content-addressed point read and pool at the training
// shape (16-bit Phi, Psi, Vb; r = 64, p = 65; fp32 tables), for the hard
// forward of ContentAssign (assign.py:431-441 at anneal = 1): every token j
// carries K (cell, weight) pairs whose forward weights are the one-hot of
// its chosen cell (pair 0), and whose weights still take gradients.
//
//   read   y_i = Phi_i F[c_i]  ->  v = F[x] dy_i for every pair (i, k) with
//          cell x:  dPhi_i = v (pair 0),  dw_ik = Phi_i . v,
//          dF[x] = sum over pair-0 entries of Phi_i^T dy_i
//   pool   F[x] = sum_{c_j = x} Psi_j^T Vb_j  ->  v = dF[x] Vb_j:
//          dPsi_j = v, dVb_j = Psi_j dF[x] (pair 0),  dw_jk = Psi_j . v
//
// One workgroup of four waves per (sequence, cell), over the CSR list of the
// (token, pair) entries that point at the cell, numbered pair * L + token so
// that the pair-0 entries come first: a step of entries with no pair-0 entry
// skips the work only pair-0 entries need (the read's dF Gram, the pool's
// dVb products), seven eighths of the steps at 2^3 pairs a token; the cell's r x p table is
// staged in LDS once.  Four workgroups share a CU (registers capped at 128
// a lane): their waves spend most of their time waiting on the gathers, and
// a fourth workgroup hides more of it (the read kernel ran 430 us at three,
// 367 us at four at C4 d = 3).  The products against the table run on fp32 MFMA
// (v_mfma_f32_16x16x4_f32; frag element j holds k = 4j + g): their sums over
// value columns cancel the normaliser column against the values, which a
// hi/lo 16-bit split would not resolve.  dF, a sum over tokens per column,
// runs on 16-bit MFMA with dy split hi/lo, like the pool.
#include "bwd_common.hpp"

namespace smat {

namespace cw {
constexpr int kThreads = 256;
constexpr int kRP = cb::kR * cb::kP;      // 4160
constexpr int kStep = 32;                 // entries a step (read backward)
}  // namespace cw

// ---------------------------------------------------------------------------
// Read backward.  Per step of 32 entries: the entries' Phi rows (LDS,
// swizzled 128-byte rows) and dy rows (fp32 rows of kS), token and pair.
// Wave w forms feature tile w of v^T = F dy^T for two 16-entry tiles (A = F
// rows, loaded once; B = dy rows), stores dPhi for pair-0 entries and reduces
// Phi . v over the lane groups and, through LDS, the waves.  The dF Gram over
// the step's pair-0 entries follows (A = Phi^T by transposing reads, B = dy
// columns split hi/lo, zero for other pairs): wave w owns value-column tile
// w, wave 0 also tile 4 (column 64).
// ---------------------------------------------------------------------------
template <typename In, typename Out>
__global__ __launch_bounds__(cw::kThreads, 4) void cell_read_bwd_kernel(
    const In* __restrict__ phr, const float* __restrict__ dY, const float* __restrict__ F,
    const int32_t* __restrict__ ent, const int64_t* __restrict__ eoffs, Out* __restrict__ dPhi,
    float* __restrict__ dF, float* __restrict__ dw, int N0, int K, int L, int64_t q_sb,
    int64_t q_st, int64_t y_sb, int64_t y_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
    int64_t w_sb) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) float sF[kR * kS];
  __shared__ __attribute__((aligned(16))) uint4 sPh[cw::kStep * kRowChunks];
  __shared__ __attribute__((aligned(16))) float sY[cw::kStep * kS];
  __shared__ float sDotB[2][4][cw::kStep];
  __shared__ int sTokB[2][cw::kStep], sPairB[2][cw::kStep];

  int x;
  int64_t b;
  xcd_item_seq(x, b);
  const int tid = threadIdx.x;
  const int64_t beg = eoffs[b * N0 + x], end = eoffs[b * N0 + x + 1];
  const In* phb = phr + b * q_sb;
  const float* dYb = dY + b * y_sb;
  CbGather<In, float> ga;
  if (beg < end) ga.load(ent, beg, beg, end, L, phb, q_st, dYb, y_st, tid);
  cb_stage_rp(sF, F + b * f_sb + (int64_t)x * cw::kRP);
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  f32x8 fa[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int j = 0; j < 8; ++j) fa[kc][j] = sF[(16 * w + r16) * kS + 32 * kc + 4 * j + g];
  const float fat = g == 0 ? sF[(16 * w + r16) * kS + 64] : 0.f;

  Out* dPb = dPhi + b * d_sb;
  float* dwb = dw + b * w_sb;
  f32x4 acc[4], acc4[4];
#pragma unroll
  for (int at = 0; at < 4; ++at) {
    acc[at] = zero4();
    acc4[at] = zero4();
  }
  for (int64_t s0 = beg; s0 < end; s0 += cw::kStep) {
    const int par = (int)(((s0 - beg) / cw::kStep) & 1);
    float (*sDot)[cw::kStep] = sDotB[par];
    int* sTok = sTokB[par];
    int* sPair = sPairB[par];
    {
      const int slot = tid >> 3, sub = tid & 7;
      sPh[cb_slot(slot, sub)] = ga.ok ? ga.r64 : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < CbGather<In, float>::kU; ++u) {
        const int col = sub + 8 * u;
        if (col < kP) sY[slot * kS + col] = ga.ok ? ga.r65[u] : 0.f;
      }
      if (sub == 0) {
        sTok[slot] = ga.ok ? ga.tok : -1;
        sPair[slot] = ga.pair;
      }
    }
    __syncthreads();
    if (s0 + cw::kStep < end) ga.load(ent, s0 + cw::kStep, beg, end, L, phb, q_st, dYb, y_st, tid);
    const bool has0 = sPair[0] == 0;                 // uniform: entry 0 of the step is valid

    // v = F dy for the two 16-entry tiles; dPhi (pair 0) and Phi . v
#pragma unroll
    for (int et = 0; et < 2; ++et) {
      const int es = 16 * et + r16;
      f32x4 v = zero4();
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        f32x8 yb;
#pragma unroll
        for (int j = 0; j < 8; ++j) yb[j] = sY[es * kS + 32 * kc + 4 * j + g];
        v = mma(v, fa[kc], yb);
      }
      v = __builtin_amdgcn_mfma_f32_16x16x4f32(fat, g == 0 ? sY[es * kS + 64] : 0.f, v, 0, 0, 0);
      // lane (es, g) holds v[16w + 4g + i]; Phi of the entry at the same columns
      const Half ph = *reinterpret_cast<const Half*>(
          reinterpret_cast<const char*>(sPh + cb_slot(es, 2 * w + (g >> 1))) + 8 * (g & 1));
      float pd = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) pd += to_f32(ph[i]) * v[i];
      pd = cb_sum_groups(pd);
      if (g == 0) sDot[w][es] = pd;
      const int t = sTok[es];
      if (t >= 0 && sPair[es] == 0) store_grad4(dPb + (int64_t)t * d_st + 16 * w + 4 * g, v);
    }

    // dF += Phi^T dy over the pair-0 entries of the step
    auto bfrag = [&](int ct, Frag& hi, Frag& lo) {
      const int col = 16 * ct + r16;
      const bool okc = col < kP;
      const int cc = okc ? col : 0;
#pragma unroll
      for (int e8 = 0; e8 < 8; ++e8) {
        const int es = 8 * g + e8;
        const bool use = okc && sTok[es] >= 0 && sPair[es] == 0;
        const float v = use ? sY[es * kS + cc] : 0.f;
        In hh, ll;
        split2<In>(v, hh, ll);
        hi[e8] = hh;
        lo[e8] = ll;
      }
    };
    if (has0) {                                      // steps past the pair-0 entries add nothing
      Frag bh, bl;
      bfrag(w, bh, bl);
#pragma unroll
      for (int at = 0; at < 4; ++at) {
        const int k = 2 * at + ((r16 & 3) >> 1), half = r16 & 1;
        const Half lo4 = cb_tr<In>(sPh, 8 * g + (r16 >> 2), k, half);
        const Half hi4 = cb_tr<In>(sPh, 8 * g + 4 + (r16 >> 2), k, half);
        Frag pa;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pa[i] = lo4[i];
          pa[4 + i] = hi4[i];
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
    __syncthreads();                                 // sDot complete; LDS free for the next step
    if (tid < cw::kStep && sTok[tid] >= 0)
      dwb[(int64_t)sTok[tid] * K + sPair[tid]] =
          (sDot[0][tid] + sDot[1][tid]) + (sDot[2][tid] + sDot[3][tid]);
  }
  // lane (c = 16w + r16, g) holds dF[16 at + 4g + i][c]
  float* out = dF + b * f_sb + (int64_t)x * cw::kRP;
#pragma unroll
  for (int at = 0; at < 4; ++at)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(16 * at + 4 * g + i) * kP + 16 * w + r16] = acc[at][i];
  if (w == 0 && r16 == 0) {
#pragma unroll
    for (int at = 0; at < 4; ++at)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[(16 * at + 4 * g + i) * kP + 64] = acc4[at][i];
  }
}

// ---------------------------------------------------------------------------
// Pool backward.  dF[x] staged once; per step of 32 entries, their Psi and Vb
// rows are staged as fp32 rows of kS (LDS).  Wave w forms feature tile w of
// v^T = dF Vb^T (A = dF rows) and value-column tile w of dVb^T = dF^T Psi^T
// (A = dF columns; wave 0 also column 64) for two 16-entry tiles, stores dPsi
// and dVb for pair-0 entries and Psi . v for every entry.
// ---------------------------------------------------------------------------
template <typename In, typename Out>
__global__ __launch_bounds__(cw::kThreads, 4) void cell_pool_bwd_kernel(
    const In* __restrict__ psi, const In* __restrict__ vb, const float* __restrict__ dF,
    const int32_t* __restrict__ ent, const int64_t* __restrict__ eoffs, Out* __restrict__ dPsi,
    Out* __restrict__ dVb, float* __restrict__ dw, int N0, int K, int L, int64_t k_sb,
    int64_t k_st, int64_t v_sb, int64_t v_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
    int64_t e_sb, int64_t e_st, int64_t w_sb) {
  using namespace cb;
  __shared__ __attribute__((aligned(16))) float sF[kR * kS];
  __shared__ __attribute__((aligned(16))) float sP[cw::kStep * kS];
  __shared__ __attribute__((aligned(16))) float sV[cw::kStep * kS];
  __shared__ float sDotB[2][4][cw::kStep];
  __shared__ int sTokB[2][cw::kStep], sPairB[2][cw::kStep];
  int x;
  int64_t b;
  xcd_item_seq(x, b);
  const int tid = threadIdx.x;
  const int64_t beg = eoffs[b * N0 + x], end = eoffs[b * N0 + x + 1];
  if (beg == end) return;                            // uniform over the workgroup
  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;
  CbGather<In, In> ga;
  ga.load(ent, beg, beg, end, L, psib, k_st, vbb, v_st, tid);
  cb_stage_rp(sF, dF + b * f_sb + (int64_t)x * cw::kRP);
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  // A operands: dF rows a = 16w + r16 (for v) and dF columns c = 16w + r16
  // (for dVb; wave 0 also c = 64 + r16, of which only 64 exists)
  f32x8 fr[2], fc[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      fr[kc][j] = sF[(16 * w + r16) * kS + 32 * kc + 4 * j + g];
      fc[kc][j] = sF[(32 * kc + 4 * j + g) * kS + 16 * w + r16];
    }
  const float frt = g == 0 ? sF[(16 * w + r16) * kS + 64] : 0.f;

  Out* dPb = dPsi + b * d_sb;
  Out* dVbb = dVb + b * e_sb;
  float* dwb = dw + b * w_sb;
  for (int64_t s0 = beg; s0 < end; s0 += cw::kStep) {
    const int par = (int)(((s0 - beg) / cw::kStep) & 1);
    float (*sDot)[cw::kStep] = sDotB[par];
    int* sTok = sTokB[par];
    int* sPair = sPairB[par];
    {
      const int slot = tid >> 3, sub = tid & 7;
      const typename Traits<In>::frag pv = __builtin_bit_cast(typename Traits<In>::frag, ga.r64);
#pragma unroll
      for (int i = 0; i < 8; ++i) sP[slot * kS + 8 * sub + i] = ga.ok ? to_f32(pv[i]) : 0.f;
#pragma unroll
      for (int u = 0; u < CbGather<In, In>::kU; ++u) {
        const int col = sub + 8 * u;
        if (col < kP) sV[slot * kS + col] = ga.ok ? to_f32(ga.r65[u]) : 0.f;
      }
      if (sub == 0) {
        sTok[slot] = ga.ok ? ga.tok : -1;
        sPair[slot] = ga.pair;
      }
    }
    __syncthreads();
    if (s0 + cw::kStep < end) ga.load(ent, s0 + cw::kStep, beg, end, L, psib, k_st, vbb, v_st, tid);
    const bool has0 = sPair[0] == 0;                 // uniform: entry 0 of the step is valid

#pragma unroll
    for (int et = 0; et < 2; ++et) {
      const int es = 16 * et + r16;
      f32x4 v = zero4(), dv = zero4();
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        f32x8 vbf, psf;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          vbf[j] = sV[es * kS + 32 * kc + 4 * j + g];
          psf[j] = sP[es * kS + 32 * kc + 4 * j + g];
        }
        v = mma(v, fr[kc], vbf);
        if (has0) dv = mma(dv, fc[kc], psf);         // dVb: pair-0 entries only
      }
      v = __builtin_amdgcn_mfma_f32_16x16x4f32(frt, g == 0 ? sV[es * kS + 64] : 0.f, v, 0, 0, 0);
      // lane (es, g): v[16w + 4g + i] (dPsi), dv[16w + 4g + i] (dVb columns)
      float pd = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) pd += sP[es * kS + 16 * w + 4 * g + i] * v[i];
      pd = cb_sum_groups(pd);
      if (g == 0) sDot[w][es] = pd;
      const int t = sTok[es];
      if (t >= 0 && sPair[es] == 0) {
        store_grad4(dPb + (int64_t)t * d_st + 16 * w + 4 * g, v);
        Out* ov = dVbb + (int64_t)t * e_st + 16 * w + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = from_f32<Out>(dv[i]);
      }
      if (w == 0 && has0) {
        // column 64 of dVb: sum_a dF[a][64] Psi[a] (lane group 0, slot 0)
        f32x4 d4 = zero4();
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          f32x8 a4, psf;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            a4[j] = r16 == 0 ? sF[(32 * kc + 4 * j + g) * kS + 64] : 0.f;
            psf[j] = sP[es * kS + 32 * kc + 4 * j + g];
          }
          d4 = mma(d4, a4, psf);
        }
        if (g == 0 && t >= 0 && sPair[es] == 0) dVbb[(int64_t)t * e_st + 64] = from_f32<Out>(d4[0]);
      }
    }
    __syncthreads();                                 // sDot complete; LDS free for the next step
    if (tid < cw::kStep && sTok[tid] >= 0)
      dwb[(int64_t)sTok[tid] * K + sPair[tid]] =
          (sDot[0][tid] + sDot[1][tid]) + (sDot[2][tid] + sDot[3][tid]);
  }
}

static bool cw_ok(int dtype, int out_dtype, int r, int p, int K) {
  return (dtype == SMAT_BF16 || dtype == SMAT_F16) &&
         (out_dtype == SMAT_F32 || out_dtype == dtype) && r == cb::kR && p == cb::kP && K >= 1;
}

template <typename In, typename Out>
static void cell_read_launch(dim3 grid, hipStream_t st, const void* phr, const float* dY,
                             const float* F, const int32_t* ent, const int64_t* eoffs, void* dPhi,
                             float* dF, float* dw, int N0, int K, int L, int64_t q_sb, int64_t q_st,
                             int64_t y_sb, int64_t y_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
                             int64_t w_sb) {
  hipLaunchKernelGGL((cell_read_bwd_kernel<In, Out>), grid, dim3(cw::kThreads), 0, st,
                     (const In*)phr, dY, F, ent, eoffs, (Out*)dPhi, dF, dw, N0, K, L, q_sb, q_st,
                     y_sb, y_st, f_sb, d_sb, d_st, w_sb);
}

template <typename In, typename Out>
static void cell_pool_launch(dim3 grid, hipStream_t st, const void* psi, const void* vb,
                             const float* dF, const int32_t* ent, const int64_t* eoffs, void* dPsi,
                             void* dVb, float* dw, int N0, int K, int L, int64_t k_sb, int64_t k_st,
                             int64_t v_sb, int64_t v_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
                             int64_t e_sb, int64_t e_st, int64_t w_sb) {
  hipLaunchKernelGGL((cell_pool_bwd_kernel<In, Out>), grid, dim3(cw::kThreads), 0, st,
                     (const In*)psi, (const In*)vb, dF, ent, eoffs, (Out*)dPsi, (Out*)dVb, dw, N0,
                     K, L, k_sb, k_st, v_sb, v_st, f_sb, d_sb, d_st, e_sb, e_st, w_sb);
}

}  // namespace smat

extern "C" int smat_cell_read_backward(int dtype, int out_dtype, const void* phr,
                                       const float* dY, const float* F, const int32_t* ent,
                                       const int64_t* eoffs, void* dPhi, float* dF, float* dw,
                                       int nb, int N0, int K, int L,
                                       int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb,
                                       int64_t y_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
                                       int64_t w_sb, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phr && dY && F && ent && eoffs && dPhi && dF && dw, SMAT_EINVAL,
               "smat_cell_read_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && L >= 1 && (int64_t)K * L < (1ll << 31), SMAT_EINVAL,
               "smat_cell_read_backward: bad sizes");
  SMAT_REQUIRE(cw_ok(dtype, out_dtype, r, p, K), SMAT_EUNSUPPORTED,
               "smat_cell_read_backward: needs dtype bf16/f16, out_dtype fp32 or dtype, r=64, "
               "p=65 (got %d, %d, %d, %d)",
               dtype, out_dtype, r, p);
  SMAT_REQUIRE(rows_vec_ok(phr, q_sb, q_st, 2) &&
                   rows_vec_ok(dPhi, d_sb, d_st, elem_bytes(out_dtype)) &&
                   aligned16(F) && f_sb % 4 == 0 && y_st >= p && f_sb >= (int64_t)N0 * r * p,
               SMAT_EINVAL, "smat_cell_read_backward: Phi, dPhi and F must be 16-byte aligned");
  SMAT_REQUIRE(N0 < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_cell_read_backward: grid too large");
  if (nb == 0) return SMAT_OK;
  const dim3 grid((unsigned)N0, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  const bool f32 = out_dtype == SMAT_F32;
  if (dtype == SMAT_BF16)
    (f32 ? cell_read_launch<bf16, float> : cell_read_launch<bf16, bf16>)(
        grid, st, phr, dY, F, ent, eoffs, dPhi, dF, dw, N0, K, L, q_sb, q_st, y_sb, y_st, f_sb,
        d_sb, d_st, w_sb);
  else
    (f32 ? cell_read_launch<f16, float> : cell_read_launch<f16, f16>)(
        grid, st, phr, dY, F, ent, eoffs, dPhi, dF, dw, N0, K, L, q_sb, q_st, y_sb, y_st, f_sb,
        d_sb, d_st, w_sb);
  return launch_status("smat_cell_read_backward");
}

extern "C" int smat_cell_pool_backward(int dtype, int out_dtype, const void* psi,
                                       const void* vb, const float* dF, const int32_t* ent,
                                       const int64_t* eoffs, void* dPsi, void* dVb, float* dw,
                                       int nb, int N0, int K, int L,
                                       int r, int p, int64_t k_sb, int64_t k_st, int64_t v_sb,
                                       int64_t v_st, int64_t f_sb, int64_t d_sb, int64_t d_st,
                                       int64_t e_sb, int64_t e_st, int64_t w_sb, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && dF && ent && eoffs && dPsi && dVb && dw, SMAT_EINVAL,
               "smat_cell_pool_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && L >= 1 && (int64_t)K * L < (1ll << 31), SMAT_EINVAL,
               "smat_cell_pool_backward: bad sizes");
  SMAT_REQUIRE(cw_ok(dtype, out_dtype, r, p, K), SMAT_EUNSUPPORTED,
               "smat_cell_pool_backward: needs dtype bf16/f16, out_dtype fp32 or dtype, r=64, "
               "p=65 (got %d, %d, %d, %d)",
               dtype, out_dtype, r, p);
  SMAT_REQUIRE(rows_vec_ok(dPsi, d_sb, d_st, elem_bytes(out_dtype)) && aligned16(dF) &&
                   f_sb % 4 == 0 &&
                   k_st >= r && v_st >= p && e_st >= p && f_sb >= (int64_t)N0 * r * p,
               SMAT_EINVAL, "smat_cell_pool_backward: dPsi and dF must be 16-byte aligned");
  SMAT_REQUIRE(N0 < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_cell_pool_backward: grid too large");
  if (nb == 0) return SMAT_OK;
  const dim3 grid((unsigned)N0, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  const bool f32 = out_dtype == SMAT_F32;
  if (dtype == SMAT_BF16)
    (f32 ? cell_pool_launch<bf16, float> : cell_pool_launch<bf16, bf16>)(
        grid, st, psi, vb, dF, ent, eoffs, dPsi, dVb, dw, N0, K, L, k_sb, k_st, v_sb, v_st, f_sb,
        d_sb, d_st, e_sb, e_st, w_sb);
  else
    (f32 ? cell_pool_launch<f16, float> : cell_pool_launch<f16, f16>)(
        grid, st, psi, vb, dF, ent, eoffs, dPsi, dVb, dw, N0, K, L, k_sb, k_st, v_sb, v_st, f_sb,
        d_sb, d_st, e_sb, e_st, w_sb);
  return launch_status("smat_cell_pool_backward");
}
