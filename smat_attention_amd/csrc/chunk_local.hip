// Fused within-chunk pass of the causal scan:
//   out_b = Phi_b Sin_b + (tril(Phi_b Psi_b^T)) Vb_b        for every chunk b.
//
// Follows the semantics of src/smat/kernels/triton_fwd.py:48-115 (and the
// torch branch of src/smat/attention.py:187-190): the score tile is
// accumulated in fp32 from the input dtype, masked causally, rounded to the
// input dtype and multiplied with Vb in fp32; the inter-chunk term uses the
// fp32 state.  The design is this library's own:
//
//   * one workgroup (4 waves) owns 128 rows of a chunk; wave w owns the 16-row
//     tiles w and 7-w, which balances the causal triangle across waves;
//   * the wave's Phi rows live in registers for the whole kernel and serve as
//     the A operand of Phi Sin and the B operand of S^T = Psi Phi^T;
//   * S^T is computed instead of S so that its fp32 accumulator tiles, masked
//     and rounded, ARE the A fragments of the following S Vb product (the
//     16x16 C layout lines up with the A layout of the next MFMA, no LDS trip);
//   * Sin is staged once in LDS, transposed and split into hi/lo 16-bit parts
//     for 16-bit inputs (two MFMAs keep ~16 mantissa bits of the fp32 state);
//     fp32 inputs use fp32 MFMA throughout;
//   * Psi and Vb are staged in 64-token blocks, only up to the diagonal.
//
// With Decay (the decayed scan, src/smat/model.py:41-82) every row m of the
// chunk also carries L_m, the running sum of the log-decays within its chunk:
// the inter-chunk term of row m is scaled by exp(L_m) and the score of (m, n),
// n <= m, by exp(L_m - L_n) after the causal mask -- the masked weights are
// never formed, so no exp of a positive difference is taken.
#include "smat_host.hpp"

namespace smat {

namespace cl {
constexpr int kThreads = 256;
constexpr int kBM = 128;                 // rows per workgroup
constexpr int kBN = 64;                  // tokens per staged block
constexpr int kRK = 4;                   // r <= 128, k-blocks of 32
constexpr int kNCT = 9;                  // p <= 144, column tiles of 16
constexpr int kRPad = kRK * 32 + 8;      // LDS row length for r-indexed rows
constexpr int kNPad = kBN + 8;           // LDS row length of Vb^T
constexpr int kCols = kNCT * 16;

template <typename In>
constexpr int sin_bytes() {
  return Traits<In>::split ? 2 * kCols * kRPad * (int)sizeof(In) : kCols * kRPad * 4;
}
template <typename In>
constexpr int blk_bytes() {
  return (kBN * kRPad + kCols * kNPad) * (int)sizeof(In);
}
template <typename In>
constexpr int smem_bytes() {
  return sin_bytes<In>() > blk_bytes<In>() ? sin_bytes<In>() : blk_bytes<In>();
}
}  // namespace cl

template <typename In, bool Decay>
__global__ __launch_bounds__(cl::kThreads, 2) void chunk_local_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ sin, const float* __restrict__ L, float* __restrict__ out, int C,
    int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
    int64_t v_st, int64_t s_sb, int64_t s_sr, int64_t o_sb, int64_t o_st, int vec_q, int vec_k) {
  using namespace cl;
  typedef typename Traits<In>::frag Frag;
  __shared__ __attribute__((aligned(16))) char smem[smem_bytes<In>()];

  const int64_t b = blockIdx.x;
  const int mb = blockIdx.y;
  const int lane = lane_id(), w = wave_id();
  const int row16 = lane & 15, grp = lane >> 4;
  const int rk = (r + 31) >> 5;
  const int nct = (p + 15) >> 4;

  const In* phib = phi + b * q_sb;
  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;

  int mrow0[2];
  mrow0[0] = mb * kBM + 16 * w;
  mrow0[1] = mb * kBM + 16 * (7 - w);

  // ---- this wave's Phi rows, as fragments (row = m, 8 consecutive k) ----
  Frag phiA[2][kRK];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int m = mrow0[t] + row16;
#pragma unroll
    for (int kb = 0; kb < kRK; ++kb) {
      const int k0 = 32 * kb + 8 * grp;
      const int nv = (kb < rk && m < C) ? min(8, r - k0) : 0;
      phiA[t][kb] = load8<In>(phib + (int64_t)m * q_st + k0, nv, vec_q);
    }
  }

  f32x4 acc[2][kNCT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) acc[t][ct] = zero4();

  // ---- inter-chunk term: Phi Sin -----------------------------------------
  {
    const float* sinb = sin + b * s_sb;
    const int ncols = nct * 16, nrows = rk * 32;
    if constexpr (Traits<In>::split) {
      In* hi = reinterpret_cast<In*>(smem);
      In* lo = hi + kCols * kRPad;
      for (int idx = threadIdx.x; idx < nrows * ncols; idx += kThreads) {
        const int a = idx / ncols, c = idx - a * ncols;
        const float v = (a < r && c < p) ? sinb[(int64_t)a * s_sr + c] : 0.f;
        In h, l;
        split2<In>(v, h, l);
        hi[c * kRPad + a] = h;
        lo[c * kRPad + a] = l;
      }
      __syncthreads();
#pragma unroll
      for (int kb = 0; kb < kRK; ++kb) {
        if (kb >= rk) continue;
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
          if (ct >= nct) continue;
          const int off = (ct * 16 + row16) * kRPad + 32 * kb + 8 * grp;
          const Frag bh = *reinterpret_cast<const Frag*>(hi + off);
          const Frag bl = *reinterpret_cast<const Frag*>(lo + off);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bh);
            acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bl);
          }
        }
      }
    } else {
      float* st = reinterpret_cast<float*>(smem);
      for (int idx = threadIdx.x; idx < nrows * ncols; idx += kThreads) {
        const int a = idx / ncols, c = idx - a * ncols;
        st[c * kRPad + a] = (a < r && c < p) ? sinb[(int64_t)a * s_sr + c] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int kb = 0; kb < kRK; ++kb) {
        if (kb >= rk) continue;
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
          if (ct >= nct) continue;
          const int off = (ct * 16 + row16) * kRPad + 32 * kb + 8 * grp;
          const Frag bf = *reinterpret_cast<const Frag*>(st + off);
#pragma unroll
          for (int t = 0; t < 2; ++t) acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bf);
        }
      }
    }
    __syncthreads();
  }

  const float* Lb = Decay ? L + b * (int64_t)C : nullptr;
  if constexpr (Decay) {
    // row m of the inter-chunk term: exp(L_m) Phi_m Sin
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mrow0[t] + 4 * grp + i;
        const float e = m < C ? expf(Lb[m]) : 0.f;
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) acc[t][ct][i] *= e;
      }
  }

  // ---- within-chunk term: tril(Phi Psi^T) Vb -----------------------------
  In* psiS = reinterpret_cast<In*>(smem);            // [kBN][kRPad]
  In* vbT = psiS + kBN * kRPad;                      // [kCols][kNPad]
  const int m_end = min(C, mb * kBM + kBM);
  const int kgroups = rk * 4;                        // 8-element groups per row
  const int ncols = nct * 16;
  for (int n0 = 0; n0 < m_end; n0 += kBN) {
    // stage Psi rows [n0, n0+64) x [0, rk*32)
    for (int idx = threadIdx.x; idx < kBN * kgroups; idx += kThreads) {
      const int nn = idx / kgroups, g8 = idx - nn * kgroups;
      const int n = n0 + nn;
      const int nv = (n < C) ? min(8, r - 8 * g8) : 0;
      *reinterpret_cast<Frag*>(psiS + nn * kRPad + 8 * g8) =
          load8<In>(psib + (int64_t)n * k_st + 8 * g8, nv, vec_k);
    }
    // stage Vb^T: [c][nn]
    for (int idx = threadIdx.x; idx < kBN * ncols; idx += kThreads) {
      const int nn = idx / ncols, c = idx - nn * ncols;
      const int n = n0 + nn;
      vbT[c * kNPad + nn] = (n < C && c < p) ? vbb[(int64_t)n * v_st + c] : from_f32<In>(0.f);
    }
    __syncthreads();

#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int mr0 = mrow0[t];
#pragma unroll
      for (int np = 0; np < 2; ++np) {
        const int nb0 = n0 + 32 * np;
        if (nb0 > mr0 + 15 || nb0 >= C) continue;   // pair above the diagonal
        f32x4 s[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          s[nt] = zero4();
          const int nt0 = nb0 + 16 * nt;
          if (nt0 <= mr0 + 15 && nt0 < C) {
#pragma unroll
            for (int kb = 0; kb < kRK; ++kb) {
              if (kb >= rk) continue;
              const Frag a = *reinterpret_cast<const Frag*>(
                  psiS + (32 * np + 16 * nt + row16) * kRPad + 32 * kb + 8 * grp);
              s[nt] = mma(s[nt], a, phiA[t][kb]);
            }
          }
          // lane holds S^T[n = nt0 + 4 grp + i][m = mr0 + row16]
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (nt0 + 4 * grp + i > mr0 + row16) s[nt][i] = 0.f;
          if constexpr (Decay) {
            const int m = mr0 + row16;
            const float Lm = m < C ? Lb[m] : 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int n = nt0 + 4 * grp + i;
              if (n <= m && n < C) s[nt][i] *= expf(Lm - Lb[n]);
            }
          }
        }
        // A fragment of S: element j < 4 is n = nb0 + 4 grp + j, j >= 4 is
        // n = nb0 + 16 + 4 grp + (j - 4).
        Frag sa;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sa[j] = from_f32<In>(s[0][j]);
          sa[j + 4] = from_f32<In>(s[1][j]);
        }
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
          if (ct >= nct) continue;
          const In* vr = vbT + (ct * 16 + row16) * kNPad + 32 * np + 4 * grp;
          Frag vf;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            vf[j] = vr[j];
            vf[j + 4] = vr[16 + j];
          }
          acc[t][ct] = mma(acc[t][ct], sa, vf);
        }
      }
    }
    __syncthreads();
  }

  // ---- store ---------------------------------------------------------------
  float* outb = out + b * o_sb;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
      if (ct >= nct) continue;
      const int c = ct * 16 + row16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mrow0[t] + 4 * grp + i;
        if (m < C && c < p) outb[(int64_t)m * o_st + c] = acc[t][ct][i];
      }
    }
  }
}

template <typename In>
static int launch_chunk_local(const void* phi, const void* psi, const void* vb, const float* sin,
                              const float* L, float* out, int64_t nbc, int C, int r, int p,
                              int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                              int64_t v_sb, int64_t v_st, int64_t s_sb, int64_t s_sr,
                              int64_t o_sb, int64_t o_st, hipStream_t stream) {
  const int eb = sizeof(In);
  const int vq = rows_vec_ok(phi, q_sb, q_st, eb);
  const int vk = rows_vec_ok(psi, k_sb, k_st, eb);
  dim3 grid((unsigned)nbc, (unsigned)((C + cl::kBM - 1) / cl::kBM));
  auto kern = L ? chunk_local_kernel<In, true> : chunk_local_kernel<In, false>;
  smat::launch(kern, grid, dim3(cl::kThreads), 0, stream, (const In*)phi, (const In*)psi,
                     (const In*)vb, sin, L, out, C, r, p, q_sb, q_st, k_sb, k_st, v_sb, v_st, s_sb,
                     s_sr, o_sb, o_st, vq, vk);
  return launch_status(L ? "smat_chunk_local_decay" : "smat_chunk_local");
}

int chunk_local_dispatch(int dtype, const void* phi, const void* psi, const void* vb,
                         const float* sin, float* out, int64_t nbc, int C, int r, int p,
                         int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                         int64_t v_st, int64_t s_sb, int64_t s_sr, int64_t o_sb, int64_t o_st,
                         hipStream_t stream, const float* L) {
  switch (dtype) {
    case SMAT_BF16:
      return launch_chunk_local<bf16>(phi, psi, vb, sin, L, out, nbc, C, r, p, q_sb, q_st, k_sb,
                                      k_st, v_sb, v_st, s_sb, s_sr, o_sb, o_st, stream);
    case SMAT_F16:
      return launch_chunk_local<f16>(phi, psi, vb, sin, L, out, nbc, C, r, p, q_sb, q_st, k_sb,
                                     k_st, v_sb, v_st, s_sb, s_sr, o_sb, o_st, stream);
    case SMAT_F32:
      return launch_chunk_local<float>(phi, psi, vb, sin, L, out, nbc, C, r, p, q_sb, q_st, k_sb,
                                       k_st, v_sb, v_st, s_sb, s_sr, o_sb, o_st, stream);
  }
  set_error("smat_chunk_local: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}

}  // namespace smat

extern "C" int smat_chunk_local(int dtype, const void* phi, const void* psi, const void* vb,
                                const float* sin, float* out, int64_t nbc, int C, int r, int p,
                                int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                                int64_t v_sb, int64_t v_st, int64_t s_sb, int64_t s_sr,
                                int64_t o_sb, int64_t o_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && sin && out, SMAT_EINVAL, "smat_chunk_local: null pointer");
  SMAT_REQUIRE(nbc >= 0 && nbc < (1ll << 31), SMAT_EINVAL, "smat_chunk_local: nbc=%lld",
               (long long)nbc);
  SMAT_REQUIRE(C >= 1 && C <= kMaxC, SMAT_EUNSUPPORTED, "smat_chunk_local: C=%d not in [1, %d]",
               C, kMaxC);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR, SMAT_EUNSUPPORTED, "smat_chunk_local: r=%d not in [1, %d]",
               r, kMaxR);
  SMAT_REQUIRE(p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED, "smat_chunk_local: p=%d not in [1, %d]",
               p, kMaxP);
  SMAT_REQUIRE(q_st >= r && k_st >= r && v_st >= p && s_sr >= p && o_st >= p, SMAT_EINVAL,
               "smat_chunk_local: a row stride is shorter than its row");
  if (nbc == 0) return SMAT_OK;
  return chunk_local_dispatch(dtype, phi, psi, vb, sin, out, nbc, C, r, p, q_sb, q_st, k_sb, k_st,
                              v_sb, v_st, s_sb, s_sr, o_sb, o_st, (hipStream_t)stream, nullptr);
}

extern "C" int smat_chunk_local_decay(int dtype, const void* phi, const void* psi, const void* vb,
                                      const float* sin, const float* L, float* out, int64_t nbc,
                                      int C, int r, int p, int64_t q_sb, int64_t q_st,
                                      int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                                      int64_t s_sb, int64_t s_sr, int64_t o_sb, int64_t o_st,
                                      void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && sin && L && out, SMAT_EINVAL,
               "smat_chunk_local_decay: null pointer");
  SMAT_REQUIRE(nbc >= 0 && nbc < (1ll << 31), SMAT_EINVAL, "smat_chunk_local_decay: nbc=%lld",
               (long long)nbc);
  SMAT_REQUIRE(C >= 1 && C <= kMaxC, SMAT_EUNSUPPORTED,
               "smat_chunk_local_decay: C=%d not in [1, %d]", C, kMaxC);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_chunk_local_decay: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && k_st >= r && v_st >= p && s_sr >= p && o_st >= p, SMAT_EINVAL,
               "smat_chunk_local_decay: a row stride is shorter than its row");
  if (nbc == 0) return SMAT_OK;
  return chunk_local_dispatch(dtype, phi, psi, vb, sin, out, nbc, C, r, p, q_sb, q_st, k_sb, k_st,
                              v_sb, v_st, s_sb, s_sr, o_sb, o_st, (hipStream_t)stream, L);
}
