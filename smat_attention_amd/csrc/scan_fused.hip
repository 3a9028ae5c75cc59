// The causal pass of the schedule fused end to end: the segmented chunked
// scan of src/smat/attention.py:134-192 (one reset at n), the long-range term
// added to recent rows and the normalisation of :446-453, in one kernel that
// reads Phi, Psi, Vb (and Y) once and writes the output once.
//
// Chunks are grouped K at a time inside a segment.  A prepass (the Gram
// kernel over each group's tokens, then the shifted exclusive scan over
// groups) gives every group its incoming state; one workgroup then walks the
// group's chunks in order with the r x p state S held in fp32 MFMA
// accumulators:
//
//   for each chunk:  out = Phi S + tril(Phi Psi^T) Vb      (as chunk_local)
//                    S  += Psi^T Vb                        (as the Gram kernel)
//                    normalise out (+ Y on recent rows, x g) and store
//
// The in-chunk products reuse chunk_local's layout (wave w owns 16-row tiles
// w and 7-w; S^T = Psi Phi^T feeds the S Vb product straight from the
// accumulators).  The state update reuses the Gram kernel's (wave w owns rows
// 32w..32w+31 of S).  After each chunk the waves write S^T to LDS, split into
// hi/lo 16-bit parts for 16-bit inputs, as the B operand of the next chunk's
// Phi S.  Psi and Vb are staged once per 64-token block and feed both the
// intra-chunk product and the update.
#include <mutex>

#include "feat_map.hpp"
#include "smat_host.hpp"

namespace smat {

namespace sf {
constexpr int kThreads = 256;
constexpr int kC = 128;                  // rows per chunk handled (chunk <= 128)

// Tile shape: RK k-blocks of 32 features (r <= 32 RK) and NCT column tiles of
// 16 (p <= 16 NCT).  The wide shape (4, 9) covers r <= 128, p <= 144; the
// narrow one (2, 5) covers r <= 64, p <= 80 with half the registers and under
// half the LDS, so two workgroups share a CU.
template <int RK> constexpr int rpad() { return RK * 32 + 8; }   // r-indexed LDS rows

// tokens per staged block: 64 for 16-bit inputs, 32 for fp32 (LDS budget)
template <typename In> constexpr int bn() { return sizeof(In) == 4 ? 32 : 64; }
template <typename In> constexpr int npad() { return bn<In>() + 8; }

template <typename In, int RK, int NCT>
constexpr int state_bytes() {
  return Traits<In>::split ? 2 * NCT * 16 * rpad<RK>() * (int)sizeof(In)
                           : NCT * 16 * rpad<RK>() * 4;
}
template <typename In, int RK, int NCT>
constexpr int block_bytes() {
  // psiS [bn][rpad], psiT [32 RK][npad], vbT [16 NCT][npad]
  return (bn<In>() * rpad<RK>() + RK * 32 * npad<In>() + NCT * 16 * npad<In>()) *
         (int)sizeof(In);
}
}  // namespace sf

template <typename In, bool VEC, int kRK, int kNCT>
__global__ __launch_bounds__(sf::kThreads, kRK <= 2 ? 2 : 1) void scan_fused_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ Sg, const float* __restrict__ Y, const float* __restrict__ gate,
    float* __restrict__ out, ScanArgs a) {
  using namespace sf;
  typedef typename Traits<In>::frag Frag;
  constexpr int kBN = bn<In>();
  constexpr int kNPad = npad<In>();
  constexpr int kRPad = rpad<kRK>();
  constexpr int kCols = kNCT * 16;
  constexpr int kTW = kRK / 2;          // 16-row tiles of S per wave: wave w owns tiles kTW w + t
  static_assert(kRK % 2 == 0, "four waves split 2 kRK row tiles of S");
  __shared__ __attribute__((aligned(16))) char smem[state_bytes<In, kRK, kNCT>() +
                                                    block_bytes<In, kRK, kNCT>()];
  In* sT_hi = reinterpret_cast<In*>(smem);                 // S^T [c][a] (hi, or fp32 whole)
  In* sT_lo = sT_hi + kCols * kRPad;
  float* sT32 = reinterpret_cast<float*>(smem);
  In* psiS = reinterpret_cast<In*>(smem + state_bytes<In, kRK, kNCT>());   // [kBN][kRPad]
  In* psiT = psiS + kBN * kRPad;                                 // [32 kRK][kNPad]
  In* vbT = psiT + kRK * 32 * kNPad;                             // [kCols][kNPad]

  const int grp = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = lane_id(), w = wave_id();
  const int row16 = lane & 15, g4 = lane >> 4;
  const int r = a.r, p = a.p, C = a.C;
  const int rk = (r + 31) >> 5;
  const int nct = (p + 15) >> 4;
  const int nrt = (r + 15) >> 4;

  // chunks of this group
  int c0, c1;
  if (grp < a.ng0) {
    c0 = grp * a.K;
    c1 = min(c0 + a.K, a.nc0);
  } else {
    c0 = a.nc0 + (grp - a.ng0) * a.K;
    c1 = min(c0 + a.K, a.nc);
  }

  const In* phib = phi + b * a.q_sb;
  const In* psib = psi + b * a.k_sb;
  const In* vbb = vb + b * a.v_sb;

  // ---- staging of one token block: 8 x 8 tiles of Psi (to psiS and psiT)
  // and of Vb (to vbT); a thread owns tiles tid and tid + kThreads ----
  const int kgroups = rk * 4;
  const int ncols = nct * 16;
  const int tpsi = (kBN / 8) * kgroups;
  const int ttot = tpsi + (kBN / 8) * (ncols / 8);
  // tiles per thread: the most the shape can stage, (kBN/8)(4 kRK + 2 kNCT)
  constexpr int kTiles = ((kBN / 8) * (4 * kRK + 2 * kNCT) + kThreads - 1) / kThreads;
  struct Pf {
    Tile8<In> tl[kTiles];
    int tt[kTiles], c0[kTiles];
    bool psi[kTiles], live[kTiles];
  } pf;
  auto stage_issue = [&](Pf& f, int chk, int nb0) {
    const int64_t tk0 = (int64_t)chk * C;
    const int cv = (int)min((int64_t)C, (int64_t)a.T - tk0);
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const int tile = threadIdx.x + j * kThreads;
      f.live[j] = tile < ttot;
      if (!f.live[j]) continue;
      const bool is_psi = tile < tpsi;
      const int tix = is_psi ? tile : tile - tpsi;
      const int per_row = is_psi ? kgroups : ncols / 8;
      f.psi[j] = is_psi;
      f.tt[j] = (tix / per_row) * 8;
      f.c0[j] = (tix % per_row) * 8;
      const In* rowp[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int nr = nb0 + f.tt[j] + u;
        rowp[u] = nr < cv ? (is_psi ? psib + (tk0 + nr) * a.k_st : vbb + (tk0 + nr) * a.v_st)
                          : nullptr;
      }
      if constexpr (VEC) {
        if (is_psi)
          tile8_issue<In>(f.tl[j], rowp, psib + tk0 * a.k_st, f.c0[j], r);
        else
          tile8_issue<In>(f.tl[j], rowp, vbb + tk0 * a.v_st, f.c0[j], p);
      } else {
        if (is_psi)
          tile8_load<In, false>(f.tl[j], rowp, psib + tk0 * a.k_st, f.c0[j], r);
        else
          tile8_load<In, false>(f.tl[j], rowp, vbb + tk0 * a.v_st, f.c0[j], p);
      }
    }
  };
  auto stage_commit = [&](Pf& f, In* dS, In* dT, In* dV) {
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      if (!f.live[j]) continue;
      if constexpr (VEC) tile8_finish<In>(f.tl[j]);
      if (f.psi[j]) {
        tile8_store<In>(f.tl[j], dS, kRPad, f.c0[j], f.tt[j]);
        tile8_store_T<In>(f.tl[j], dT, kNPad, f.c0[j], f.tt[j]);
      } else {
        tile8_store_T<In>(f.tl[j], dV, kNPad, f.c0[j], f.tt[j]);
      }
    }
  };
  if (c0 < c1) stage_issue(pf, c0, 0);

  // ---- incoming state: this wave's rows of S in accumulators, S^T in LDS ----
  f32x4 accS[kTW][kNCT];
  {
    const float* Sb = Sg + ((int64_t)b * gridDim.x + grp) * (int64_t)r * p;
#pragma unroll
    for (int t = 0; t < kTW; ++t) {
      const int rt = kTW * w + t;
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) {
        const int c = ct * 16 + row16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ar = rt * 16 + 4 * g4 + i;
          const bool ok = ar < r && c < p;            // (rt < nrt, ct < nct follow)
          const float v = Sb[ok ? (int64_t)ar * p + c : 0];   // branch-free
          accS[t][ct][i] = ok ? v : 0.f;
        }
      }
    }
  }

  int mrow[2];
  mrow[0] = 16 * w;
  mrow[1] = 16 * (7 - w);

  for (int ch = c0; ch < c1; ++ch) {
    const int64_t t0 = (int64_t)ch * C;                  // first token of the chunk
    const int Cv = (int)min((int64_t)C, (int64_t)a.T - t0);   // valid rows (ragged tail)

    // ---- publish S^T (state before this chunk) ----
    // lane (g4, row16) holds S[rt*16 + 4*g4 + i][ct*16 + row16], i = 0..3:
    // four consecutive rows of one column, one 8-byte (fp32: 16-byte) store.
    lds_barrier();        // previous chunk's readers of sT are done
#pragma unroll
    for (int t = 0; t < kTW; ++t) {
      const int rt = kTW * w + t;
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) {
        const int off = (ct * 16 + row16) * kRPad + rt * 16 + 4 * g4;
        if constexpr (Traits<In>::split) {
          typename Traits<In>::half_frag h4, l4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            In h, l;
            split2<In>(accS[t][ct][i], h, l);
            h4[i] = h;
            l4[i] = l;
          }
          *reinterpret_cast<typename Traits<In>::half_frag*>(sT_hi + off) = h4;
          *reinterpret_cast<typename Traits<In>::half_frag*>(sT_lo + off) = l4;
        } else {
          *reinterpret_cast<f32x4*>(sT32 + off) = accS[t][ct];
        }
      }
    }

    // ---- this wave's Phi rows ----
    Frag phiA[2][kRK];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int m = mrow[t] + row16;
#pragma unroll
      for (int kb = 0; kb < kRK; ++kb) {
        const int k0 = 32 * kb + 8 * g4;
        const int nv = (kb < rk && m < Cv) ? min(8, r - k0) : 0;
        phiA[t][kb] = load8v<In, VEC>(phib + (t0 + m) * a.q_st + k0, phib + t0 * a.q_st, nv);
      }
    }
    // ---- this chunk's long-range rows (recent rows only), branch-free from a
    // clamped address.  The wide shape loads them now so the latency overlaps
    // the products; the narrow one, two workgroups to a CU, loads them just
    // before they are added and keeps the registers for the products ----
    float yv[2][kNCT][4];
    auto load_y = [&]() {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mrow[t] + 4 * g4 + i;
          const int64_t row = t0 + m;
          const bool rec = m < Cv && !a.write_H && Y != nullptr && row >= a.n;
          const float* yrow = rec ? Y + b * a.y_sb + (row - a.n) * a.y_st : Y;
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) {
            const int c = ct * 16 + row16;
            const bool ok = rec && c < p;
            const float v = (Y != nullptr) ? yrow[ok ? c : 0] : 0.f;
            yv[t][ct][i] = ok ? v : 0.f;
          }
        }
      }
    };
    if constexpr (kRK > 2) load_y();
    lds_barrier();        // sT complete

    // ---- inter-chunk term: Phi S ----
    f32x4 acc[2][kNCT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) acc[t][ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < kRK; ++kb) {
      if (kb >= rk) continue;
#pragma unroll
      for (int ct = 0; ct < kNCT; ++ct) {
        if (ct >= nct) continue;
        const int off = (ct * 16 + row16) * kRPad + 32 * kb + 8 * g4;
        if constexpr (Traits<In>::split) {
          const Frag bh = *reinterpret_cast<const Frag*>(sT_hi + off);
          const Frag bl = *reinterpret_cast<const Frag*>(sT_lo + off);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bh);
            acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bl);
          }
        } else {
          const Frag bf = *reinterpret_cast<const Frag*>(sT32 + off);
#pragma unroll
          for (int t = 0; t < 2; ++t) acc[t][ct] = mma(acc[t][ct], phiA[t][kb], bf);
        }
      }
    }

    // ---- token blocks: intra-chunk product and the state update ----
    for (int n0 = 0; n0 < Cv; n0 += kBN) {
      lds_barrier();      // previous block's readers are done
      stage_commit(pf, psiS, psiT, vbT);
      lds_barrier();
      // the next block's loads fly while this block is multiplied
      {
        int nch = ch, nn0 = n0 + kBN;
        if (nn0 >= Cv) {
          nch = ch + 1;
          nn0 = 0;
        }
        if (nch < c1) stage_issue(pf, nch, nn0);
      }

      // intra-chunk: rows of this wave against tokens [n0, n0+64)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int mr0 = mrow[t];
#pragma unroll
        for (int np = 0; np < kBN / 32; ++np) {
          const int nb0 = n0 + 32 * np;
          if (nb0 > mr0 + 15 || nb0 >= Cv) continue;
          f32x4 s[2];
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            s[nt] = zero4();
            const int nt0 = nb0 + 16 * nt;
            if (nt0 <= mr0 + 15 && nt0 < Cv) {
#pragma unroll
              for (int kb = 0; kb < kRK; ++kb) {
                if (kb >= rk) continue;
                const Frag av = *reinterpret_cast<const Frag*>(
                    psiS + (32 * np + 16 * nt + row16) * kRPad + 32 * kb + 8 * g4);
                s[nt] = mma(s[nt], av, phiA[t][kb]);
              }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (nt0 + 4 * g4 + i > mr0 + row16) s[nt][i] = 0.f;
          }
          Frag sa;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sa[j] = from_f32<In>(s[0][j]);
            sa[j + 4] = from_f32<In>(s[1][j]);
          }
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) {
            if (ct >= nct) continue;
            const In* vr = vbT + (ct * 16 + row16) * kNPad + 32 * np + 4 * g4;
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

      // state update: S += Psi_blk^T Vb_blk (this wave's rows of S)
#pragma unroll
      for (int kk = 0; kk < kBN / 32; ++kk) {
        if (n0 + 32 * kk >= Cv) continue;
#pragma unroll
        for (int t = 0; t < kTW; ++t) {
          const int rt = kTW * w + t;
          if (rt >= nrt) continue;
          const Frag av = *reinterpret_cast<const Frag*>(psiT + (rt * 16 + row16) * kNPad +
                                                         32 * kk + 8 * g4);
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) {
            if (ct >= nct) continue;
            const Frag bv = *reinterpret_cast<const Frag*>(vbT + (ct * 16 + row16) * kNPad +
                                                           32 * kk + 8 * g4);
            accS[t][ct] = mma(accS[t][ct], av, bv);
          }
        }
      }
    }

    // ---- normalise and store the chunk's rows ----
    if constexpr (kRK <= 2) load_y();
    const int pn = p - 1;                         // the normaliser column
    const int ctn = pn >> 4, ln = pn & 15;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float den[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // the normaliser of row m sits in lane (g4, ln) of column tile ctn
        float hn = 0.f;
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct)
          if (ct == ctn) hn = acc[t][ct][i] + yv[t][ct][i];
        den[i] = __shfl(hn, g4 * 16 + ln, 64);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mrow[t] + 4 * g4 + i;
        if (m >= Cv) continue;
        const int64_t row = t0 + m;
        float* orow = out + b * a.o_sb + row * a.o_st;
        if (a.write_H) {
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) {
            const int c = ct * 16 + row16;
            if (ct < nct && c < p) orow[c] = acc[t][ct][i];
          }
        } else {
          const float gv = gate ? gate[b * a.g_sb + row] : 1.f;
          const float inv = 1.f / den[i];        // one division per row
#pragma unroll
          for (int ct = 0; ct < kNCT; ++ct) {
            const int c = ct * 16 + row16;
            if (ct < nct && c < pn) {
              float v = (acc[t][ct][i] + yv[t][ct][i]) * inv;
              if (gate) v *= gv;
              orow[c] = v;
            }
          }
        }
      }
    }
  }
}

template <typename In, int RK, int NCT>
static int launch_scan_fused_shape(const void* phi, const void* psi, const void* vb,
                                   const float* Sg, const float* Y, const float* gate, float* out,
                                   int nb, int ng, const ScanArgs& a, hipStream_t stream) {
  const bool vec = rows_vec8_ok(phi, a.q_sb, a.q_st) && rows_vec8_ok(psi, a.k_sb, a.k_st) &&
                   rows_vec8_ok(vb, a.v_sb, a.v_st);
  dim3 grid((unsigned)ng, (unsigned)nb);
  if (vec)
    smat::launch((scan_fused_kernel<In, true, RK, NCT>), grid, dim3(sf::kThreads), 0,
                       stream, (const In*)phi, (const In*)psi, (const In*)vb, Sg, Y, gate, out, a);
  else
    smat::launch((scan_fused_kernel<In, false, RK, NCT>), grid, dim3(sf::kThreads), 0,
                       stream, (const In*)phi, (const In*)psi, (const In*)vb, Sg, Y, gate, out, a);
  return launch_status("smat_causal_scan");
}

template <typename In>
static int launch_scan_fused(const void* phi, const void* psi, const void* vb, const float* Sg,
                             const float* Y, const float* gate, float* out, int nb, int ng,
                             const ScanArgs& a, hipStream_t stream) {
  if (a.r <= 64 && a.p <= 80)
    return launch_scan_fused_shape<In, 2, 5>(phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
  return launch_scan_fused_shape<In, 4, 9>(phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
}

int chunk_states_dispatch(int dtype, const void* psi, const void* vb, float* D, int nb, int T,
                          int C, int K, int n, int r, int p, int64_t k_sb, int64_t k_st,
                          int64_t v_sb, int64_t v_st, float* partials, int64_t partial_bytes,
                          hipStream_t stream, int* ngroups_out, int* ng0_out);
int segment_scan_dispatch(const float* D, float* Sin, int nb, int nc, int nc0, int64_t rp,
                          hipStream_t stream);
bool scan_stream_ok(int dtype, const void* phi, const void* psi, const void* vb, const float* Y,
                    const float* out, const ScanArgs& a);
int scan_stream_launch(int dtype, const void* phi, const void* psi, const void* vb,
                       const float* Sg, const float* Y, const float* gate, float* out, int nb,
                       int ng, const ScanArgs& a, hipStream_t stream);
int scan_stream_launch_feat(int dtype, const void* q, const void* k, const void* v,
                            const float* Sg, const float* Y, const float* gate, float* out,
                            int nb, int ng, const ScanArgs& a, const FeatArgs& fa,
                            bool psi_formed, hipStream_t stream);
int gram_stream_launch_feat(int dtype, const void* k, const void* v, float* G, float* G_last,
                            const GramItems& it, int nitems, int nb, int64_t k_sb, int64_t k_st,
                            int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                            int64_t gl_sb, const FeatArgs& fa, hipStream_t stream,
                            const char* who);

// Group size: enough workgroups to fill the GPU (one per CU at a time), and
// no more than needed so the prepass stays small.
static int scan_group_chunks(int nb, int nc) {
  int K = 8;
  while (K > 1 && (int64_t)nb * ((nc + K - 1) / K) < 1024) K >>= 1;
  return K;
}

// F[b] = sum of the group sums G[b][g], g < ng0 (the tokens [0, n)).  A
// block takes 64 float4 columns of the r*p floats; its four waves sum every
// fourth group (each wave's loads independent of one another), then wave 0
// adds the other three partial sums in wave order.
__global__ __launch_bounds__(256) void group_sum_kernel(const float* __restrict__ G,
                                                        float* __restrict__ F, int ng0,
                                                        int64_t rp4, int64_t g_sb,
                                                        int64_t f_sb) {
  __shared__ float4 part[3][64];
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (e < rp4) {
    const float4* Gb = reinterpret_cast<const float4*>(G + b * g_sb) + e;
#pragma unroll 4
    for (int g = w; g < ng0; g += 4) {
      const float4 x = Gb[(int64_t)g * rp4];
      acc.x += x.x;
      acc.y += x.y;
      acc.z += x.z;
      acc.w += x.w;
    }
  }
  if (w > 0) part[w - 1][lane] = acc;
  __syncthreads();
  if (w == 0 && e < rp4) {
    for (int k = 0; k < 3; ++k) {
      const float4 x = part[k][lane];
      acc.x += x.x;
      acc.y += x.y;
      acc.z += x.z;
      acc.w += x.w;
    }
    reinterpret_cast<float4*>(F + b * f_sb)[e] = acc;
  }
}

int causal_scan_run(int dtype, const void* phi, const void* psi, const void* vb, const float* Y,
                    const float* gate, float* out, int nb, int T, int n, int C, int K, int r,
                    int p, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                    int64_t v_st, int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st,
                    int64_t g_sb, int write_H, void* ws, float* F_out, int64_t f_sb,
                    int phases, hipStream_t stream);

int64_t causal_scan_workspace_bytes(int nb, int T, int C, int r, int p) {
  const int nc = (T + C - 1) / C;
  const int K = scan_group_chunks(nb, nc);
  const int ng = (nc + K - 1) / K + 1;             // +1: the segment split may add a group
  return 2 * (((int64_t)nb * ng * r * p * 4 + 255) & ~(int64_t)255);
}

int causal_scan_dispatch(int dtype, const void* phi, const void* psi, const void* vb,
                         const float* Y, const float* gate, float* out, int nb, int T, int n,
                         int C, int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb,
                         int64_t k_st, int64_t v_sb, int64_t v_st, int64_t y_sb, int64_t y_st,
                         int64_t o_sb, int64_t o_st, int64_t g_sb, int write_H, void* ws,
                         int64_t ws_bytes, hipStream_t stream, float* F_out, int64_t f_sb,
                         int phases) {
  if (nb == 0 || T == 0) return SMAT_OK;
  const int nc = (T + C - 1) / C;
  const int K = scan_group_chunks(nb, nc);
  const int64_t need = causal_scan_workspace_bytes(nb, T, C, r, p);
  if (ws_bytes < need) {
    set_error("smat_causal_scan: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)ws_bytes);
    return SMAT_EINVAL;
  }
  return causal_scan_run(dtype, phi, psi, vb, Y, gate, out, nb, T, n, C, K, r, p, q_sb, q_st,
                         k_sb, k_st, v_sb, v_st, y_sb, y_st, o_sb, o_st, g_sb, write_H, ws,
                         F_out, f_sb, phases, stream);
}

// The causal pass with groups of K chunks; ws holds 2 * al256(nb * ng * r * p
// floats) bytes (ng = ceil(nc / K) + 1): the group summaries, then their scan.
int causal_scan_run(int dtype, const void* phi, const void* psi, const void* vb, const float* Y,
                    const float* gate, float* out, int nb, int T, int n, int C, int K, int r,
                    int p, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                    int64_t v_st, int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st,
                    int64_t g_sb, int write_H, void* ws, float* F_out, int64_t f_sb,
                    int phases, hipStream_t stream) {
  const int nc = (T + C - 1) / C;
  const int ng_max = (nc + K - 1) / K + 1;
  float* G = (float*)ws;
  float* Sg = (float*)((char*)ws + (((int64_t)nb * ng_max * r * p * 4 + 255) & ~(int64_t)255));
  // the group layout chunk_states_dispatch uses: groups of K chunks over
  // [0, n), then over [n, T)
  const int ng0 = (n / C + K - 1) / K;
  const int ng = ng0 + (nc - n / C + K - 1) / K;
  const int64_t rp = (int64_t)r * p;
  int rc = SMAT_OK;
  if (phases & 1) {
    int ng_d = 0, ng0_d = 0;
    rc = chunk_states_dispatch(dtype, psi, vb, G, nb, T, C, K, n, r, p, k_sb, k_st, v_sb, v_st,
                               nullptr, 0, stream, &ng_d, &ng0_d);
    if (rc) return rc;
    SMAT_REQUIRE(ng_d == ng && ng0_d == ng0, SMAT_EINVAL,
                 "smat_causal_scan: group layout %d/%d, expected %d/%d", ng_d, ng0_d, ng, ng0);
    if (F_out) {
      SMAT_REQUIRE(rp % 4 == 0 && f_sb % 4 == 0, SMAT_EINVAL,
                   "smat_forward: group sums need r*p and the row stride of F a multiple of 4");
      smat::launch(group_sum_kernel, dim3((unsigned)((rp / 4 + 63) / 64), (unsigned)nb),
                   dim3(256), 0, stream, (const float*)G, F_out, ng0, rp / 4, (int64_t)ng * rp,
                   f_sb);
      rc = launch_status("smat_forward");
      if (rc) return rc;
    }
  }
  if (!(phases & 2)) return SMAT_OK;
  rc = segment_scan_dispatch(G, Sg, nb, ng, ng0, (int64_t)r * p, stream);
  if (rc) return rc;
  ScanArgs a{};
  a.T = T;
  a.n = n;
  a.C = C;
  a.K = K;
  a.nc = nc;
  a.nc0 = n / C;
  a.ng0 = ng0;
  a.r = r;
  a.p = p;
  a.q_sb = q_sb;
  a.q_st = q_st;
  a.k_sb = k_sb;
  a.k_st = k_st;
  a.v_sb = v_sb;
  a.v_st = v_st;
  a.y_sb = y_sb;
  a.y_st = y_st;
  a.o_sb = o_sb;
  a.o_st = o_st;
  a.g_sb = g_sb;
  a.write_H = write_H;
  if (scan_stream_ok(dtype, phi, psi, vb, Y, out, a))
    return scan_stream_launch(dtype, phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
  switch (dtype) {
    case SMAT_BF16:
      return launch_scan_fused<bf16>(phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
    case SMAT_F16:
      return launch_scan_fused<f16>(phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
    case SMAT_F32:
      return launch_scan_fused<float>(phi, psi, vb, Sg, Y, gate, out, nb, ng, a, stream);
  }
  set_error("smat_causal_scan: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}

// The streaming causal pass with the feature map computed inside the kernels:
// q, k, v are the Q, K, V rows (r = d_qk = d_v = 128); the prepass Gram sums
// and the scan form Psi (and Phi) tiles in LDS from the DMA'd K (and Q) rows,
// and Vb = [V, 1] from V.  Same workspace as causal_scan_dispatch.  With
// psi_buf (nb x T rows of 128, 16-bit) the prepass also stores the Psi tiles
// it forms there and the scan reads them, forming only Phi.  phases: 1 the
// prepass (and, with F_out, F_out[b] = the sum over the tokens [0, n) of
// Psi^T Vb, from its group sums: one profile's pool), 2 the segment scan and
// the streaming scan, 3 both; a call of phase 2 follows one of phase 1 with
// the same workspace.
int causal_scan_run_feat(int dtype, const void* q, const void* k, const void* v, const float* Y,
                         const float* gate, float* out, int nb, int T, int n, int C,
                         int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                         int64_t v_st, int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st,
                         int64_t g_sb, const FeatArgs& fa, void* ws, int64_t ws_bytes,
                         void* psi_buf, float* F_out, int64_t f_sb, int phases,
                         hipStream_t stream) {
  if (nb == 0 || T == 0) return SMAT_OK;
  constexpr int r = 128, p = 129;
  const int64_t rp = (int64_t)r * p;
  const int nc = (T + C - 1) / C;
  const int K = scan_group_chunks(nb, nc);
  const int64_t need = causal_scan_workspace_bytes(nb, T, C, r, p);
  if (ws_bytes < need) {
    set_error("smat_forward_fused: causal-pass workspace of %lld bytes needed, %lld given",
              (long long)need, (long long)ws_bytes);
    return SMAT_EINVAL;
  }
  const int ng_max = (nc + K - 1) / K + 1;
  float* G = (float*)ws;
  float* Sg = (float*)((char*)ws + (((int64_t)nb * ng_max * rp * 4 + 255) & ~(int64_t)255));
  GramItems it{};
  it.mode = 0;
  it.T = T;
  it.C = C;
  it.K = K;
  it.nc = nc;
  it.nc0 = n / C;
  it.ng0 = (it.nc0 + K - 1) / K;
  it.nsplit = 1;
  it.per = K * C;
  const int ng = it.ng0 + (nc - it.nc0 + K - 1) / K;
  FeatArgs fp = fa;
  fp.psi_out = psi_buf;
  fp.psi_sb = (int64_t)T * 128;
  int rc = SMAT_OK;
  if (phases & 1) {
    rc = gram_stream_launch_feat(dtype, k, v, G, nullptr, it, ng, nb, k_sb, k_st, v_sb, v_st,
                                 (int64_t)ng * rp, rp, 0, fp, stream, "smat_forward_fused");
    if (rc) return rc;
    if (F_out) {
      const int64_t rp4 = rp / 4;
      smat::launch(group_sum_kernel, dim3((unsigned)((rp4 + 63) / 64), (unsigned)nb),
                   dim3(256), 0, stream, (const float*)G, F_out, it.ng0, rp4,
                   (int64_t)ng * rp, f_sb);
      rc = launch_status("smat_forward_fused");
      if (rc) return rc;
    }
  }
  if (!(phases & 2)) return SMAT_OK;
  rc = segment_scan_dispatch(G, Sg, nb, ng, it.ng0, rp, stream);
  if (rc) return rc;
  ScanArgs a{};
  a.T = T;
  a.n = n;
  a.C = C;
  a.K = K;
  a.nc = nc;
  a.nc0 = n / C;
  a.ng0 = it.ng0;
  a.r = r;
  a.p = p;
  a.q_sb = q_sb;
  a.q_st = q_st;
  a.k_sb = psi_buf ? fp.psi_sb : k_sb;
  a.k_st = psi_buf ? 128 : k_st;
  a.v_sb = v_sb;
  a.v_st = v_st;
  a.y_sb = y_sb;
  a.y_st = y_st;
  a.o_sb = o_sb;
  a.o_st = o_st;
  a.g_sb = g_sb;
  a.write_H = 0;
  return scan_stream_launch_feat(dtype, q, psi_buf ? psi_buf : k, v, Sg, Y, gate, out, nb, ng, a,
                                 fa, psi_buf != nullptr, stream);
}

// ---------------------------------------------------------------------------
// The allocation-free variant: scratch in a fixed device array.
//
// `scratch` holds the group summaries and their segmented scan that the
// workspace of smat_causal_scan holds otherwise.  The name is a host-side
// stand-in, not a device address: host code uses the address that
// hipGetSymbolAddress returns for the current device (each GPU holds its own
// copy of the array), looked up once per device on the first call there.
// Every element the kernels read from it is written earlier in the same call
// (all group summaries, then their scan), so nothing needs clearing; calls
// that overlap on one GPU (different streams) share the array and race.
// ---------------------------------------------------------------------------

constexpr int64_t kNoAllocScratchBytes = 64ll << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("smat_causal_scan_noalloc: no current device (%s, device %d)",
              hipGetErrorString(e), dev);
    return SMAT_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("smat_causal_scan_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                hipGetErrorString(e));
      return SMAT_ELAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SMAT_OK;
}

// Scratch bytes for group size K (as causal_scan_workspace_bytes at its K).
static int64_t scan_scratch_bytes(int nb, int nc, int K, int r, int p) {
  const int ng = (nc + K - 1) / K + 1;
  return 2 * (((int64_t)nb * ng * r * p * 4 + 255) & ~(int64_t)255);
}

// The group size of the allocating entry point when its scratch fits the
// array, else the least power-of-two multiple of it that fits (larger groups,
// fewer summaries; 0 when not even one group per segment fits).
static int noalloc_group_chunks(int nb, int nc, int r, int p) {
  int K = scan_group_chunks(nb, nc);
  while (scan_scratch_bytes(nb, nc, K, r, p) > kNoAllocScratchBytes) {
    if (K >= nc) return 0;
    K *= 2;
  }
  return K;
}

}  // namespace smat

extern "C" int64_t smat_causal_scan_noalloc_max_bytes(void) {
  return smat::kNoAllocScratchBytes;
}

extern "C" int smat_causal_scan_noalloc(int dtype, const void* phi, const void* psi,
                                        const void* vb, const float* Y, const float* gate,
                                        float* out, int nb, int T, int n, int C, int r, int p,
                                        int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                                        int64_t v_sb, int64_t v_st, int64_t y_sb, int64_t y_st,
                                        int64_t o_sb, int64_t o_st, int64_t g_sb, int write_H,
                                        void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && out, SMAT_EINVAL, "smat_causal_scan_noalloc: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && C >= 1 && C <= sf::kC, SMAT_EUNSUPPORTED,
               "smat_causal_scan_noalloc: chunk C=%d not in [1, %d]", C, sf::kC);
  SMAT_REQUIRE(n >= 0 && n <= T && n % C == 0, SMAT_EINVAL,
               "smat_causal_scan_noalloc: n=%d must be a multiple of C=%d in [0, T]", n, C);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 2 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_causal_scan_noalloc: r=%d p=%d beyond r<=%d, 2<=p<=%d", r, p, kMaxR,
               kMaxP);
  SMAT_REQUIRE(q_st >= r && k_st >= r && v_st >= p && o_st >= (write_H ? p : p - 1),
               SMAT_EINVAL, "smat_causal_scan_noalloc: a row stride is shorter than its row");
  if (nb == 0 || T == 0) return SMAT_OK;
  const int nc = (T + C - 1) / C;
  const int K = noalloc_group_chunks(nb, nc, r, p);
  SMAT_REQUIRE(K > 0, SMAT_EUNSUPPORTED,
               "smat_causal_scan_noalloc: nb=%d sequences of r=%d x p=%d states need more "
               "than the %lld-byte scratch array even with one group per segment; use "
               "smat_causal_scan with a workspace",
               nb, r, p, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return causal_scan_run(dtype, phi, psi, vb, Y, gate, out, nb, T, n, C, K, r, p, q_sb, q_st,
                         k_sb, k_st, v_sb, v_st, y_sb, y_st, o_sb, o_st, g_sb, write_H, ws,
                         nullptr, 0, 3, (hipStream_t)stream);
}

extern "C" int64_t smat_causal_scan_workspace_bytes(int nb, int T, int C, int r, int p) {
  if (nb <= 0 || T <= 0 || C <= 0 || r <= 0 || p <= 0) return 0;
  return smat::causal_scan_workspace_bytes(nb, T, C, r, p);
}

extern "C" int smat_causal_scan(int dtype, const void* phi, const void* psi, const void* vb,
                                const float* Y, const float* gate, float* out, int nb, int T,
                                int n, int C, int r, int p, int64_t q_sb, int64_t q_st,
                                int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                                int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st,
                                int64_t g_sb, int write_H, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && out && workspace, SMAT_EINVAL,
               "smat_causal_scan: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && C >= 1 && C <= sf::kC, SMAT_EUNSUPPORTED,
               "smat_causal_scan: chunk C=%d not in [1, %d]", C, sf::kC);
  SMAT_REQUIRE(n >= 0 && n <= T && n % C == 0, SMAT_EINVAL,
               "smat_causal_scan: n=%d must be a multiple of C=%d in [0, T]", n, C);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 2 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_causal_scan: r=%d p=%d beyond r<=%d, 2<=p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && k_st >= r && v_st >= p && o_st >= (write_H ? p : p - 1), SMAT_EINVAL,
               "smat_causal_scan: a row stride is shorter than its row");
  SMAT_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, SMAT_EINVAL,
               "smat_causal_scan: workspace must be 256-byte aligned");
  return causal_scan_dispatch(dtype, phi, psi, vb, Y, gate, out, nb, T, n, C, r, p, q_sb, q_st,
                              k_sb, k_st, v_sb, v_st, y_sb, y_st, o_sb, o_st, g_sb, write_H,
                              workspace, workspace_bytes, (hipStream_t)stream, nullptr, 0, 3);
}
