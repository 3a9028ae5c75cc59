// Gram sums  G = sum_{t in set} Psi_t^T Vb_t  (r x p, fp32) over token sets
// that are arithmetic progressions {start + s*stride : s < count}.
//
// One kernel serves every place the schedule pools keys against values:
//   * chunk summaries D_c (src/smat/attention.py:162): stride 1, one chunk;
//   * profile pooling F_x (src/smat/attention.py:199-236, the Triton pool
//     kernel src/smat/kernels/triton_fwd.py:226-311): prof(j) = (j - n_P)
//     mod N0 is round-robin, so profile x is the progression n_P + x + s*N0;
//   * the global-channel rank-one term (src/smat/attention.py:422-425):
//     tokens [0, n_P), stride 1;
//   * the decoder's prefix pooling (src/smat/attention.py:515-519).
//
// MFMA layout: M = a (feature, r), N = c (value column, p), K = tokens.  Both
// operands need 8 consecutive TOKENS per lane, so each 32-token block of Psi
// and Vb is staged in LDS transposed (Psi^T[a][t], Vb^T[c][t]); wave w owns
// the 16-row tiles 2w and 2w+1 of G and every column tile.
#include "bwd_common.hpp"

namespace smat {

namespace gr {
constexpr int kThreads = 256;
constexpr int kBT = 32;                 // token granularity of split-K runs

// Tile shape: wave w owns the 16-row tiles kTW w .. kTW w + kTW - 1 of G and
// the first 16 kNCT columns.  Wide (2, 9): r <= 128, p <= 144; narrow (1, 5):
// r <= 64, p <= 80, a quarter of the accumulators and under half the LDS.
// Tokens per staged block: 64 for 16-bit inputs, 32 for fp32.
template <typename In> constexpr int bt() { return sizeof(In) == 4 ? 32 : 64; }
}  // namespace gr

// G = sum Psi_t^T Vb_t over one progression.  Each block of tokens is staged
// in LDS transposed (Psi^T[a][t], Vb^T[c][t]) from 8 x 8 tiles; the next
// block's tiles are loaded into registers while the current block is
// multiplied, so one memory latency per block overlaps the MFMAs.
template <typename In, bool VEC, int kTW, int kNCT>
__global__ __launch_bounds__(gr::kThreads, kTW == 1 ? 4 : 2) void gram_kernel(
    const In* __restrict__ psi, const In* __restrict__ vb, float* __restrict__ G,
    float* __restrict__ G_last, GramItems it, int r, int p, int64_t k_sb, int64_t k_st,
    int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si, int64_t gl_sb) {
  using namespace gr;
  typedef typename Traits<In>::frag Frag;
  constexpr int kB = bt<In>();
  constexpr int kTPad = kB + 8;           // LDS row length (tokens) of the transposed tiles
  constexpr int kRows = 64 * kTW;
  constexpr int kCols = 16 * kNCT;
  __shared__ __attribute__((aligned(16))) In psiT[kRows * kTPad];
  __shared__ __attribute__((aligned(16))) In vbT[kCols * kTPad];

  const int item = blockIdx.x / it.nsplit;
  const int sp = blockIdx.x - item * it.nsplit;
  const int64_t b = blockIdx.y;
  const int lane = lane_id(), w = wave_id();
  const int row16 = lane & 15, grp = lane >> 4;
  const int nrt = (r + 15) >> 4;     // 16-row tiles of G
  const int nct = (p + 15) >> 4;

  int64_t start, stride;
  int count;
  gram_item(it, item, start, stride, count);
  if (it.nsplit > 1) {           // this run: terms [sp*per, min((sp+1)*per, count))
    const int lo = sp * it.per;
    const int hi = min(count, lo + it.per);
    start += (int64_t)lo * stride;
    count = max(0, hi - lo);
  }

  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;

  f32x4 acc[kTW][kNCT];
#pragma unroll
  for (int t = 0; t < kTW; ++t)
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) acc[t][ct] = zero4();

  // staging: tiles [0, tpsi) are Psi's, the rest Vb's; a thread owns tiles
  // tid + j kThreads, at most kTiles of them
  const int nrows = nrt * 16, ncols = nct * 16;
  const int tpsi = (kB / 8) * (nrows / 8);
  const int ttot = tpsi + (kB / 8) * (ncols / 8);
  constexpr int kTiles = ((kB / 8) * (kRows / 8 + kCols / 8) + kThreads - 1) / kThreads;
  struct Pf {
    Tile8<In> tl[kTiles];
    int tt[kTiles], c0[kTiles];
    bool psi[kTiles], live[kTiles];
  } pf;
  auto stage_issue = [&](int s0) {
    const int64_t tok0 = gram_token(it, item, start, stride, s0);    // valid: s0 < count
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const int tile = threadIdx.x + j * kThreads;
      pf.live[j] = tile < ttot;
      if (!pf.live[j]) continue;
      const bool is_psi = tile < tpsi;
      const int tix = is_psi ? tile : tile - tpsi;
      const int per_row = is_psi ? nrows / 8 : ncols / 8;
      pf.psi[j] = is_psi;
      pf.tt[j] = (tix / per_row) * 8;
      pf.c0[j] = (tix % per_row) * 8;
      const In* rowp[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int sidx = s0 + pf.tt[j] + u;
        const int64_t tok = sidx < count ? gram_token(it, item, start, stride, sidx) : 0;
        rowp[u] = sidx < count ? (is_psi ? psib + tok * k_st : vbb + tok * v_st) : nullptr;
      }
      const In* safe = is_psi ? psib + tok0 * k_st : vbb + tok0 * v_st;
      if constexpr (VEC)
        tile8_issue<In>(pf.tl[j], rowp, safe, pf.c0[j], is_psi ? r : p);
      else
        tile8_load<In, false>(pf.tl[j], rowp, safe, pf.c0[j], is_psi ? r : p);
    }
  };
  auto stage_commit = [&]() {
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      if (!pf.live[j]) continue;
      if constexpr (VEC) tile8_finish<In>(pf.tl[j]);
      tile8_store_T<In>(pf.tl[j], pf.psi[j] ? psiT : vbT, kTPad, pf.c0[j], pf.tt[j]);
    }
  };

  if (count > 0) stage_issue(0);
  for (int s0 = 0; s0 < count; s0 += kB) {
    if (s0 > 0) lds_barrier();       // the previous block's readers are done
    stage_commit();
    lds_barrier();
    if (s0 + kB < count) stage_issue(s0 + kB);
#pragma unroll
    for (int ks = 0; ks < kB / 32; ++ks) {
#pragma unroll
      for (int t = 0; t < kTW; ++t) {
        const int rt = kTW * w + t;
        if (rt >= nrt) continue;
        const Frag a =
            *reinterpret_cast<const Frag*>(psiT + (rt * 16 + row16) * kTPad + 32 * ks + 8 * grp);
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
          if (ct >= nct) continue;
          const Frag bf = *reinterpret_cast<const Frag*>(vbT + (ct * 16 + row16) * kTPad +
                                                         32 * ks + 8 * grp);
          acc[t][ct] = mma(acc[t][ct], a, bf);
        }
      }
    }
  }

  // nsplit > 1: G is the partial buffer (nb, nitems, nsplit, r, p) and G_last
  // is unused; otherwise item nitems-1 goes to G_last when that is given.
  const int nitems = gridDim.x / it.nsplit;
  float* Gb;
  if (it.nsplit > 1)
    Gb = G + ((b * nitems + item) * it.nsplit + sp) * (int64_t)r * p;
  else
    Gb = (G_last != nullptr && item == nitems - 1) ? G_last + b * gl_sb : G + b * g_sb + item * g_si;
#pragma unroll
  for (int t = 0; t < kTW; ++t) {
    const int rt = kTW * w + t;
    if (rt >= nrt) continue;
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
      if (ct >= nct) continue;
      const int c = ct * 16 + row16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int a = rt * 16 + 4 * grp + i;
        if (a < r && c < p) Gb[(int64_t)a * p + c] = acc[t][ct][i];
      }
    }
  }
}

// Sum the nsplit partials of every (b, item) in run order into G / G_last.
__global__ __launch_bounds__(256) void gram_reduce_kernel(const float* __restrict__ part,
                                                          float* __restrict__ G,
                                                          float* __restrict__ G_last, int nitems,
                                                          int nsplit, int64_t rp, int64_t g_sb,
                                                          int64_t g_si, int64_t gl_sb) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int item = blockIdx.y;
  const int64_t b = blockIdx.z;
  if (e >= rp) return;
  const float* src = part + (b * nitems + item) * (int64_t)nsplit * rp + e;
  float acc = 0.f;
  for (int s = 0; s < nsplit; ++s) acc += src[(int64_t)s * rp];
  float* dst = (G_last != nullptr && item == nitems - 1) ? G_last + b * gl_sb
                                                          : G + b * g_sb + item * g_si;
  dst[e] = acc;
}

template <typename In, int TW, int NCT>
static int launch_gram_shape(const void* psi, const void* vb, float* G, float* G_last,
                       const GramItems& it, int nitems, int nb, int r, int p, int64_t k_sb,
                       int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                       int64_t gl_sb, float* partials, hipStream_t stream, const char* who) {
  const int64_t gx = (int64_t)nitems * it.nsplit;
  const int vk = rows_vec8_ok(psi, k_sb, k_st);
  const int vv = rows_vec8_ok(vb, v_sb, v_st);
  if (gx >= (1ll << 31) || nb >= 65536) {
    set_error("%s: problem too large", who);
    return SMAT_EUNSUPPORTED;
  }
  if (it.nsplit > 1) {
    if (vk && vv)
      smat::launch((gram_kernel<In, true, TW, NCT>), dim3((unsigned)gx, (unsigned)nb),
                         dim3(gr::kThreads), 0, stream, (const In*)psi, (const In*)vb, partials,
                         nullptr, it, r, p, k_sb, k_st, v_sb, v_st, 0, 0, 0);
    else
      smat::launch((gram_kernel<In, false, TW, NCT>), dim3((unsigned)gx, (unsigned)nb),
                         dim3(gr::kThreads), 0, stream, (const In*)psi, (const In*)vb, partials,
                         nullptr, it, r, p, k_sb, k_st, v_sb, v_st, 0, 0, 0);
    int st = launch_status(who);
    if (st != SMAT_OK) return st;
    const int64_t rp = (int64_t)r * p;
    smat::launch(gram_reduce_kernel, dim3((unsigned)((rp + 255) / 256), nitems, nb),
                       dim3(256), 0, stream, partials, G, G_last, nitems, it.nsplit, rp, g_sb,
                       g_si, gl_sb);
    return launch_status(who);
  }
  if (vk && vv)
    smat::launch((gram_kernel<In, true, TW, NCT>), dim3((unsigned)gx, (unsigned)nb),
                       dim3(gr::kThreads), 0, stream, (const In*)psi, (const In*)vb, G, G_last,
                       it, r, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb);
  else
    smat::launch((gram_kernel<In, false, TW, NCT>), dim3((unsigned)gx, (unsigned)nb),
                       dim3(gr::kThreads), 0, stream, (const In*)psi, (const In*)vb, G, G_last,
                       it, r, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb);
  return launch_status(who);
}

template <typename In>
static int launch_gram(const void* psi, const void* vb, float* G, float* G_last,
                       const GramItems& it, int nitems, int nb, int r, int p, int64_t k_sb,
                       int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                       int64_t gl_sb, float* partials, hipStream_t stream, const char* who) {
  if (r <= 64 && p <= 80)
    return launch_gram_shape<In, 1, 5>(psi, vb, G, G_last, it, nitems, nb, r, p, k_sb, k_st, v_sb,
                                       v_st, g_sb, g_si, gl_sb, partials, stream, who);
  return launch_gram_shape<In, 2, 9>(psi, vb, G, G_last, it, nitems, nb, r, p, k_sb, k_st, v_sb,
                                     v_st, g_sb, g_si, gl_sb, partials, stream, who);
}

// Choose the split of the longest progression so that a launch has enough
// workgroups to fill the GPU; returns bytes of partials needed (0: no split).
static int64_t plan_split(GramItems& it, int nitems, int nb, int max_count, int r, int p) {
  const int64_t wgs = (int64_t)nitems * nb;
  int nsplit = 1;
  if (wgs < 2048 && max_count > 8 * gr::kBT) {
    const int by_work = (max_count + 4 * gr::kBT - 1) / (4 * gr::kBT);   // >= 128 terms a run
    const int by_fill = (int)((2048 + wgs - 1) / wgs);
    nsplit = max(1, min(by_work, by_fill));
  }
  int per = (max_count + nsplit - 1) / nsplit;
  per = (per + gr::kBT - 1) / gr::kBT * gr::kBT;
  if (per > 0) nsplit = (max_count + per - 1) / per;
  if (nsplit < 1) nsplit = 1;
  it.nsplit = nsplit;
  it.per = per;
  return nsplit > 1 ? (int64_t)nb * nitems * nsplit * r * p * 4 : 0;
}


// Gram sums at r = 64, p = 65 for 16-bit inputs (the training shape), any
// progression or token list of GramItems: item i of sequence b sums its
// terms kB at a time (128 for chunk summaries, 32 for the short profiles and
// cell lists, whose workgroups then take a quarter of the LDS; the last
// block is staged in whole 32-row groups, rows past the end zero).  One workgroup of four waves per item: Psi's rows to LDS as
// 16-bit rows (swizzled), Vb's columns 0..63 the same and column 64 on its
// own; wave w forms rows 16w .. 16w+15 of G (features) across five
// value-column tiles, A = Psi^T and B = Vb read down the tokens with the
// transposing reads, 32 tokens a product (both operands exact in 16 bits).
// Item nitems-1 goes to G_last when that is given.
namespace cg {
constexpr int kThreads = 256;
}  // namespace cg

template <typename In, int kB>
__global__ __launch_bounds__(cg::kThreads) void gram64_kernel(
    const In* __restrict__ psi, const In* __restrict__ vb, float* __restrict__ G,
    float* __restrict__ G_last, GramItems it, int vec_v, int64_t k_sb, int64_t k_st,
    int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si, int64_t gl_sb) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 sPsi[kB * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sVb[kB * kRowChunks];
  __shared__ In sVb64[kB];

  const int item = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  int64_t start, stride;
  int count;
  gram_item(it, item, start, stride, count);
  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  // lane (m = 16 ct + lane % 16, g), k-slot e <- column m of row row0 + 8g + e
  auto col8 = [&](const uint4* tile, int row0, int ct) {
    const int k = 2 * ct + ((r16 & 3) >> 1), half = r16 & 1;
    const Half lo4 = cb_tr<In>(tile, row0 + 8 * g + (r16 >> 2), k, half);
    const Half hi4 = cb_tr<In>(tile, row0 + 8 * g + 4 + (r16 >> 2), k, half);
    Frag f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = lo4[e];
      f[4 + e] = hi4[e];
    }
    return f;
  };
  f32x4 acc[5];
#pragma unroll
  for (int ct = 0; ct < 5; ++ct) acc[ct] = zero4();
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  for (int s0 = 0; s0 < count; s0 += kB) {
    const int nv = min(kB, count - s0);              // valid rows of the block
    const int n32 = (nv + 31) & ~31;                 // rows staged (whole 32-row groups)
    if (s0 > 0) __syncthreads();                     // the last block's readers are done
    // Psi: n32 rows x 8 chunks
    for (int e = tid; e < n32 * kRowChunks; e += cg::kThreads) {
      const int row = e >> 3, k = e & 7;
      const int64_t t = gram_token(it, item, start, stride, s0 + (row < nv ? row : 0));
      uint4 v = *reinterpret_cast<const uint4*>(psib + t * k_st + 8 * k);
      if (row >= nv) v = z4;
      sPsi[cb_slot(row, k)] = v;
    }
    if (vec_v) {
      // Vb: nine 16-byte pieces a row (columns 0..71)
      for (int e = tid; e < n32 * 9; e += cg::kThreads) {
        const int row = e / 9, k = e - 9 * row;
        const int64_t t = gram_token(it, item, start, stride, s0 + (row < nv ? row : 0));
        uint4 v = *reinterpret_cast<const uint4*>(vbb + t * v_st + 8 * k);
        if (row >= nv) v = z4;
        if (k < 8)
          sVb[cb_slot(row, k)] = v;
        else
          sVb64[row] = __builtin_bit_cast(Frag, v)[0];
      }
    } else {
      for (int e = tid; e < n32 * kP; e += cg::kThreads) {
        const int row = e / kP, col = e - row * kP;
        const int64_t t = gram_token(it, item, start, stride, s0 + (row < nv ? row : 0));
        const In v = row < nv ? vbb[t * v_st + col] : from_f32<In>(0.f);
        if (col < 64)
          reinterpret_cast<In*>(sVb + cb_slot(row, col >> 3))[col & 7] = v;
        else
          sVb64[row] = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kB / 32; ++ks) {
      if (32 * ks >= nv) break;                      // uniform: the staged rows end at n32
      const Frag pa = col8(sPsi, 32 * ks, w);        // Psi^T rows 16w + r16
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) acc[ct] = mma(acc[ct], pa, col8(sVb, 32 * ks, ct));
      Frag bv;                                       // column 64: lane r16 = 0
#pragma unroll
      for (int e = 0; e < 8; ++e)
        bv[e] = r16 == 0 ? sVb64[32 * ks + 8 * g + e] : from_f32<In>(0.f);
      acc[4] = mma(acc[4], pa, bv);
    }
  }
  float* out = (G_last != nullptr && item == (int)gridDim.x - 1) ? G_last + b * gl_sb
                                                                 : G + b * g_sb + item * g_si;
#pragma unroll
  for (int ct = 0; ct < 5; ++ct) {
    const int col = 16 * ct + r16;
    if (col < kP) {
#pragma unroll
      for (int e = 0; e < 4; ++e) out[(16 * w + 4 * g + e) * kP + col] = acc[ct][e];
    }
  }
}

// The r = 64, p = 65 fast path: 16-bit inputs, Psi rows 16-byte aligned, and
// enough items to fill the device without split-K.
static bool gram64_ok(int dtype, const void* psi, int r, int p, int64_t k_sb, int64_t k_st,
                      int nitems, int nb) {
  return (dtype == SMAT_BF16 || dtype == SMAT_F16) && r == cb::kR && p == cb::kP &&
         rows_vec_ok(psi, k_sb, k_st, 2) && (int64_t)nitems * nb >= 512 && nb < 65536 &&
         variant(SMAT_VARIANT_GRAM) == 0;
}

static int gram64_launch(int dtype, const void* psi, const void* vb, float* G, float* G_last,
                         const GramItems& it, int nitems, int nb, int64_t k_sb, int64_t k_st,
                         int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si, int64_t gl_sb,
                         hipStream_t stream, const char* who) {
  // nine 16-byte pieces a row stay inside the row's stride
  const int vec_v = v_st >= 72 && v_st % 8 == 0 && v_sb % 8 == 0 && aligned16(vb);
  const dim3 grid((unsigned)nitems, (unsigned)nb);
  const bool wide = it.mode == 0;                    // chunk summaries: 128 or more terms
#define SMAT_G64(T_, B_)                                                                     \
  smat::launch(gram64_kernel<T_, B_>, grid, dim3(cg::kThreads), 0, stream, (const T_*)psi, \
               (const T_*)vb, G, G_last, it, vec_v, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb)
  if (dtype == SMAT_BF16) {
    if (wide)
      SMAT_G64(bf16, 128);
    else
      SMAT_G64(bf16, 32);
  } else {
    if (wide)
      SMAT_G64(f16, 128);
    else
      SMAT_G64(f16, 32);
  }
#undef SMAT_G64
  return launch_status(who);
}

bool gram_stream_ok(int dtype, const void* psi, const void* vb, int r, int p, int64_t k_sb,
                    int64_t k_st, int64_t v_sb, int64_t v_st, const GramItems& it, int nitems,
                    int nb);
int gram_stream_launch(int dtype, const void* psi, const void* vb, float* G, float* G_last,
                       const GramItems& it, int nitems, int nb, int p, int64_t k_sb,
                       int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                       int64_t gl_sb, hipStream_t stream, const char* who);

int gram_dispatch(int dtype, const void* psi, const void* vb, float* G, float* G_last,
                  const GramItems& it, int nitems, int nb, int r, int p, int64_t k_sb,
                  int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                  int64_t gl_sb, float* partials, hipStream_t stream, const char* who) {
  if (nitems == 0 || nb == 0) return SMAT_OK;
  if (gram64_ok(dtype, psi, r, p, k_sb, k_st, nitems, nb))
    return gram64_launch(dtype, psi, vb, G, G_last, it, nitems, nb, k_sb, k_st, v_sb, v_st, g_sb,
                         g_si, gl_sb, stream, who);
  if (gram_stream_ok(dtype, psi, vb, r, p, k_sb, k_st, v_sb, v_st, it, nitems, nb))
    return gram_stream_launch(dtype, psi, vb, G, G_last, it, nitems, nb, p, k_sb, k_st, v_sb, v_st,
                              g_sb, g_si, gl_sb, stream, who);
  if (it.nsplit > 1 && partials == nullptr) {
    set_error("%s: split-K needs a workspace", who);
    return SMAT_EINVAL;
  }
  switch (dtype) {
    case SMAT_BF16:
      return launch_gram<bf16>(psi, vb, G, G_last, it, nitems, nb, r, p, k_sb, k_st, v_sb, v_st,
                               g_sb, g_si, gl_sb, partials, stream, who);
    case SMAT_F16:
      return launch_gram<f16>(psi, vb, G, G_last, it, nitems, nb, r, p, k_sb, k_st, v_sb, v_st,
                              g_sb, g_si, gl_sb, partials, stream, who);
    case SMAT_F32:
      return launch_gram<float>(psi, vb, G, G_last, it, nitems, nb, r, p, k_sb, k_st, v_sb,
                                v_st, g_sb, g_si, gl_sb, partials, stream, who);
  }
  set_error("%s: unknown dtype %d", who, dtype);
  return SMAT_EINVAL;
}

// Chunk summaries for chunks of width C (K = 1) or groups of K chunks.
int chunk_states_dispatch(int dtype, const void* psi, const void* vb, float* D, int nb, int T,
                          int C, int K, int n, int r, int p, int64_t k_sb, int64_t k_st,
                          int64_t v_sb, int64_t v_st, float* partials, int64_t partial_bytes,
                          hipStream_t stream, int* ngroups_out, int* ng0_out) {
  GramItems it{};
  it.mode = 0;
  it.T = T;
  it.C = C;
  it.K = K;
  it.nc = (T + C - 1) / C;
  it.nc0 = n / C;
  it.ng0 = (it.nc0 + K - 1) / K;
  const int ng = it.ng0 + (it.nc - it.nc0 + K - 1) / K;
  if (ngroups_out) *ngroups_out = ng;
  if (ng0_out) *ng0_out = it.ng0;
  const int64_t need = plan_split(it, ng, nb, K * C, r, p);
  if (need > partial_bytes) {   // not enough scratch: run unsplit
    it.nsplit = 1;
    it.per = K * C;
  }
  const int64_t rp = (int64_t)r * p;
  return gram_dispatch(dtype, psi, vb, D, nullptr, it, ng, nb, r, p, k_sb, k_st, v_sb, v_st,
                       (int64_t)ng * rp, rp, 0, partials, stream, "smat_chunk_states");
}

static GramItems pool_items(int n_P, int n, int N0, bool glob, int nb, int r, int p,
                            int64_t* need) {
  GramItems it{};
  it.mode = 1;
  it.n_P = n_P;
  it.n = n;
  it.N0 = N0;
  const int nX = n - n_P;
  int maxc = (nX + N0 - 1) / N0;
  if (glob) maxc = maxc > n_P ? maxc : n_P;
  *need = plan_split(it, N0 + (glob ? 1 : 0), nb, maxc, r, p);
  return it;
}

int64_t pool_workspace_bytes(int nb, int n_P, int n, int N0, int r, int p, bool glob) {
  int64_t need = 0;
  pool_items(n_P, n, N0, glob, nb, r, p, &need);
  return need;
}

// F: (nb, N0) rows of r * p floats, f_ld floats apart.
int pool_dispatch(int dtype, const void* psi, const void* vb, float* F, float* F_glob, int nb,
                  int n_P, int n, int N0, int r, int p, int64_t k_sb, int64_t k_st, int64_t v_sb,
                  int64_t v_st, float* partials, int64_t partial_bytes, hipStream_t stream,
                  int64_t f_ld) {
  const bool glob = (F_glob != nullptr && n_P > 0);
  int64_t need = 0;
  GramItems it = pool_items(n_P, n, N0, glob, nb, r, p, &need);
  if (need > partial_bytes) {
    set_error("smat_pool: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)partial_bytes);
    return SMAT_EINVAL;
  }
  const int64_t rp = (int64_t)r * p;
  return gram_dispatch(dtype, psi, vb, F, glob ? F_glob : nullptr, it, N0 + (glob ? 1 : 0), nb, r,
                       p, k_sb, k_st, v_sb, v_st, (int64_t)N0 * f_ld, f_ld, rp, partials, stream,
                       "smat_pool");
}

// Unpooled long-range sums U_h = sum_{j in cols_h} Psi_{n_P+j}^T Vb_{n_P+j}: one
// item per row type over its compacted column list.
int direct_dispatch(int dtype, const void* psi, const void* vb, const int32_t* cols,
                    const int32_t* counts, int kappa, float* U, int nb, int B, int n_P, int r,
                    int p, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                    hipStream_t stream) {
  GramItems it{};
  it.mode = 2;
  it.n_P = n_P;
  it.cols = cols;
  it.counts = counts;
  it.kappa = kappa;
  it.nsplit = 1;
  it.per = 1 << 30;
  const int64_t rp = (int64_t)r * p;
  return gram_dispatch(dtype, psi, vb, U, nullptr, it, B, nb, r, p, k_sb, k_st, v_sb, v_st,
                       (int64_t)B * rp, rp, 0, nullptr, stream, "smat_direct");
}

// Gram sums over token lists in CSR form: item i sums rows tokens[offs[i] ..
// offs[i+1]) of the (rows, r) / (rows, p) matrices psi / vb -- the pool of a
// content-addressed assignment, items (sequence, cell) over tokens sorted by
// cell.  G: (nitems, r, p) contiguous.
int gram_lists_dispatch(int dtype, const void* psi, const void* vb, const int32_t* tokens,
                        const int64_t* offs, float* G, int nitems, int r, int p, int64_t k_st,
                        int64_t v_st, hipStream_t stream) {
  GramItems it{};
  it.mode = 2;
  it.n_P = 0;
  it.cols = tokens;
  it.offs = offs;
  it.nsplit = 1;
  it.per = 1 << 30;
  const int64_t rp = (int64_t)r * p;
  return gram_dispatch(dtype, psi, vb, G, nullptr, it, nitems, 1, r, p, 0, k_st, 0, v_st, 0, rp,
                       0, nullptr, stream, "smat_gram_lists");
}

}  // namespace smat

extern "C" int smat_chunk_states(int dtype, const void* psi, const void* vb, float* D, int nb,
                                 int T, int C, int r, int p, int64_t k_sb, int64_t k_st,
                                 int64_t v_sb, int64_t v_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && D, SMAT_EINVAL, "smat_chunk_states: null pointer");
  SMAT_REQUIRE(nb >= 0 && T >= 0 && C >= 1 && C <= kMaxC, SMAT_EINVAL,
               "smat_chunk_states: bad sizes (C=%d)", C);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_chunk_states: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(k_st >= r && v_st >= p, SMAT_EINVAL, "smat_chunk_states: row stride too short");
  return chunk_states_dispatch(dtype, psi, vb, D, nb, T, C, 1, 0, r, p, k_sb, k_st, v_sb, v_st,
                               nullptr, 0, (hipStream_t)stream, nullptr, nullptr);
}

extern "C" int64_t smat_pool_workspace_bytes(int nb, int n_P, int n, int N0, int r, int p) {
  if (nb <= 0 || N0 < 1 || n_P < 0 || n < n_P) return 0;
  return smat::pool_workspace_bytes(nb, n_P, n, N0, r, p, n_P > 0);
}

extern "C" int smat_pool(int dtype, const void* psi, const void* vb, float* F, float* F_glob,
                         int nb, int n_P, int n, int N0, int r, int p, int64_t k_sb, int64_t k_st,
                         int64_t v_sb, int64_t v_st, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && F, SMAT_EINVAL, "smat_pool: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && n_P >= 0 && n >= n_P, SMAT_EINVAL,
               "smat_pool: need N0 >= 1 and 0 <= n_P <= n (N0=%d n_P=%d n=%d)", N0, n_P, n);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_pool: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(k_st >= r && v_st >= p, SMAT_EINVAL, "smat_pool: row stride too short");
  SMAT_REQUIRE(workspace == nullptr || aligned16(workspace), SMAT_EINVAL,
               "smat_pool: workspace must be 16-byte aligned");
  return pool_dispatch(dtype, psi, vb, F, F_glob, nb, n_P, n, N0, r, p, k_sb, k_st, v_sb, v_st,
                       (float*)workspace, workspace ? workspace_bytes : 0, (hipStream_t)stream,
                       (int64_t)r * p);
}

extern "C" int smat_direct(int dtype, const void* psi, const void* vb, const int32_t* cols,
                           const int32_t* counts, int kappa, float* U, int nb, int B, int n_P,
                           int r, int p, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                           void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && cols && counts && U, SMAT_EINVAL, "smat_direct: null pointer");
  SMAT_REQUIRE(nb >= 0 && B >= 0 && kappa >= 0 && n_P >= 0, SMAT_EINVAL,
               "smat_direct: bad sizes");
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_direct: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(k_st >= r && v_st >= p, SMAT_EINVAL, "smat_direct: row stride too short");
  return direct_dispatch(dtype, psi, vb, cols, counts, kappa, U, nb, B, n_P, r, p, k_sb, k_st,
                         v_sb, v_st, (hipStream_t)stream);
}

extern "C" int smat_gram_lists(int dtype, const void* psi, const void* vb, const int32_t* tokens,
                               const int64_t* offs, float* G, int nitems, int r, int p,
                               int64_t k_st, int64_t v_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(psi && vb && tokens && offs && G, SMAT_EINVAL, "smat_gram_lists: null pointer");
  SMAT_REQUIRE(nitems >= 0, SMAT_EINVAL, "smat_gram_lists: bad sizes");
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_gram_lists: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(k_st >= r && v_st >= p, SMAT_EINVAL, "smat_gram_lists: row stride too short");
  return gram_lists_dispatch(dtype, psi, vb, tokens, offs, G, nitems, r, p, k_st, v_st,
                             (hipStream_t)stream);
}
