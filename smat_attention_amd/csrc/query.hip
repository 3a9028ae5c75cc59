// Type-major query  Y[i] = Phi_rec[i] U_{i mod B}  -- the application of R
// (src/smat/attention.py:310-330).
//
// rho(i) = i mod B makes the rows of type h the stride-B progression
// h, h+B, h+2B, ...; one workgroup takes up to 64 of them (four 16-row tiles)
// and one hyperplane's U_h, so U_h is read from HBM exactly once per 64 rows.
// The four waves split U_h's column tiles (wave w: tiles w, w+4, w+8), which
// also means each U element is loaded by exactly one lane.  Phi rows are
// gathered straight into A fragments (8 consecutive features per lane).  U is
// fp32; for 16-bit inputs each U fragment is split into hi + lo 16-bit parts
// (two MFMAs, ~16 mantissa bits), for fp32 inputs it goes to fp32 MFMA whole.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "feat_map.hpp"
#include "smat_host.hpp"

namespace smat {

namespace qy {
constexpr int kThreads = 256;
constexpr int kRowsPerWG = 64;
constexpr int kMT = kRowsPerWG / 16;
}  // namespace qy

// Tile shape: kRK k-blocks of 32 features and kNCT column tiles of 16, split
// over the four waves (wave w: tiles w, w + 4, ...).  Wide (4, 9): r <= 128,
// p <= 144.  Narrow (2, 5): r <= 64, p <= 80, half the accumulators and
// fragments, for head_dim 64; (3, 5) for contractions over head_dim + 1
// columns (r <= 96).
template <typename In, int kRK, int kNCT, bool kLoop>
__global__ __launch_bounds__(qy::kThreads) void query_kernel(
    const In* __restrict__ phi, const float* __restrict__ U, float* __restrict__ Y, int T_R, int B,
    int r, int p, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st, int nrb,
    int vec_q, const int32_t* __restrict__ rows, const int64_t* __restrict__ roffs) {
  using namespace qy;
  typedef typename Traits<In>::frag Frag;
  constexpr int kCTPerWave = (kNCT + 3) / 4;
  const int h = blockIdx.x / nrb;
  const int rb = blockIdx.x - h * nrb;
  const int64_t b = blockIdx.y;
  const int lane = lane_id(), w = wave_id();
  const int row16_ = lane & 15, grp_ = lane >> 4;
  const int rk = (r + 31) >> 5;
  const int nct = (p + 15) >> 4;
  // rows of type h: i = h + k*B, k < cnt -- or, with a row table, the rows
  // rows[roffs[h] .. roffs[h+1])
  const int cnt = rows ? (int)(roffs[h + 1] - roffs[h]) : (h < T_R) ? (T_R - h + B - 1) / B : 0;
  const int32_t* hrows = rows ? rows + roffs[h] : nullptr;
  // Row block rb alone (kLoop false: the grid covers every block), or row
  // blocks rb, rb + nrb, ... (kLoop true: a list longer than the grid was
  // sized for is still covered)
  for (int rbi = rb; rbi * kRowsPerWG < cnt; rbi += nrb) {
    const int k0 = rbi * kRowsPerWG;
    const int nmt = min(kMT, (cnt - k0 + 15) / 16);

    const In* phib = phi + b * q_sb;
    const float* Uh = U + (b * B + h) * u_ld;
    // U's loads, their offsets and predicates do not depend on the row block.
    // In the walk they are computed from opaque copies, so they stay inside it
    // instead of being hoisted into registers for a second pass that only
    // over-long lists take (63 VGPRs at r = 64 instead of 128).
    int pu = p, ru = r, row16 = row16_, grp = grp_;
    if constexpr (kLoop) asm volatile("" : "+s"(Uh), "+s"(pu), "+s"(ru), "+v"(row16), "+v"(grp));

    f32x4 acc[kMT][kCTPerWave];
#pragma unroll
    for (int t = 0; t < kMT; ++t)
#pragma unroll
      for (int j = 0; j < kCTPerWave; ++j) acc[t][j] = zero4();

    // this lane's row of each 16-row tile, looked up once (a list entry or
    // h + kB); the stores below take their rows from these lanes by shuffle
    int64_t ri[kMT];
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
      const int k = k0 + 16 * t + row16;
      ri[t] = !(k < cnt) ? 0 : hrows ? (int64_t)hrows[k] : (int64_t)h + (int64_t)k * B;
    }
#pragma unroll
    for (int kb = 0; kb < kRK; ++kb) {
      if (kb >= rk) continue;
      const int a0 = 32 * kb + 8 * grp;
      Frag pa[kMT];
#pragma unroll
      for (int t = 0; t < kMT; ++t) {
        const int k = k0 + 16 * t + row16;
        const int nv = (t < nmt && k < cnt) ? min(8, r - a0) : 0;
        pa[t] = load8<In>(phib + ri[t] * q_st + a0, nv, vec_q);
      }
#pragma unroll
      for (int j = 0; j < kCTPerWave; ++j) {
        const int ct = w + 4 * j;
        if (ct >= nct) continue;
        const int c = ct * 16 + row16;
        float u[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          u[e] = (c < pu && a0 + e < ru) ? Uh[(int64_t)(a0 + e) * pu + c] : 0.f;
        if constexpr (Traits<In>::split) {
          Frag bh, bl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            In hh, ll;
            split2<In>(u[e], hh, ll);
            bh[e] = hh;
            bl[e] = ll;
          }
#pragma unroll
          for (int t = 0; t < kMT; ++t) {
            if (t >= nmt) continue;
            acc[t][j] = mma(acc[t][j], pa[t], bh);
            acc[t][j] = mma(acc[t][j], pa[t], bl);
          }
        } else {
          Frag bf;
#pragma unroll
          for (int e = 0; e < 8; ++e) bf[e] = u[e];
#pragma unroll
          for (int t = 0; t < kMT; ++t) {
            if (t >= nmt) continue;
            acc[t][j] = mma(acc[t][j], pa[t], bf);
          }
        }
      }
    }

    float* Yb = Y + b * y_sb;
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
      if (t >= nmt) continue;
      // row of output element i4: tile row 4 grp + i4, held by lane 4 grp + i4
      int64_t ro[4];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int src = 4 * grp + i4;
        const int lo = __shfl((int)(ri[t] & 0xffffffff), src, 64);
        const int hi = __shfl((int)(ri[t] >> 32), src, 64);
        ro[i4] = ((int64_t)hi << 32) | (uint32_t)lo;
      }
#pragma unroll
      for (int j = 0; j < kCTPerWave; ++j) {
        const int ct = w + 4 * j;
        if (ct >= nct) continue;
        const int c = ct * 16 + row16;
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int k = k0 + 16 * t + 4 * grp + i4;
          if (k < cnt && c < p) Yb[ro[i4] * y_st + c] = acc[t][j][i4];
        }
      }
    }
    if constexpr (!kLoop) break;
  }
}

// ---------------------------------------------------------------------------
// Head-dim-128 variant (16-bit inputs, r = 128, p = 129): persistent
// workgroups of nine waves walk the (sequence, row type) items, MT 16-row
// tiles an item (MT = 3: up to 48 rows a type, MT = 4: up to 64).  The product
// is taken transposed, Y^T = U_h^T Phi^T: wave w owns column tile w, its A
// operand is U_h^T read from LDS and split hi/lo, its B operand the Phi rows
// (row chunks swizzled by row so sixteen rows read without bank conflicts),
// and each lane ends with four consecutive columns of one row -- 16-byte
// stores into Y rows padded to 4 floats.
//
// U_h (66 KB fp32) is copied HBM -> LDS with global_load_lds_dwordx4 in
// slices of one k-block (32 rows, 16.5 KB) through a ring of slots, the
// copies of the next slices in flight while one slice is multiplied; an
// item's Phi rows (12 or 16 KB) go to one of three buffers, copied just
// before the item's first slice.  Seven slots (six slices, 1.5 items, ahead)
// beside the three 12 KB Phi buffers; six beside 16 KB ones.  At MT = 3 this
// runs as fast as two whole-item buffers did (at about 90 % of a device copy's
// rate), and it leaves room for the fourth row tile, which two whole-item
// buffers do not (165 KB).
// ---------------------------------------------------------------------------

namespace qs {
constexpr int kWaves = 9;
constexpr int kThreads = 64 * kWaves;
constexpr int kR = 128, kP = 129;
constexpr int kKB = 4;                                    // slices (k-blocks) per item
constexpr int kSliceChunks = 32 * kP / 4;                 // 16-byte chunks of a slice: 1032
constexpr int kSliceLoads = (kSliceChunks + 63) / 64;     // wave-wide copies: 17
constexpr int kSlotFloats = kSliceLoads * 256;            // 4352 (the tail included)
constexpr int kPhiBufs = 3;
template <int MT>
struct Shape {
  static constexpr int kPhiLoads = 16 * MT * 16 / 64;     // MT x 16 rows x 16 chunks: 12 or 16
  static constexpr int kPhiChunks = kPhiLoads * 64;
  static constexpr int kSlots = MT == 3 ? 7 : 6;
  static constexpr int kAhead = kSlots - 1;               // slices issued ahead
  static constexpr int kLds = kSlots * kSlotFloats * 4 + kPhiBufs * kPhiChunks * 16;
  static_assert(kLds <= 160 * 1024, "LDS");
  // copies wave w issues for a slice and for a Phi block (copies w and w + 9)
  static constexpr int slice_loads(int w) { return w + kWaves < kSliceLoads ? 2 : 1; }
  static constexpr int phi_loads(int w) { return w + kWaves < kPhiLoads ? 2 : 1; }
  static_assert(kSliceLoads <= 2 * kWaves && kPhiLoads <= 2 * kWaves, "two copies a wave");
  // Phi blocks among slices j + 1 .. j + kAhead - 1 when slice j is k-block kb
  static constexpr int phi_after(int kb) {
    int z = 0;
    for (int k = kb + 1; k < kb + kAhead; ++k) z += k % kKB == 0;
    return z;
  }
  // The slice copies before j + kAhead - 1 and one Phi block each item: with
  // kAhead slots ahead, item i + kAhead / kKB + 1's Phi copy goes out once
  // item i's last use of its buffer is past a barrier.
  static_assert((kAhead + kKB - 1) / kKB + 1 <= kPhiBufs, "Phi buffers in use at once");
};
}  // namespace qs

// The copies of k-block kb of item into a ring slot, preceded, for the first
// k-block, by the item's Phi rows into pbuf: older than the slice's copies,
// they have landed whenever the slice has.  Untracked (the waits are the
// kernel's own); lanes past the slice re-read its first chunk, rows past the
// type's count its first row.
template <typename In, int MT>
__device__ __forceinline__ void query_issue(float* slot, uint4* pbuf, const float* U,
                                            const In* phi, int64_t item, int kb, int T_R, int B,
                                            int64_t u_ld, int64_t q_sb, int64_t q_st, int w,
                                            int lane) {
  using namespace qs;
  if (kb == 0) {
    const int64_t b = item / B;
    const int h = (int)(item - b * B);
    const int cnt = (T_R - h + B - 1) / B;
    const In* phib = phi + b * q_sb;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int I = w + kWaves * u;
      if (I < Shape<MT>::kPhiLoads) {
        const int row = 4 * I + (lane >> 4);
        const int k = (lane & 15) ^ (row & 15);
        const int rr = row < cnt ? row : 0;
        lds_dma16<true>(phib + ((int64_t)h + (int64_t)rr * B) * q_st + 8 * k, pbuf + 64 * I);
      }
    }
  }
  const float* Us = U + item * u_ld + (int64_t)kb * (32 * kP);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int I = w + kWaves * u;
    if (I < kSliceLoads) {
      const int c = 64 * I + lane;
      lds_dma16<true>(Us + 4 * (c < kSliceChunks ? c : 0), slot + 256 * I);
    }
  }
}

// Before slice j (k-block KB) is read: the copies issued after its own are
// those of slices j + 1 .. j + kAhead - 1 and the Phi block of each first
// slice among them, so waiting down to their number lands slice j and its Phi
// block.  Three classes of waves issue different numbers of copies.
template <int MT, int KB>
__device__ __forceinline__ void query_wait(int w) {
  using S = qs::Shape<MT>;
  constexpr int kAfter = S::kAhead - 1;
  constexpr int z = S::phi_after(KB);
  constexpr int kP2 = S::kPhiLoads - qs::kWaves;          // waves with two Phi copies
  static_assert(S::slice_loads(kP2 - 1) == 2 && S::slice_loads(7) == 2 &&
                    S::slice_loads(8) == 1 && S::phi_loads(kP2) == 1 && kP2 <= 8,
                "the three wave classes");
  if (w < kP2)
    wait_vmcnt<kAfter * 2 + z * 2>();
  else if (w < 8)
    wait_vmcnt<kAfter * 2 + z * 1>();
  else
    wait_vmcnt<kAfter * 1 + z * 1>();
}

// FEAT: phi holds Q rows; each item's Phi rows are formed in place from the
// copied Q rows (feat_rows: waves 0..7 one feature tile each, W in registers;
// wave 8 meets the barriers).
template <typename In, bool FEAT, int MT>
__global__ __launch_bounds__(qs::kThreads, 1) void query_stream_kernel(
    const In* __restrict__ phi, const float* __restrict__ U, float* __restrict__ Y, int T_R,
    int B, int64_t nitems, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st,
    FeatArgs fa) {
  using namespace qs;
  using S = Shape<MT>;
  typedef typename Traits<In>::frag Frag;
  __shared__ __attribute__((aligned(16))) float ring[S::kSlots * kSlotFloats];
  __shared__ __attribute__((aligned(16))) uint4 pbufs[kPhiBufs * S::kPhiChunks];
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  __builtin_assume(w >= 0 && w < kWaves);
  const int64_t G = gridDim.x;
  const int64_t item0 = blockIdx.x;
  const int nmine = item0 < nitems ? (int)((nitems - 1 - item0) / G + 1) : 0;
  const int nsl = kKB * nmine;                        // slices this workgroup walks
  Frag wa[4];
  if constexpr (FEAT) {
    if (w < 8) {
      feat_w_load<In>(wa, (const In*)fa.W, w, lane_id());
      // landed here, before any copy: no compiler wait for W inside the loop
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(wa[kb]));
    }
  }
  for (int j = 0; j < S::kAhead && j < nsl; ++j)
    query_issue<In, MT>(ring + j * kSlotFloats, pbufs + ((j / kKB) % kPhiBufs) * S::kPhiChunks,
                        U, phi, item0 + (int64_t)(j / kKB) * G, j % kKB, T_R, B, u_ld, q_sb,
                        q_st, w, lane_id());

  f32x4 acc[MT];
  int slot = 0;                                       // j mod kSlots
  int pbi = 0;                                        // (j / kKB) mod kPhiBufs
  auto step = [&](auto KBC, int j, int64_t item) {
    constexpr int KB = decltype(KBC)::value;
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int r16 = lane & 15, g = lane >> 4;
    if (j + S::kAhead - 1 < nsl)
      query_wait<MT, KB>(w);
    else
      wait_vmcnt<0>();
    lds_barrier();      // slice j (and its Phi block) is in LDS; slice j - 1's slot is free
    if (j + S::kAhead < nsl) {
      // slice j + kAhead: k-block (KB + kAhead) % 4 of the item that many ahead
      constexpr int kbn = (KB + S::kAhead) % kKB;
      constexpr int ahead = (KB + S::kAhead) / kKB;
      const int sn = slot == 0 ? S::kSlots - 1 : slot - 1;
      const int pn = (pbi + ahead) % kPhiBufs;
      query_issue<In, MT>(ring + sn * kSlotFloats, pbufs + pn * S::kPhiChunks, U, phi,
                          item + (int64_t)ahead * G, kbn, T_R, B, u_ld, q_sb, q_st, w, lane);
    }
    uint4* ps = pbufs + pbi * S::kPhiChunks;
    if constexpr (FEAT && KB == 0) {
      const float none[MT] = {};
      feat_rows<In, MT>(ps, ps, 0, w < 8, wa, w, fa.kind, false, none, lane,
                        [](int t) { return t & 15; });
      lds_barrier();    // the item's Phi rows are complete
    }
    const float* us = ring + slot * kSlotFloats;
    const int c = 16 * w + r16;
    // Lane group g takes the k-slots of feature group pg of each 32: 0, 2, 1, 3
    // for g = 0..3.  A 4-byte LDS read is served 32 lanes at a time, and U_h
    // rows 16 apart (rows of 129 floats) fall on disjoint banks where rows 8
    // apart overlap.  U_h^T and Phi^T agree on the order, so the product is
    // unchanged.
    const int pg = (g >> 1) | ((g & 1) << 1);
    if constexpr (KB == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = zero4();
    }
    Frag ah, al;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float uv = c < kP ? us[(8 * pg + e) * kP + c] : 0.f;
      In hh, ll;
      split2<In>(uv, hh, ll);
      ah[e] = hh;
      al[e] = ll;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int row = 16 * t + r16;
      const Frag pb = *reinterpret_cast<const Frag*>(ps + row * 16 + ((4 * KB + pg) ^ (row & 15)));
      acc[t] = mma(acc[t], ah, pb);
      acc[t] = mma(acc[t], al, pb);
    }
    if constexpr (KB == kKB - 1) {
      const int64_t b = item / B;
      const int h = (int)(item - b * B);
      const int cnt = (T_R - h + B - 1) / B;
      float* Yb = Y + b * y_sb;
      const int c0 = 16 * w + 4 * g;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int k = 16 * t + r16;
        if (k < cnt) {
          float* yrow = Yb + ((int64_t)h + (int64_t)k * B) * y_st;
          if (c0 + 3 < kP) {
            *reinterpret_cast<float4*>(yrow + c0) =
                make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (c0 + i < kP) yrow[c0 + i] = acc[t][i];
          }
        }
      }
      pbi = pbi == kPhiBufs - 1 ? 0 : pbi + 1;
    }
    slot = slot == S::kSlots - 1 ? 0 : slot + 1;
  };
  for (int j = 0; j < nsl; j += kKB) {
    const int64_t item = item0 + (int64_t)(j / kKB) * G;
    step(std::integral_constant<int, 0>{}, j, item);
    step(std::integral_constant<int, 1>{}, j + 1, item);
    step(std::integral_constant<int, 2>{}, j + 2, item);
    step(std::integral_constant<int, 3>{}, j + 3, item);
  }
}

template <typename In>
static int launch_query(const void* phi, const float* U, float* Y, int nb, int T_R, int B, int r,
                        int p, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                        int64_t y_st, hipStream_t stream);

static bool query_stream_ok(int dtype, const void* phi, const float* U, const float* Y, int T_R,
                            int B, int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb,
                            int64_t y_st) {
  if (dtype != SMAT_BF16 && dtype != SMAT_F16) return false;
  if (r != qs::kR || p != qs::kP) return false;
  if ((T_R + B - 1) / B > 64) return false;                 // <= 64 rows per type
  if (!rows_vec_ok(phi, q_sb, q_st, 2) || !aligned16(U) || !rows_vec_ok(Y, y_sb, y_st, 4))
    return false;
  return variant(SMAT_VARIANT_QUERY) == 0;
}

template <typename In>
static int launch_query(const void* phi, const float* U, float* Y, int nb, int T_R, int B, int r,
                        int p, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                        int64_t y_st, hipStream_t stream) {
  const int maxcnt = (T_R + B - 1) / B;
  const int nrb = (maxcnt + qy::kRowsPerWG - 1) / qy::kRowsPerWG;
  const int64_t gx = (int64_t)B * nrb;
  if (gx >= (1ll << 31)) {
    set_error("smat_query: problem too large");
    return SMAT_EUNSUPPORTED;
  }
  const int vq = rows_vec_ok(phi, q_sb, q_st, sizeof(In));
  if (r <= 64 && p <= 80)
    smat::launch((query_kernel<In, 2, 5, false>), dim3((unsigned)gx, (unsigned)nb),
                       dim3(qy::kThreads), 0, stream, (const In*)phi, U, Y, T_R, B, r, p, u_ld,
                       q_sb, q_st, y_sb, y_st, nrb, vq, nullptr, nullptr);
  else if (r <= 96 && p <= 80)
    smat::launch((query_kernel<In, 3, 5, false>), dim3((unsigned)gx, (unsigned)nb),
                       dim3(qy::kThreads), 0, stream, (const In*)phi, U, Y, T_R, B, r, p, u_ld,
                       q_sb, q_st, y_sb, y_st, nrb, vq, nullptr, nullptr);
  else
    smat::launch((query_kernel<In, 4, 9, false>), dim3((unsigned)gx, (unsigned)nb),
                       dim3(qy::kThreads), 0, stream, (const In*)phi, U, Y, T_R, B, r, p, u_ld,
                       q_sb, q_st, y_sb, y_st, nrb, vq, nullptr, nullptr);
  return launch_status("smat_query");
}

template <typename In>
static int launch_query_lists(const void* phi, const float* U, float* Y, const int32_t* rows,
                              const int64_t* roffs, int ntypes, int maxcnt, int r, int p,
                              int64_t q_st, int64_t y_st, hipStream_t stream) {
  // maxcnt only sizes the grid: a workgroup walks row blocks rb, rb + nrb, ...
  const int nrb = std::max(1, (maxcnt + qy::kRowsPerWG - 1) / qy::kRowsPerWG);
  const int64_t gx = (int64_t)ntypes * nrb;
  if (gx >= (1ll << 31)) {
    set_error("smat_query_lists: problem too large");
    return SMAT_EUNSUPPORTED;
  }
  if (gx == 0) return SMAT_OK;
  const int vq = rows_vec_ok(phi, 0, q_st, sizeof(In));
  if (r <= 64 && p <= 80)
    smat::launch((query_kernel<In, 2, 5, true>), dim3((unsigned)gx, 1u), dim3(qy::kThreads), 0,
                       stream, (const In*)phi, U, Y, 0, ntypes, r, p, (int64_t)r * p,
                       (int64_t)0, q_st, (int64_t)0, y_st, nrb, vq, rows, roffs);
  else if (r <= 96 && p <= 80)
    smat::launch((query_kernel<In, 3, 5, true>), dim3((unsigned)gx, 1u), dim3(qy::kThreads), 0,
                       stream, (const In*)phi, U, Y, 0, ntypes, r, p, (int64_t)r * p,
                       (int64_t)0, q_st, (int64_t)0, y_st, nrb, vq, rows, roffs);
  else
    smat::launch((query_kernel<In, 4, 9, true>), dim3((unsigned)gx, 1u), dim3(qy::kThreads), 0,
                       stream, (const In*)phi, U, Y, 0, ntypes, r, p, (int64_t)r * p,
                       (int64_t)0, q_st, (int64_t)0, y_st, nrb, vq, rows, roffs);
  return launch_status("smat_query_lists");
}

template <bool FEAT>
static int query_stream_go(int dtype, const void* phi, const float* U, float* Y, int nb, int T_R,
                           int B, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                           int64_t y_st, const FeatArgs& fa, hipStream_t stream) {
  int dev = 0, ncu = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t nitems = (int64_t)nb * B;
  const unsigned grid = (unsigned)std::min<int64_t>(nitems, (int64_t)ncu);
  // three row tiles up to 48 rows a type, four up to 64
  const bool four = (T_R + B - 1) / B > 48;
  if (dtype == SMAT_BF16) {
    if (four)
      smat::launch((query_stream_kernel<bf16, FEAT, 4>), dim3(grid), dim3(qs::kThreads), 0,
                   stream, (const bf16*)phi, U, Y, T_R, B, nitems, u_ld, q_sb, q_st, y_sb, y_st,
                   fa);
    else
      smat::launch((query_stream_kernel<bf16, FEAT, 3>), dim3(grid), dim3(qs::kThreads), 0,
                   stream, (const bf16*)phi, U, Y, T_R, B, nitems, u_ld, q_sb, q_st, y_sb, y_st,
                   fa);
  } else {
    if (four)
      smat::launch((query_stream_kernel<f16, FEAT, 4>), dim3(grid), dim3(qs::kThreads), 0,
                   stream, (const f16*)phi, U, Y, T_R, B, nitems, u_ld, q_sb, q_st, y_sb, y_st,
                   fa);
    else
      smat::launch((query_stream_kernel<f16, FEAT, 3>), dim3(grid), dim3(qs::kThreads), 0,
                   stream, (const f16*)phi, U, Y, T_R, B, nitems, u_ld, q_sb, q_st, y_sb, y_st,
                   fa);
  }
  return launch_status("smat_query");
}

static int launch_query_stream(int dtype, const void* phi, const float* U, float* Y, int nb,
                               int T_R, int B, int64_t u_ld, int64_t q_sb, int64_t q_st,
                               int64_t y_sb, int64_t y_st, hipStream_t stream) {
  return query_stream_go<false>(dtype, phi, U, Y, nb, T_R, B, u_ld, q_sb, q_st, y_sb, y_st,
                                FeatArgs{}, stream);
}

// The streaming query with the feature map in place: q holds Q rows of the
// recent block (d_qk = 128), U fp32 (nb, B) rows of 128 x 129 floats, u_ld
// floats apart, at most 48 rows a type.
int query_stream_launch_feat(int dtype, const void* q, const float* U, float* Y, int nb, int T_R,
                             int B, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                             int64_t y_st, const FeatArgs& fa, hipStream_t stream) {
  if (nb == 0 || T_R == 0 || B == 0) return SMAT_OK;
  return query_stream_go<true>(dtype, q, U, Y, nb, T_R, B, u_ld, q_sb, q_st, y_sb, y_st, fa,
                               stream);
}

// U: (nb, B) rows of r * p floats, u_ld floats apart (u_ld % 4 == 0 for the
// streaming kernel's 16-byte copies).
int query_dispatch(int dtype, const void* phi, const float* U, float* Y, int nb, int T_R, int B,
                   int r, int p, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                   int64_t y_st, hipStream_t stream) {
  if (nb == 0 || T_R == 0 || B == 0) return SMAT_OK;
  if (u_ld % 4 == 0 && query_stream_ok(dtype, phi, U, Y, T_R, B, r, p, q_sb, q_st, y_sb, y_st))
    return launch_query_stream(dtype, phi, U, Y, nb, T_R, B, u_ld, q_sb, q_st, y_sb, y_st,
                               stream);
  switch (dtype) {
    case SMAT_BF16:
      return launch_query<bf16>(phi, U, Y, nb, T_R, B, r, p, u_ld, q_sb, q_st, y_sb, y_st,
                                stream);
    case SMAT_F16:
      return launch_query<f16>(phi, U, Y, nb, T_R, B, r, p, u_ld, q_sb, q_st, y_sb, y_st, stream);
    case SMAT_F32:
      return launch_query<float>(phi, U, Y, nb, T_R, B, r, p, u_ld, q_sb, q_st, y_sb, y_st,
                                 stream);
  }
  set_error("smat_query: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}

}  // namespace smat

extern "C" int smat_query(int dtype, const void* phi_rec, const float* U, float* Y, int nb,
                          int T_R, int B, int r, int p, int64_t q_sb, int64_t q_st, int64_t y_sb,
                          int64_t y_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi_rec && U && Y, SMAT_EINVAL, "smat_query: null pointer");
  SMAT_REQUIRE(nb >= 0 && T_R >= 0 && B >= 1, SMAT_EINVAL, "smat_query: bad sizes");
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_query: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && y_st >= p, SMAT_EINVAL, "smat_query: row stride too short");
  return query_dispatch(dtype, phi_rec, U, Y, nb, T_R, B, r, p, (int64_t)r * p, q_sb, q_st, y_sb,
                        y_st, (hipStream_t)stream);
}

extern "C" int smat_query_lists(int dtype, const void* phi, const float* U, float* Y,
                                const int32_t* rows, const int64_t* roffs, int ntypes, int maxcnt,
                                int r, int p, int64_t q_st, int64_t y_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && U && Y && rows && roffs, SMAT_EINVAL, "smat_query_lists: null pointer");
  SMAT_REQUIRE(ntypes >= 0 && maxcnt >= 0, SMAT_EINVAL, "smat_query_lists: bad sizes");
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 1 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_query_lists: r=%d p=%d beyond r<=%d, p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && y_st >= p, SMAT_EINVAL, "smat_query_lists: row stride too short");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case SMAT_BF16:
      return launch_query_lists<bf16>(phi, U, Y, rows, roffs, ntypes, maxcnt, r, p, q_st, y_st, st);
    case SMAT_F16:
      return launch_query_lists<f16>(phi, U, Y, rows, roffs, ntypes, maxcnt, r, p, q_st, y_st, st);
    case SMAT_F32:
      return launch_query_lists<float>(phi, U, Y, rows, roffs, ntypes, maxcnt, r, p, q_st, y_st,
                                       st);
  }
  set_error("smat_query_lists: unknown dtype %d", dtype);
  return SMAT_EINVAL;
}
