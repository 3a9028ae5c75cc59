// Fused backward of the intra-chunk causal scan for 16-bit inputs at
// r = 64 features and p = 65 value columns (head_dim 64 plus the ones column),
// chunks of C = 128 tokens -- the training shape.  Per chunk, with the
// chunk's incoming state Sin (r x p) and the state Q flowing backwards from
// the later chunks of its segment (r x p, the exclusive reverse scan of
// Phi^T dH):
//
//   A  = tril(Phi Psi^T),   dA = tril(dH Vb^T)               (C x C, on chip)
//   dPhi = dA Psi + dH Sin^T
//   dPsi = dA^T Phi + Vb Q^T
//   dVb  = A^T dH + Psi Q
//
// (the gradient of src/smat/attention.py:134-192 inside one chunk; the
// reference fuses the same products in src/smat/kernels/triton_bwd.py:49-147
// as a row-parallel dPhi kernel and a column-parallel dPsi/dVb kernel.)
//
// One workgroup of eight waves per (sequence, chunk).  The chunk's Phi, Psi,
// Vb, dH, Sin and Q are staged in LDS once.  Wave w then does two passes:
//
//   * row pass, row tile i = w (tokens 16w .. 16w+15): for every column tile
//     s <= i it forms the 16 x 16 block of dA^T = Vb dH^T in MFMA
//     accumulators and feeds it, split hi/lo, straight back in as the B
//     operand of dPhi^T = Psi^T dA^T (+ Sin dH^T);
//   * column pass, column tile j = w: for every row tile t >= j it forms the
//     blocks of dA = dH Vb^T and A = Phi Psi^T the same way and feeds them to
//     dPsi^T = Phi^T dA (+ Q Vb^T) and dVb^T = dH^T A (+ Q^T Psi^T).
//
// The row pass of wave w visits w + 1 tiles and the column pass 8 - w, so
// every wave does the same work.  The outputs are formed transposed so that
// each lane ends with four consecutive columns of one token row.
//
// k-slot order.  A 16 x 16 accumulator tile gives lane (n, g) rows 4g .. 4g+3;
// two tiles give it {4g + e, 16 + 4g + e}.  The MFMA contracts over any order
// of its 32 k-slots as long as both operands use it, so a pair of
// accumulator tiles is a B operand as it stands, and the matching A operand
// is read from LDS along those tokens: the gfx950 transposing read
// ds_read_b64_tr_b16 returns four consecutive token rows of one column per
// lane.
//
// Precision: Phi, Psi and Vb are exact in the MFMA's 16-bit inputs; every
// fp32 operand (dH, Sin, Q, A, dA) goes in as hi + lo (about 2^-17
// relative), and a product of two fp32 operands takes hi.hi + hi.lo + lo.hi.
// Value column 64 (the ones column) is the K = 16 tail of the contractions
// over p and a fifth output column tile of dVb.
//
// LDS: Phi, Psi and Vb columns 0..63 as 128 rows of 128 bytes, 16-byte chunk
// k of row t at k ^ (t & 6), which keeps both the row-wise 16-byte reads and
// the transposing reads free of bank conflicts; Vb column 64 on its own; dH,
// Sin and Q as fp32 rows of 68 floats (column reads by sixteen lanes of rows
// 4 or 8 apart fall on disjoint banks).
#include "bwd_common.hpp"

namespace smat {

struct ChunkBwdArgs {
  int nc;                       // chunks per sequence
  int vec_dh, vec_vb;           // dH / Vb staged in 16-byte loads (see the kernel)
  int64_t q_sb, q_st, k_sb, k_st, v_sb, v_st;   // Phi, Psi, Vb (elements)
  int64_t h_sb, h_st;           // dH (floats)
  int64_t d_sb, d_st;           // dPhi and dPsi (elements of Out)
  int64_t e_sb, e_st;           // dVb (elements of Out)
  // optional fp32 terms added before the store (NULL: none): add_phi on rows
  // [add_split, add_end) of dPhi, add_psi and add_vb on rows [0, add_split)
  // of dPsi and dVb; rows are addressed by their absolute index
  const float* add_phi;
  const float* add_psi;
  const float* add_vb;
  int64_t ap_sb, ap_st, ak_sb, ak_st, av_sb, av_st;
  int64_t add_split, add_end;
};

template <typename In, typename Out>
__global__ __launch_bounds__(cb::kThreads, 1) void chunk_bwd_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ dH, const float* __restrict__ Sin, const float* __restrict__ Qs,
    Out* __restrict__ dPhi, Out* __restrict__ dPsi, Out* __restrict__ dVb, ChunkBwdArgs a) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 sPhi[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sPsi[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sVb[kC * kRowChunks];
  // the fp32 operands split once into 16-bit hi and lo tiles, laid out as the
  // 16-bit ones (columns 0..63 swizzled, column 64 on its own)
  __shared__ __attribute__((aligned(16))) uint4 sdHh[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sdHl[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sSinh[kR * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sSinl[kR * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sQh[kR * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sQl[kR * kRowChunks];
  __shared__ In sVb64[kC], sdH64h[kC], sdH64l[kC];
  __shared__ In sSin64h[kR], sSin64l[kR], sQ64h[kR], sQ64l[kR];

  const int c = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)c * kC;
  const In* phib = phi + b * a.q_sb + t0 * a.q_st;
  const In* psib = psi + b * a.k_sb + t0 * a.k_st;
  const In* vbb = vb + b * a.v_sb + t0 * a.v_st;
  const float* dHb = dH + b * a.h_sb + t0 * a.h_st;
  const int64_t st_off = ((int64_t)b * a.nc + c) * (kR * kP);
  const float* Sinb = Sin + st_off;
  const float* Qb = Qs + st_off;

  // ---- stage the chunk in LDS -------------------------------------------
  // Phi and Psi rows: 64 elements, 16-byte aligned (checked on the host).
  // Sin and Q (64 x 65 floats, contiguous) as float4s.  dH as float4s of the
  // chunk's contiguous block when its rows are 65 floats apart (vec_dh); Vb
  // as nine 16-byte pieces a row (columns 0..71: 64 to the swizzled rows,
  // column 64 from the ninth) when its rows are 16-byte aligned and at least
  // 72 elements apart (vec_vb); otherwise element-wise, consecutive threads
  // on consecutive elements.  All loads are issued before the first LDS
  // write.
  constexpr int kVbN = kC * kP;                     // 8320
  constexpr int kVbIt = (kVbN + kThreads - 1) / kThreads;   // 17
  constexpr int kS4 = kR * kP / 4;                  // 1040 float4s of Sin / Q
  constexpr int kS4It = (kS4 + kThreads - 1) / kThreads;    // 3
  constexpr int kH4 = kVbN / 4;                     // 2080 float4s of dH
  constexpr int kH4It = (kH4 + kThreads - 1) / kThreads;    // 5
  constexpr int kV16 = kC * 9;                      // 1152 16-byte pieces of Vb
  constexpr int kV16It = (kV16 + kThreads - 1) / kThreads;  // 3
  uint4 rphi[2], rpsi[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = tid + kThreads * u;              // chunk of 8 elements, < 1024
    const int row = e >> 3, k = e & 7;
    rphi[u] = *reinterpret_cast<const uint4*>(phib + row * a.q_st + 8 * k);
    rpsi[u] = *reinterpret_cast<const uint4*>(psib + row * a.k_st + 8 * k);
  }
  float4 rsin[kS4It], rq[kS4It];
#pragma unroll
  for (int u = 0; u < kS4It; ++u) {
    const int e4 = tid + kThreads * u;
    const int ee = e4 < kS4 ? e4 : 0;
    rsin[u] = reinterpret_cast<const float4*>(Sinb)[ee];
    rq[u] = reinterpret_cast<const float4*>(Qb)[ee];
  }
  // element e of a row-major block of rows of kP floats, split hi/lo, to its
  // place in a pair of 16-bit tiles (and their column-64 arrays)
  auto put = [](uint4* th, uint4* tl, In* h64, In* l64, int e, In h, In l) {
    const int row = e / kP, col = e - row * kP;
    if (col < 64) {
      reinterpret_cast<In*>(th + cb_slot(row, col >> 3))[col & 7] = h;
      reinterpret_cast<In*>(tl + cb_slot(row, col >> 3))[col & 7] = l;
    } else {
      h64[row] = h;
      l64[row] = l;
    }
  };
  auto put4 = [&](uint4* th, uint4* tl, In* h64, In* l64, int e, const float4& v) {
    Half h, l;
    split4<In>(f32x4{v.x, v.y, v.z, v.w}, h, l);
#pragma unroll
    for (int q = 0; q < 4; ++q) put(th, tl, h64, l64, e + q, h[q], l[q]);
  };
  if (a.vec_dh) {
    float4 rdh[kH4It];
#pragma unroll
    for (int u = 0; u < kH4It; ++u) {
      const int e4 = tid + kThreads * u;
      rdh[u] = reinterpret_cast<const float4*>(dHb)[e4 < kH4 ? e4 : 0];
    }
#pragma unroll
    for (int u = 0; u < kH4It; ++u) {
      const int e4 = tid + kThreads * u;
      if (e4 < kH4) put4(sdHh, sdHl, sdH64h, sdH64l, 4 * e4, rdh[u]);
    }
  } else {
    float rdh[kVbIt];
#pragma unroll
    for (int u = 0; u < kVbIt; ++u) {
      const int e = tid + kThreads * u;
      const int ee = e < kVbN ? e : 0;
      const int row = ee / kP, col = ee - row * kP;
      rdh[u] = dHb[row * a.h_st + col];
    }
#pragma unroll
    for (int u = 0; u < kVbIt; ++u) {
      const int e = tid + kThreads * u;
      if (e < kVbN) {
        In h, l;
        split2<In>(rdh[u], h, l);
        put(sdHh, sdHl, sdH64h, sdH64l, e, h, l);
      }
    }
  }
  if (a.vec_vb) {
    uint4 rvb[kV16It];
#pragma unroll
    for (int u = 0; u < kV16It; ++u) {
      const int q = tid + kThreads * u;
      const int qq = q < kV16 ? q : 0;
      const int row = qq / 9, k = qq - 9 * row;
      rvb[u] = *reinterpret_cast<const uint4*>(vbb + row * a.v_st + 8 * k);
    }
#pragma unroll
    for (int u = 0; u < kV16It; ++u) {
      const int q = tid + kThreads * u;
      if (q < kV16) {
        const int row = q / 9, k = q - 9 * row;
        if (k < 8)
          sVb[cb_slot(row, k)] = rvb[u];
        else
          sVb64[row] = __builtin_bit_cast(Frag, rvb[u])[0];
      }
    }
  } else {
    In rvb[kVbIt];
#pragma unroll
    for (int u = 0; u < kVbIt; ++u) {
      const int e = tid + kThreads * u;
      const int ee = e < kVbN ? e : 0;
      const int row = ee / kP, col = ee - row * kP;
      rvb[u] = vbb[row * a.v_st + col];
    }
#pragma unroll
    for (int u = 0; u < kVbIt; ++u) {
      const int e = tid + kThreads * u;
      if (e < kVbN) {
        const int row = e / kP, col = e - row * kP;
        if (col < 64)
          reinterpret_cast<In*>(sVb + cb_slot(row, col >> 3))[col & 7] = rvb[u];
        else
          sVb64[row] = rvb[u];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = tid + kThreads * u;
    const int row = e >> 3, k = e & 7;
    sPhi[cb_slot(row, k)] = rphi[u];
    sPsi[cb_slot(row, k)] = rpsi[u];
  }
#pragma unroll
  for (int u = 0; u < kS4It; ++u) {
    const int e4 = tid + kThreads * u;
    if (e4 < kS4) {
      put4(sSinh, sSinl, sSin64h, sSin64l, 4 * e4, rsin[u]);
      put4(sQh, sQl, sQ64h, sQ64l, 4 * e4, rq[u]);
    }
  }
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int lane = lane_id();
  const int r16 = lane & 15, g = lane >> 4;
  const Half hzero = {};
  // the K = 16 tail over value columns 64..79: column 64 in k-slot 0 of lane
  // group 0
  auto tail16 = [&](const In* h64, const In* l64, int row, Half& hi, Half& lo) {
    hi = hzero;
    lo = hzero;
    if (g == 0) {
      hi[0] = h64[row];
      lo[0] = l64[row];
    }
  };
  // A operand down 8 consecutive rows row0 + 8g .. +7 of a 16-bit tile: lane
  // (m = 16 ct + lane % 16, g), k-slot e <- column m of row row0 + 8g + e
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

  // ---- row pass: dPhi rows of tile i = w ----------------------------------
  {
    const int i = w;
    const int trow = 16 * i + r16;
    Frag dh_hi[2], dh_lo[2];
    Half dht_hi, dht_lo;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      dh_hi[kc] = cb_row<In>(sdHh, i, kc, lane);
      dh_lo[kc] = cb_row<In>(sdHl, i, kc, lane);
    }
    tail16(sdH64h, sdH64l, trow, dht_hi, dht_lo);

    f32x4 acc[4];
    // dPhi^T += Sin dH^T: A = Sin rows a (k = value column), B = dH^T
#pragma unroll
    for (int at = 0; at < 4; ++at) {
      f32x4 s = zero4();
      const int arow = 16 * at + r16;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const Frag hi = cb_row<In>(sSinh, at, kc, lane);
        const Frag lo = cb_row<In>(sSinl, at, kc, lane);
        s = mma(s, hi, dh_hi[kc]);
        s = mma(s, hi, dh_lo[kc]);
        s = mma(s, lo, dh_hi[kc]);
      }
      Half thi, tlo;
      tail16(sSin64h, sSin64l, arow, thi, tlo);
      s = mma_k16(s, thi, dht_hi);
      s = mma_k16(s, thi, dht_lo);
      s = mma_k16(s, tlo, dht_hi);
      acc[at] = s;
    }
    // dPhi^T += Psi^T dA^T over column tiles s <= i, two at a time
    for (int sp = 0; 2 * sp <= i; ++sp) {
      f32x4 dat[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int st = 2 * sp + h;
        f32x4 d = zero4();
        if (st <= i) {
          // dA^T[s][t] = sum_c Vb[s][c] dH[t][c]: A = Vb rows s, B = dH^T
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const Frag vf = cb_row<In>(sVb, st, kc, lane);
            d = mma(d, vf, dh_hi[kc]);
            d = mma(d, vf, dh_lo[kc]);
          }
          Half vt = hzero;
          if (g == 0) vt[0] = sVb64[16 * st + r16];
          d = mma_k16(d, vt, dht_hi);
          d = mma_k16(d, vt, dht_lo);
          if (st == i) {
            // lane (t = r16, g) holds s = 16 st + 4g + e: keep s <= t
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = 4 * g + e <= r16 ? d[e] : 0.f;
          }
        }
        dat[h] = d;
      }
      Frag bh, bl;
      cb_split_pair<In>(dat[0], dat[1], bh, bl);
      const int st1 = 2 * sp + 1 < 8 ? 2 * sp + 1 : 2 * sp;
#pragma unroll
      for (int at = 0; at < 4; ++at) {
        const Frag pa = cb_tr_pair<In>(sPsi, 2 * sp, st1, at, lane);
        acc[at] = mma(acc[at], pa, bh);
        acc[at] = mma(acc[at], pa, bl);
      }
    }
    // lane (t, g) holds dPhi[t][16 at + 4g + e]
    const int64_t row = t0 + trow;
    if (a.add_phi != nullptr && row >= a.add_split && row < a.add_end) {
      const float* ad = a.add_phi + b * a.ap_sb + row * a.ap_st + 4 * g;
#pragma unroll
      for (int at = 0; at < 4; ++at) {
        const float4 v = *reinterpret_cast<const float4*>(ad + 16 * at);
        acc[at][0] += v.x;
        acc[at][1] += v.y;
        acc[at][2] += v.z;
        acc[at][3] += v.w;
      }
    }
    Out* out = dPhi + b * a.d_sb + row * a.d_st;
#pragma unroll
    for (int at = 0; at < 4; ++at) store_grad4(out + 16 * at + 4 * g, acc[at]);
  }

  // ---- column pass: dPsi and dVb rows of tile j = w -----------------------
  {
    const int j = w;
    const int srow = 16 * j + r16;
    Frag vf[2], pf[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      vf[kc] = cb_row<In>(sVb, j, kc, lane);
      pf[kc] = cb_row<In>(sPsi, j, kc, lane);
    }
    Half vt = hzero;
    if (g == 0) vt[0] = sVb64[srow];

    f32x4 accq[4], accv[5];
    // dPsi^T += Q Vb^T: A = Q rows a, B = Vb^T
#pragma unroll
    for (int at = 0; at < 4; ++at) {
      f32x4 s = zero4();
      const int arow = 16 * at + r16;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        s = mma(s, cb_row<In>(sQh, at, kc, lane), vf[kc]);
        s = mma(s, cb_row<In>(sQl, at, kc, lane), vf[kc]);
      }
      Half thi, tlo;
      tail16(sQ64h, sQ64l, arow, thi, tlo);
      s = mma_k16(s, thi, vt);
      s = mma_k16(s, tlo, vt);
      accq[at] = s;
    }
    // dVb^T += Q^T Psi^T: A = Q^T (rows = value column c, k = feature a)
#pragma unroll
    for (int ct = 0; ct < 5; ++ct) {
      f32x4 s = zero4();
      const bool okc = 16 * ct + r16 < kP;
#pragma unroll
      for (int ka = 0; ka < 2; ++ka) {
        // A = Q^T: lane (c, g), k-slot e <- Q[32 ka + 8g + e][c]
        Frag hi, lo;
        if (ct < 4) {
          hi = col8(sQh, 32 * ka, ct);
          lo = col8(sQl, 32 * ka, ct);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            hi[e] = okc ? sQ64h[32 * ka + 8 * g + e] : from_f32<In>(0.f);
            lo[e] = okc ? sQ64l[32 * ka + 8 * g + e] : from_f32<In>(0.f);
          }
        }
        s = mma(s, hi, pf[ka]);
        s = mma(s, lo, pf[ka]);
      }
      accv[ct] = s;
    }
    // over row tiles t >= j, two at a time
    for (int tp = 0; j + 2 * tp < 8; ++tp) {
      const int tt0 = j + 2 * tp;
      const int tt1 = tt0 + 1 < 8 ? tt0 + 1 : tt0;
      const bool has1 = tt0 + 1 < 8;
      f32x4 da[2], aa[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tt = h ? tt1 : tt0;
        f32x4 d = zero4(), s = zero4();
        if (h == 0 || has1) {
          const int trow = 16 * tt + r16;
          // dA[t][s] = sum_c dH[t][c] Vb[s][c]: A = dH rows t, B = Vb^T
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            d = mma(d, cb_row<In>(sdHh, tt, kc, lane), vf[kc]);
            d = mma(d, cb_row<In>(sdHl, tt, kc, lane), vf[kc]);
            // A[t][s] = sum_a Phi[t][a] Psi[s][a]
            s = mma(s, cb_row<In>(sPhi, tt, kc, lane), pf[kc]);
          }
          Half thi, tlo;
          tail16(sdH64h, sdH64l, trow, thi, tlo);
          d = mma_k16(d, thi, vt);
          d = mma_k16(d, tlo, vt);
          if (tt == j) {
            // lane (s = r16, g) holds t = 16 tt + 4g + e: keep t >= s
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool keep = 4 * g + e >= r16;
              d[e] = keep ? d[e] : 0.f;
              s[e] = keep ? s[e] : 0.f;
            }
          }
        }
        da[h] = d;
        aa[h] = s;
      }
      Frag dah, dal, aah, aal;
      cb_split_pair<In>(da[0], da[1], dah, dal);
      cb_split_pair<In>(aa[0], aa[1], aah, aal);
      // dPsi^T += Phi^T dA
#pragma unroll
      for (int at = 0; at < 4; ++at) {
        const Frag pa = cb_tr_pair<In>(sPhi, tt0, tt1, at, lane);
        accq[at] = mma(accq[at], pa, dah);
        accq[at] = mma(accq[at], pa, dal);
      }
      // dVb^T += dH^T A: A operand = dH^T (rows = value column c, k = token t)
#pragma unroll
      for (int ct = 0; ct < 5; ++ct) {
        // A = dH^T: lane (c, g), k-slot 4h + e <- dH[16 tile[h] + 4g + e][c]
        Frag hi, lo;
        if (ct < 4) {
          hi = cb_tr_pair<In>(sdHh, tt0, tt1, ct, lane);
          lo = cb_tr_pair<In>(sdHl, tt0, tt1, ct, lane);
        } else {
          const bool okc = r16 == 0;                 // column 64
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int trr = 16 * (e < 4 ? tt0 : tt1) + 4 * g + (e & 3);
            hi[e] = okc ? sdH64h[trr] : from_f32<In>(0.f);
            lo[e] = okc ? sdH64l[trr] : from_f32<In>(0.f);
          }
        }
        if (!has1) {
#pragma unroll
          for (int e = 4; e < 8; ++e) {
            hi[e] = from_f32<In>(0.f);
            lo[e] = from_f32<In>(0.f);
          }
        }
        accv[ct] = mma(accv[ct], hi, aah);
        accv[ct] = mma(accv[ct], hi, aal);
        accv[ct] = mma(accv[ct], lo, aah);
      }
    }
    // lane (s, g) holds dPsi[s][16 at + 4g + e] and dVb[s][16 ct + 4g + e]
    const int64_t row = t0 + srow;
    if (a.add_psi != nullptr && row < a.add_split) {
      const float* ad = a.add_psi + b * a.ak_sb + row * a.ak_st + 4 * g;
#pragma unroll
      for (int at = 0; at < 4; ++at) {
        const float4 v = *reinterpret_cast<const float4*>(ad + 16 * at);
        accq[at][0] += v.x;
        accq[at][1] += v.y;
        accq[at][2] += v.z;
        accq[at][3] += v.w;
      }
    }
    if (a.add_vb != nullptr && row < a.add_split) {
      const float* ad = a.add_vb + b * a.av_sb + row * a.av_st;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) accv[ct][e] += ad[16 * ct + 4 * g + e];
      if (g == 0) accv[4][0] += ad[64];
    }
    Out* op = dPsi + b * a.d_sb + row * a.d_st;
#pragma unroll
    for (int at = 0; at < 4; ++at) store_grad4(op + 16 * at + 4 * g, accq[at]);
    Out* ov = dVb + b * a.e_sb + row * a.e_st;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[16 * ct + 4 * g + e] = from_f32<Out>(accv[ct][e]);
    if (g == 0) ov[64] = from_f32<Out>(accv[4][0]);
  }
}

bool chunk_bwd_ok(int dtype, int out_dtype, const void* phi, const void* psi, int r, int p,
                  int C, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t d_sb,
                  int64_t d_st, const void* dphi, const void* dpsi) {
  if (dtype != SMAT_BF16 && dtype != SMAT_F16) return false;
  if (out_dtype != SMAT_F32 && out_dtype != dtype) return false;
  if (r != cb::kR || p != cb::kP || C != cb::kC) return false;
  const int ob = elem_bytes(out_dtype);
  return rows_vec_ok(phi, q_sb, q_st, 2) && rows_vec_ok(psi, k_sb, k_st, 2) &&
         rows_vec_ok(dphi, d_sb, d_st, ob) && rows_vec_ok(dpsi, d_sb, d_st, ob);
}

template <typename In, typename Out>
static void chunk_bwd_launch(const void* phi, const void* psi, const void* vb, const float* dH,
                             const float* Sin, const float* Q, void* dPhi, void* dPsi, void* dVb,
                             const ChunkBwdArgs& a, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((chunk_bwd_kernel<In, Out>), grid, dim3(cb::kThreads), 0, st,
                     (const In*)phi, (const In*)psi, (const In*)vb, dH, Sin, Q, (Out*)dPhi,
                     (Out*)dPsi, (Out*)dVb, a);
}

// ---------------------------------------------------------------------------
// The per-chunk state gradient Dr_c = Phi_c^T dH_c (r x p fp32, one matrix per
// (sequence, chunk); the input of the reverse scan that gives Q), one
// workgroup of four waves per item.  Phi's chunk is staged as 16-bit rows
// (swizzled), dH's split into 16-bit hi/lo tiles as in chunk_bwd_kernel.
// Wave w forms rows 16w .. 16w+15 of Dr (features) across five value-column
// tiles: A = Phi^T and B = dH, both read down the chunk's tokens with the
// transposing reads, 32 tokens a product; lane (c, g) ends with
// Dr[16w + 4g + e][c].
// ---------------------------------------------------------------------------
namespace cds {
constexpr int kThreads = 256;
}  // namespace cds

template <typename In>
__global__ __launch_bounds__(cds::kThreads) void chunk_dstate_kernel(
    const In* __restrict__ phi, const float* __restrict__ dH, float* __restrict__ Dr, int nc,
    int vec_dh, int64_t q_sb, int64_t q_st, int64_t h_sb, int64_t h_st) {
  using namespace cb;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 sPhi[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sdHh[kC * kRowChunks];
  __shared__ __attribute__((aligned(16))) uint4 sdHl[kC * kRowChunks];
  __shared__ In sdH64h[kC], sdH64l[kC];

  const int c = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)c * kC;
  const In* phib = phi + b * q_sb + t0 * q_st;
  const float* dHb = dH + b * h_sb + t0 * h_st;
  constexpr int kN = kC * kP;                       // 8320 dH values
  constexpr int kPhiIt = kC * kRowChunks / cds::kThreads;   // 4
  constexpr int kH4 = kN / 4;                       // 2080 float4s
  constexpr int kH4It = (kH4 + cds::kThreads - 1) / cds::kThreads;   // 9
  constexpr int kHIt = (kN + cds::kThreads - 1) / cds::kThreads;     // 33

  auto put = [&](int e, In h, In l) {
    const int row = e / kP, col = e - row * kP;
    if (col < 64) {
      reinterpret_cast<In*>(sdHh + cb_slot(row, col >> 3))[col & 7] = h;
      reinterpret_cast<In*>(sdHl + cb_slot(row, col >> 3))[col & 7] = l;
    } else {
      sdH64h[row] = h;
      sdH64l[row] = l;
    }
  };
  // Phi's rows straight to LDS (issued after dH's loads, which stay in flight)
  auto put_phi = [&]() {
#pragma unroll
    for (int u = 0; u < kPhiIt; ++u) {
      const int e = tid + cds::kThreads * u;
      sPhi[cb_slot(e >> 3, e & 7)] =
          *reinterpret_cast<const uint4*>(phib + (e >> 3) * q_st + 8 * (e & 7));
    }
  };
  if (vec_dh) {
    float4 rdh[kH4It];
#pragma unroll
    for (int u = 0; u < kH4It; ++u) {
      const int e4 = tid + cds::kThreads * u;
      rdh[u] = reinterpret_cast<const float4*>(dHb)[e4 < kH4 ? e4 : 0];
    }
    put_phi();
#pragma unroll
    for (int u = 0; u < kH4It; ++u) {
      const int e4 = tid + cds::kThreads * u;
      if (e4 < kH4) {
        Half h, l;
        split4<In>(f32x4{rdh[u].x, rdh[u].y, rdh[u].z, rdh[u].w}, h, l);
#pragma unroll
        for (int q = 0; q < 4; ++q) put(4 * e4 + q, h[q], l[q]);
      }
    }
  } else {
    put_phi();
    for (int u = 0; u < kHIt; ++u) {
      const int e = tid + cds::kThreads * u;
      if (e < kN) {
        const int row = e / kP, col = e - row * kP;
        In h, l;
        split2<In>(dHb[row * h_st + col], h, l);
        put(e, h, l);
      }
    }
  }
  __syncthreads();

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
#pragma unroll
  for (int ks = 0; ks < kC / 32; ++ks) {
    const Frag pa = col8(sPhi, 32 * ks, w);          // Phi^T rows 16w + r16
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      acc[ct] = mma(acc[ct], pa, col8(sdHh, 32 * ks, ct));
      acc[ct] = mma(acc[ct], pa, col8(sdHl, 32 * ks, ct));
    }
    Frag bh, bl;                                     // column 64: lane r16 = 0
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 32 * ks + 8 * g + e;
      bh[e] = r16 == 0 ? sdH64h[t] : from_f32<In>(0.f);
      bl[e] = r16 == 0 ? sdH64l[t] : from_f32<In>(0.f);
    }
    acc[4] = mma(acc[4], pa, bh);
    acc[4] = mma(acc[4], pa, bl);
  }
  float* out = Dr + ((int64_t)b * nc + c) * (kR * kP);
#pragma unroll
  for (int ct = 0; ct < 5; ++ct) {
    const int col = 16 * ct + r16;
    if (col < kP) {
#pragma unroll
      for (int e = 0; e < 4; ++e) out[(16 * w + 4 * g + e) * kP + col] = acc[ct][e];
    }
  }
}

}  // namespace smat

extern "C" int smat_chunk_backward(int dtype, int out_dtype, const void* phi, const void* psi,
                                   const void* vb, const float* dH, const float* Sin,
                                   const float* Q, void* dPhi, void* dPsi, void* dVb, int nb,
                                   int nc, int r, int p, int C,
                                   int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                                   int64_t v_sb, int64_t v_st, int64_t h_sb, int64_t h_st,
                                   int64_t d_sb, int64_t d_st, int64_t e_sb, int64_t e_st,
                                   const float* add_phi, const float* add_psi,
                                   const float* add_vb, int64_t ap_sb, int64_t ap_st,
                                   int64_t ak_sb, int64_t ak_st, int64_t av_sb, int64_t av_st,
                                   int64_t add_split, int64_t add_end, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && dH && Sin && Q && dPhi && dPsi && dVb, SMAT_EINVAL,
               "smat_chunk_backward: null pointer");
  SMAT_REQUIRE(nb >= 0 && nc >= 0, SMAT_EINVAL, "smat_chunk_backward: bad sizes");
  SMAT_REQUIRE(nc < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_chunk_backward: grid %d x %d too large", nc, nb);
  SMAT_REQUIRE(chunk_bwd_ok(dtype, out_dtype, phi, psi, r, p, C, q_sb, q_st, k_sb, k_st, d_sb,
                            d_st, dPhi, dPsi),
               SMAT_EUNSUPPORTED,
               "smat_chunk_backward: needs 16-bit inputs, fp32 or input-typed gradients, r=64, "
               "p=65, C=128 and 16-byte aligned rows of Phi, Psi, dPhi and dPsi (got dtype=%d "
               "out_dtype=%d r=%d p=%d C=%d)",
               dtype, out_dtype, r, p, C);
  SMAT_REQUIRE(v_st >= p && h_st >= p && e_st >= p && d_st >= r, SMAT_EINVAL,
               "smat_chunk_backward: row stride too short");
  SMAT_REQUIRE(0 <= add_split && add_split <= add_end && add_end <= (int64_t)nc * C &&
                   (!add_phi || (rows_vec_ok(add_phi, ap_sb, ap_st, 4) && ap_st >= r)) &&
                   (!add_psi || (rows_vec_ok(add_psi, ak_sb, ak_st, 4) && ak_st >= r)) &&
                   (!add_vb || av_st >= p),
               SMAT_EINVAL,
               "smat_chunk_backward: added terms need 0 <= add_split <= add_end <= nc*C, "
               "16-byte aligned rows for Phi and Psi and full rows");
  if (nb == 0 || nc == 0) return SMAT_OK;
  SMAT_REQUIRE(aligned16(Sin) && aligned16(Q), SMAT_EINVAL,
               "smat_chunk_backward: Sin and Q must be 16-byte aligned");
  // dH: the chunk's 128 rows of 65 floats are one 16-byte aligned block
  const int vec_dh = h_st == p && h_sb % 4 == 0 && aligned16(dH);
  // Vb: nine 16-byte pieces a row stay inside the row's stride
  const int vec_vb = v_st >= 72 && v_st % 8 == 0 && v_sb % 8 == 0 && aligned16(vb);
  ChunkBwdArgs a{nc,    vec_dh, vec_vb, q_sb,  q_st,    k_sb,    k_st,   v_sb,  v_st,
                 h_sb,  h_st,   d_sb,   d_st,  e_sb,    e_st,    add_phi, add_psi, add_vb,
                 ap_sb, ap_st,  ak_sb,  ak_st, av_sb,   av_st,   add_split, add_end};
  const dim3 grid((unsigned)nc, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  const bool f32 = out_dtype == SMAT_F32;
  if (dtype == SMAT_BF16)
    (f32 ? chunk_bwd_launch<bf16, float> : chunk_bwd_launch<bf16, bf16>)(
        phi, psi, vb, dH, Sin, Q, dPhi, dPsi, dVb, a, grid, st);
  else
    (f32 ? chunk_bwd_launch<f16, float> : chunk_bwd_launch<f16, f16>)(
        phi, psi, vb, dH, Sin, Q, dPhi, dPsi, dVb, a, grid, st);
  return launch_status("smat_chunk_backward");
}

extern "C" int smat_chunk_dstates(int dtype, const void* phi, const float* dH, float* Dr, int nb,
                                  int nc, int r, int p, int C, int64_t q_sb, int64_t q_st,
                                  int64_t h_sb, int64_t h_st, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && dH && Dr, SMAT_EINVAL, "smat_chunk_dstates: null pointer");
  SMAT_REQUIRE(nb >= 0 && nc >= 0, SMAT_EINVAL, "smat_chunk_dstates: bad sizes");
  SMAT_REQUIRE(nc < 65536 * 32 && nb < 65536, SMAT_EUNSUPPORTED,
               "smat_chunk_dstates: grid %d x %d too large", nc, nb);
  SMAT_REQUIRE((dtype == SMAT_BF16 || dtype == SMAT_F16) && r == cb::kR && p == cb::kP &&
                   C == cb::kC && rows_vec_ok(phi, q_sb, q_st, 2) && h_st >= p && aligned16(Dr),
               SMAT_EUNSUPPORTED,
               "smat_chunk_dstates: needs 16-bit Phi with 16-byte aligned rows, r=64, p=65, "
               "C=128 (got dtype=%d r=%d p=%d C=%d)",
               dtype, r, p, C);
  if (nb == 0 || nc == 0) return SMAT_OK;
  const int vec_dh = h_st == p && h_sb % 4 == 0 && aligned16(dH);
  const dim3 grid((unsigned)nc, (unsigned)nb);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == SMAT_BF16)
    hipLaunchKernelGGL(chunk_dstate_kernel<bf16>, grid, dim3(cds::kThreads), 0, st,
                       (const bf16*)phi, dH, Dr, nc, vec_dh, q_sb, q_st, h_sb, h_st);
  else
    hipLaunchKernelGGL(chunk_dstate_kernel<f16>, grid, dim3(cds::kThreads), 0, st,
                       (const f16*)phi, dH, Dr, nc, vec_dh, q_sb, q_st, h_sb, h_st);
  return launch_status("smat_chunk_dstates");
}
