// Incidence  U_h = sum_{x in H_h} F_x  -- the application of C
// (src/smat/attention.py:239-285; the Triton kernel it replaces is
// src/smat/kernels/triton_fwd.py:162-216).
//
// A gather-reduce over fp32 rows of rp = r*p floats.  Each point lies on D
// hyperplanes (D = q+1 for d = 3), so the adds read nnz(C)*rp floats while
// only N0*rp distinct ones exist; the kernels are built around where those
// re-reads are served from.
//
// incidence_lds_kernel (the default): one workgroup per (batch, slice of E
//   floats).  The N0 x E panel of F is staged once in LDS (E = 16: 108 KB at
//   N0 = 1681), then every hyperplane of the batch is summed out of LDS by four
//   lanes.  F crosses HBM once; the re-reads hit LDS, whose bandwidth is twice
//   the vector L1's.
// incidence_l2_kernel (fallback: panels too large for LDS, rp % 4 != 0): one
//   wave per (hyperplane, 256-float slice), the panel re-read from L2.  Flat
//   ids are remapped so each XCD (workgroup L runs on XCD L mod 8) walks a
//   contiguous run of (batch, slice) groups and the panel stays in that XCD's
//   L2; each lane keeps 8 loads in flight.
//
// Both sum a hyperplane's points in the order of the table they are given.
//
// For d = 3 (N0 = q^2, hyperplanes are the q(q+1) lines of the plane over F_q)
// the lines are generated from their codes and no point table is read:
// incidence_wave_kernel (prime q <= 41: four 16-byte planes an item, a line
//   group per pair of sixteen-lane rows, two planes a lane),
// incidence_row_kernel (prime 43 <= q <= 83: one plane an item, a line group
//   per row), and incidence_plane_kernel (any other q: a line per lane).
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "smat_host.hpp"

namespace smat {

namespace inc {
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSlice = 256;               // L2 kernel: floats per wave per hyperplane
constexpr int kPlanesPerWave = 2;
constexpr int kPlanesPerWG = kWaves * kPlanesPerWave;
constexpr int kXCD = 8;
constexpr int kUnroll = 8;                // loads in flight per lane (L2 kernel)
constexpr int kLdsBudget = 150 * 1024;    // bytes of LDS for the F panel
constexpr int kPlaneLdsBudget = 160 * 1024;   // the plane kernel's panel + line table
}  // namespace inc

__device__ __forceinline__ void add4(float4& a, const float4& v) {
  a.x += v.x;
  a.y += v.y;
  a.z += v.z;
  a.w += v.w;
}

// ---------------------------------------------------------------------------
// LDS panel kernel
// ---------------------------------------------------------------------------

// Four consecutive lanes own one hyperplane, lane k of the four the floats
// [4k, 4k+4) of the 16-float slice, so eight lanes (one 128-byte LDS cycle)
// read the 64-byte rows of two points.  Rows are 64 B apart, so the two reads
// are conflict-free exactly when the two points differ in parity; tables
// prepared by the host (parity_interleaved_table in attention.py) order each
// hyperplane's points even-first or odd-first, alternating between
// hyperplanes, which makes that the common case.  Any table is accepted.
template <typename Idx, int E, int DMAX>
__global__ __launch_bounds__(inc::kThreads) void incidence_lds_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const Idx* __restrict__ idx,
    const int64_t* __restrict__ indptr, int deg, float* __restrict__ U, int N0, int B, int64_t rp,
    int nslices, int64_t total, int64_t per_xcd) {
  using namespace inc;
  constexpr int Q = E / 4;          // float4 per point (= lanes per hyperplane)
  constexpr int kLines = kThreads / Q;
  extern __shared__ float4 panel[];

  const int64_t L = blockIdx.x;
  const int64_t work = (L % kXCD) * per_xcd + L / kXCD;
  if (work >= total) return;
  const int64_t b = work / nslices;
  const int slice = (int)(work - b * nslices);
  const int64_t e0 = (int64_t)slice * E;

  const float* Fb = F + b * (int64_t)N0 * rp + e0;
  for (int i = threadIdx.x; i < N0 * Q; i += kThreads) {
    const int x = i / Q, k = i - x * Q;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + 4 * k < rp) v = *reinterpret_cast<const float4*>(Fb + (int64_t)x * rp + 4 * k);
    panel[i] = v;
  }

  const int k = threadIdx.x % Q;                  // float4 of the slice
  const bool live = e0 + 4 * k < rp;
  float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
  if (Fg && live) g = *reinterpret_cast<const float4*>(Fg + b * rp + e0 + 4 * k);
  float* Ub = U + b * (int64_t)B * rp + e0 + 4 * k;

  if (indptr == nullptr && deg <= DMAX) {
    // Uniform degree: a hyperplane's whole index row is loaded into registers
    // in one burst, and the next hyperplane's row while this one is summed,
    // so index latency overlaps the LDS work.
    int cur[DMAX], nxt[DMAX];
    int h = threadIdx.x / Q;
#pragma unroll
    for (int u = 0; u < DMAX; ++u)
      cur[u] = (h < B && u < deg) ? (int)idx[(int64_t)h * deg + u] : 0;
    __syncthreads();                              // panel staged
    for (; h < B; h += kLines) {
      const int hn = h + kLines;
#pragma unroll
      for (int u = 0; u < DMAX; ++u)
        nxt[u] = (hn < B && u < deg) ? (int)idx[(int64_t)hn * deg + u] : 0;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < DMAX; ++u)
        if (u < deg) add4(acc, panel[cur[u] * Q + k]);
      if (live) {
        if (Fg) add4(acc, g);
        *reinterpret_cast<float4*>(Ub + (int64_t)h * rp) = acc;
      }
#pragma unroll
      for (int u = 0; u < DMAX; ++u) cur[u] = nxt[u];
    }
    return;
  }
  __syncthreads();                                // panel staged
  for (int h = threadIdx.x / Q; h < B; h += kLines) {
    int64_t lo, hi;
    if (indptr) {
      lo = indptr[h];
      hi = indptr[h + 1];
    } else {
      lo = (int64_t)h * deg;
      hi = lo + deg;
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int64_t t = lo;
    for (; t + 8 <= hi; t += 8) {
      int x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = (int)idx[t + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) add4(acc, panel[x[u] * Q + k]);
    }
    for (; t < hi; ++t) add4(acc, panel[(int)idx[t] * Q + k]);
    if (live) {
      if (Fg) add4(acc, g);
      *reinterpret_cast<float4*>(Ub + (int64_t)h * rp) = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// LDS panel kernel, lines of the affine plane (d = 3) generated in-kernel
// ---------------------------------------------------------------------------

// For d = 3 every row type is a line <a_e, x> = b of F_q^2 (a_0 = (0, 1),
// a_e = (1, e-1) for e >= 1), point x = x0*q + x1.  Its q points follow from
// the line code e*q + b, so no index table is read: a line with e >= 1 has one
// point in each column x1 (x0 = b - m*x1 mod q, m = e-1), the line e = 0 is
// the column x1 = b.
//
// The N0 x E slice of F is staged in LDS column by column: entry W*x1 + i holds
// point (i mod q, x1) for i in [0, W), W = q + 15, so each column's first 15
// points appear twice.  The E floats of an entry are split into Q = E/4
// 16-byte chunks kept in Q separate planes of PLANE entries (chunk k of entry P
// at float4 index k*PLANE + P), so a lane's Q reads of one entry share one
// address and differ by an immediate offset.  Sixteen consecutive lanes own
// the lines b0 .. b0+15 of one direction.  At step x1 = t they need
// x0 = s + j (mod q), j = 0..15, s = b0 - m*t mod q: the entries W*t + s + j,
// sixteen CONSECUTIVE entries (the duplicates absorb the wrap), i.e. 256
// contiguous bytes of a plane: one ds_read_b128 of sixteen lanes touches each
// of the 64 banks once.  Lines e = 0 walk their column from a lane-dependent
// start, entry W*b + j + t, so neighbouring lanes are W + 1 entries apart --
// an odd stride for odd q, again sixteen distinct bank groups.  Points are
// summed in x1 order (e >= 1) or from the lane's start around the column
// (e = 0).
template <int E, int PLANE, int MINB>
__global__ __launch_bounds__(1024, MINB) void incidence_plane_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const int* __restrict__ code,
    int q, float* __restrict__ U, int N0, int B, int64_t rp, int nslices, int64_t total,
    int64_t per_xcd) {
  using namespace inc;
  constexpr int kT = 1024;
  constexpr int Q = E / 4;          // 16-byte chunks per entry = planes
  constexpr int kU = 4;             // steps in flight per lane
  extern __shared__ float4 smem[];
  const int W = q + 15;
  const int nlines = q * (q + 1);
  float4* panel = smem;
  short* line_type = reinterpret_cast<short*>(smem + (size_t)Q * PLANE);

  const int64_t L = blockIdx.x;
  const int64_t work = (L % kXCD) * per_xcd + L / kXCD;
  if (work >= total) return;
  const int64_t b = work / nslices;
  const int slice = (int)(work - b * nslices);
  const int64_t e0 = (int64_t)slice * E;

  // line code -> row type (the inverse of code[])
  for (int c = threadIdx.x; c < nlines; c += kT) line_type[c] = -1;
  const float* Fb = F + b * (int64_t)N0 * rp + e0;
  for (int idx = threadIdx.x; idx < N0 * Q; idx += kT) {
    const int x = idx / Q, k = idx - x * Q;
    const int x0 = x / q, x1 = x - x0 * q;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + 4 * k < rp) v = *reinterpret_cast<const float4*>(Fb + (int64_t)x * rp + 4 * k);
    for (int i = x0; i < W; i += q) panel[k * PLANE + W * x1 + i] = v;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < B; h += kT) {
    const int c = code[h];
    if (c >= 0 && c < nlines) line_type[c] = (short)h;
  }
  __syncthreads();

  float* Ub = U + b * (int64_t)B * rp + e0;
  const float* Fgb = Fg ? Fg + b * rp + e0 : nullptr;
  // Lane L owns line (e, b) = divmod(L, q): no idle lanes.  Within a run of
  // consecutive b of one direction the entries read at a step are consecutive
  // (mod q); a run that wraps, or a sixteen-lane group that straddles two
  // directions, costs a two-way bank conflict at worst.
  const int nlines_all = q * (q + 1);
  for (int L = threadIdx.x; L < nlines_all; L += kT) {
    const int e = L / q;
    const int bl = L - e * q;
    // e >= 1: entry W*t + (b - m t mod q).  e = 0 (the column x1 = b): entry
    // W*b + (b + t mod q), i.e. m = q - 1 = -1 mod q and no column stride,
    // so neighbouring lanes are W + 1 entries apart (odd): distinct banks.
    const int m = e == 0 ? q - 1 : e - 1;
    const int stride = e == 0 ? 0 : W;
    int pt = e == 0 ? W * bl : 0;                // entry of step t, less s
    int s = bl;
    float4 acc[Q];
#pragma unroll
    for (int k = 0; k < Q; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    int t = 0;
    for (; t + kU <= q; t += kU) {
      const float4* row[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        row[u] = panel + pt + s;
        pt += stride;
        s -= m;
        s += s < 0 ? q : 0;
      }
      float4 v[kU][Q];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int k = 0; k < Q; ++k) v[u][k] = row[u][k * PLANE];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int k = 0; k < Q; ++k) add4(acc[k], v[u][k]);
    }
    for (; t < q; ++t) {
      const float4* row = panel + pt + s;
      pt += stride;
      s -= m;
      s += s < 0 ? q : 0;
#pragma unroll
      for (int k = 0; k < Q; ++k) add4(acc[k], row[k * PLANE]);
    }
    {
      const int h = line_type[e * q + bl];
      if (h >= 0) {
#pragma unroll
        for (int k = 0; k < Q; ++k) {
          if (e0 + 4 * k < rp) {
            if (Fgb) add4(acc[k], *reinterpret_cast<const float4*>(Fgb + 4 * k));
            *reinterpret_cast<float4*>(Ub + (int64_t)h * rp + 4 * k) = acc[k];
          }
        }
      }
    }
  }
}

// LDS bytes of the plane kernel: Q planes of PLANE entries and the line table.
static int64_t plane_lds_bytes(int q, int E, int plane) {
  (void)E;
  return (int64_t)(E / 4) * plane * 16 + (((int64_t)q * (q + 1) * 2 + 15) & ~(int64_t)15);
}

template <int E, int PLANE, int MINB>
static int launch_plane(const float* F, const float* F_glob, const int* code, int q, float* U,
                        int nb, int N0, int B, int64_t rp, hipStream_t stream) {
  using namespace inc;
  const int nslices = (int)((rp + E - 1) / E);
  const int64_t total = (int64_t)nb * nslices;
  const int64_t per_xcd = (total + kXCD - 1) / kXCD;
  const int64_t grid = per_xcd * kXCD;
  const size_t smem = (size_t)plane_lds_bytes(q, E, PLANE);
  auto kern = incidence_plane_kernel<E, PLANE, MINB>;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              kPlaneLdsBudget);
    attr_set = true;
  }
  smat::launch(kern, dim3((unsigned)grid), dim3(1024), smem, stream, F, F_glob, code, q,
                     U, N0, B, rp, nslices, total, per_xcd);
  return launch_status("smat_incidence_plane");
}

// ---------------------------------------------------------------------------
// Line-group kernel (d = 3): persistent, two line groups per wave
// ---------------------------------------------------------------------------

// An item is one sequence's N0 x 16 slice of F (floats [e0, e0 + 16) of every
// r*p row).  It sits in LDS as four planes of 16-byte entries (floats
// [e0 + 4k, e0 + 4k + 4) in plane k), column by column: entry kCW*x1 + i of a
// plane holds point (i mod q, x1) for i < q + 15, so the first 15 points of a
// column appear again after its end and no run of sixteen consecutive entries
// wraps.  The planes are kPlane entries apart, a multiple of sixteen, so the
// same entry of two planes sits at the same bank phase.
//
// A sixteen-lane row owns sixteen consecutive lines b0 .. b0+15 of one
// direction (a group) and one plane pair: rows 0 and 1 of a wave take group A
// with planes (0, 1) and (2, 3), rows 2 and 3 group B, so the two rows of each
// 32-lane half read the same entries of two planes -- the pattern ds_read_b128
// serves at its full rate.  Lane j of a row reads, at step t,
//   sloped line (m, b), points (b - m t mod q, t):  entry kCW*t + s_t + j,
//       s_t = (b0 - m t) mod q, one value per row: sixteen consecutive entries,
//       256 contiguous bytes, every bank once;
//   vertical line b (the column x1 = b):  entry kCW*b + j + t, the column
//       summed from a lane-dependent start; lanes kCW + 1 entries apart, an
//       odd stride, so sixteen distinct 16-byte phases.
// Either address is a lane part plus a row part.  Lane l of each row holds the
// row part of step 16*run + l in ot[run], and a step broadcasts it within the
// row (DPP) into the address add: one vector instruction, then two 16-byte
// reads (the second plane of the pair is an immediate offset of the first) and
// eight adds.  Steps are issued two at a time with three pairs in flight.
// Lanes past q in a direction's last group read in bounds and store nothing.
//
// The panel (4 x kPlane entries, 147 KB) leaves no room for a second one, so
// the workgroup is persistent and prefetches the next item's panel into
// registers while it sums the current one.  Nothing in the summing loop may
// wait on the vector memory counter, which counts those loads too: the kernel
// fits 128 VGPRs without spilling (a spill reload waits for every load issued
// before it), the chunk map is recomputed per item rather than kept live.
namespace iw {
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kE = 16;            // floats of r*p per item (four planes)
constexpr int kPlanes = kE / 4;
constexpr int kPF = 7;            // panel chunks each thread prefetches (N0 <= 1792)
constexpr int kGroup = 16;        // lines per row
constexpr int kCW = 56;           // entries per column: >= q + 15
constexpr int kQMax = kCW - 15;   // largest q the layout holds
constexpr int kPlane = (kCW * kQMax + 15) / 16 * 16;   // 2304 entries
constexpr int kPlaneBytes = kPlane * 16;               // 36864: fits the 16-bit offset
}  // namespace iw

// Lane n of each sixteen-lane row of v, broadcast to the whole row (DPP row_newbcast).
template <int N>
__device__ __forceinline__ int row_bcast(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x150 + N, 0xf, 0xf, false);
}

// x = (x_lo, y_lo), y = (x_hi, y_hi) over the 32-lane halves of the wave
// (v_permlane32_swap).
__device__ __forceinline__ void swap_halves(float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false,
                                                  false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap_halves(int& x, int& y) {
  const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)y, false, false);
  x = (int)r[0];
  y = (int)r[1];
}

// Step N: both planes of the pair at the lane part plus the row part of step N.
template <int N>
__device__ __forceinline__ void lg_issue(float4* v, const char* vb, const int* ot) {
  const char* a = vb + row_bcast<N % 16>(ot[N / 16]);
  v[0] = *reinterpret_cast<const float4*>(a);
  v[1] = *reinterpret_cast<const float4*>(a + iw::kPlaneBytes);
}

// Pair K of steps (2K, 2K + 1), into buffer K mod 3.
template <int Q, int K>
__device__ __forceinline__ void lg_issue_pair(float4 (&buf)[3][4], const char* vb, const int* ot) {
  if constexpr (2 * K < Q) lg_issue<2 * K>(&buf[K % 3][0], vb, ot);
  if constexpr (2 * K + 1 < Q) lg_issue<2 * K + 1>(&buf[K % 3][2], vb, ot);
}

// The sums so far are materialised here and no memory access moves across:
// without it the compiler sinks every add below every read, and the Q pairs of
// reads in flight spill.
__device__ __forceinline__ void lg_fence(float4& a0, float4& a1) {
  asm volatile("" : "+v"(a0.x), "+v"(a0.y), "+v"(a0.z), "+v"(a0.w), "+v"(a1.x), "+v"(a1.y),
               "+v"(a1.z), "+v"(a1.w)::"memory");
}

// Sum pair K (the compiler waits for its reads only), then issue pair K + 3
// into the registers it frees; steps are summed in order 0 .. Q-1.
template <int Q, int K>
__device__ __forceinline__ void lg_pipe(float4& a0, float4& a1, float4 (&buf)[3][4],
                                        const char* vb, const int* ot) {
  if constexpr (2 * K < Q) {
    if constexpr (K == 0) {
      a0 = buf[0][0];
      a1 = buf[0][1];
    } else {
      add4(a0, buf[K % 3][0]);
      add4(a1, buf[K % 3][1]);
    }
    if constexpr (2 * K + 1 < Q) {
      add4(a0, buf[K % 3][2]);
      add4(a1, buf[K % 3][3]);
    }
    lg_fence(a0, a1);
    __builtin_amdgcn_sched_barrier(0);
    lg_issue_pair<Q, K + 3>(buf, vb, ot);
    __builtin_amdgcn_sched_barrier(0);
    lg_pipe<Q, K + 1>(a0, a1, buf, vb, ot);
  }
}

// a0, a1 = the sums of a line's Q points in the two planes of the pair.
template <int Q>
__device__ __forceinline__ void lg_line_sums(float4& a0, float4& a1, const char* vb,
                                             const int* ot) {
  float4 buf[3][4];
  lg_issue_pair<Q, 0>(buf, vb, ot);
  lg_issue_pair<Q, 1>(buf, vb, ot);
  lg_issue_pair<Q, 2>(buf, vb, ot);
  __builtin_amdgcn_sched_barrier(0);
  lg_pipe<Q, 0>(a0, a1, buf, vb, ot);
}

// x / Q and x mod Q for x below Max by a multiply and a shift: M and S are the
// smallest pair with floor(x M / 2^S) = floor(x / Q) over that range (where
// x M stays below 2^24, v_mul_u32_u24 forms it; otherwise a 32-bit multiply).
template <int Q, int Max>
struct LgDiv {
  static constexpr bool exact(unsigned M, int S) {
    for (unsigned x = 0; x < (unsigned)Max; ++x)
      if ((x * M) >> S != x / Q) return false;
    return true;
  }
  static constexpr int shift() {
    int S = 1;
    while (!exact(((1u << S) + Q - 1) / Q, S)) ++S;
    return S;
  }
  static constexpr int S = shift();
  static constexpr unsigned M = ((1u << S) + Q - 1) / Q;
  static constexpr bool k24 = (unsigned long long)Max * M < (1ull << 24);
  static_assert((unsigned long long)Max * M < (1ull << 32), "32-bit product");
  __device__ __forceinline__ static unsigned div(unsigned x) {
    return (k24 ? __umul24(x, M) : x * M) >> S;
  }
  __device__ __forceinline__ static unsigned mod(unsigned x) { return x - Q * div(x); }
};
// b0 + (Q - m) j of a group's lane: below 16 P + 16 Q.
template <int Q>
using LgMod = LgDiv<Q, 16 * ((Q + 15) / 16) + 16 * Q>;

// One group of the item: sixteen consecutive lines b0 .. b0+15 of direction
// dir (dir < Q sloped with slope m = dir, dir = Q vertical; groups past the
// last are dead and store nothing).  Lane j's row part at step t is built from
// s_t = (s0 + qm t) mod Q with s0 = b0 for a sloped group (s_t = b0 - m t) and
// s0 = qm = 0 for a vertical one; s advances by d16 over sixteen steps.  lcb + j
// is lane j's line code (e*q + b).  PD groups a direction: all q lines by
// default; q / 16 leaves each direction's last q mod 16 lines to the caller.
template <int Q, int PD = (Q + 15) / 16>
struct LgGroup {
  static constexpr int P = PD;
  static constexpr int G = (Q + 1) * P;
  int b0, s0, qm, d16, lcb, nvalid, sloped;
  __device__ __forceinline__ explicit LgGroup(int g) {
    const int dir = g / P;
    b0 = (g - dir * P) * 16;
    sloped = dir < Q;
    s0 = sloped ? b0 : 0;
    qm = sloped ? Q - dir : 0;
    d16 = (16 * qm) % Q;
    lcb = sloped ? (dir + 1) * Q + b0 : b0;
    nvalid = g < G ? min(16, Q - b0) : 0;
  }
  // Hide how the (scalar) fields were derived, so a per-lane choice between
  // two groups selects the values instead of recomputing them per lane.
  __device__ __forceinline__ void opaque() {
    b0 = __builtin_amdgcn_readfirstlane(b0);
    s0 = __builtin_amdgcn_readfirstlane(s0);
    qm = __builtin_amdgcn_readfirstlane(qm);
    d16 = __builtin_amdgcn_readfirstlane(d16);
    lcb = __builtin_amdgcn_readfirstlane(lcb);
    nvalid = __builtin_amdgcn_readfirstlane(nvalid);
    sloped = __builtin_amdgcn_readfirstlane(sloped);
  }
};

// Panel chunk u of thread tid: plane kx = (tid >> 4) & 3 and slot
// ps = 16 * (wave + 16 u) + (tid & 15) in column-major point order
// (x1 = ps / q, x0 = ps mod q), so the sixteen lanes of a row write sixteen
// consecutive entries of one plane.  Its F offset in bytes (4 N0 rp < 2^32,
// checked on the host) is 4 (x*rp + 4*kx) for the point x = x0*q + x1; its LDS
// entry is kx*kPlane + kCW*x1 + x0, with copies at + q, + 2q, ... below q + 15.
template <int Q>
using LgSlot = LgDiv<Q, 16 * iw::kWaves * iw::kPF>;

// Byte offsets into one sequence's F panel rows and U type rows are 32-bit;
// ld is their row stride in floats.
static bool wave_kernel_fits(int q, int N0, int B, int64_t ld) {
  return q >= 2 && q <= iw::kQMax && N0 == q * q &&
         (int64_t)N0 * iw::kPlanes <= (int64_t)iw::kPF * iw::kThreads &&
         (int64_t)N0 * ld < (1ll << 30) && (int64_t)B * ld < (1ll << 30);
}

static int64_t wave_lds_bytes(int q) {
  return (int64_t)iw::kPlanes * iw::kPlane * 16 + (((int64_t)q * (q + 1) * 2 + 15) & ~15);
}

// A line of its own per lane (the last q mod 16 lines of each direction, when
// fewer than ten): at step N the entry c1 N + s_N (kCW entries a column), s
// advancing by qm modulo m -- sloped lines c1 = kCW, s_0 = b, qm = q - slope,
// m = q (x1 = N, x0 = b - slope N mod q); vertical ones c1 = 1, s_0 = kCW b,
// qm = 0 and an m no sum reaches (the column x1 = b from x0 = 0).  All in
// bytes (times 16).  Four address instructions a step against a group's one,
// for lanes that would otherwise idle in a direction's last group.
struct LrLane {
  uint32_t s16, qm16, m16, c16;
};

// The line-group kernel's lines of their own take all four planes: two
// addresses a step (planes 2 and 3 lie past the 16-bit read offset), four
// 16-byte reads and sixteen adds; two steps in flight.
typedef __attribute__((address_space(3))) const float lds_cfloat;
typedef float lds_f4v __attribute__((ext_vector_type(4)));
// 16 bytes at LDS address addr (16-byte aligned: one ds_read_b128)
__device__ __forceinline__ float4 lds_at(uint32_t addr) {
  const lds_f4v v = *(__attribute__((address_space(3))) const lds_f4v*)(size_t)addr;
  return make_float4(v.x, v.y, v.z, v.w);
}
// pb: the panel's LDS address
template <int N>
__device__ __forceinline__ void lw_issue(float4 (&v)[4], uint32_t pb, LrLane& ln) {
  const uint32_t a = pb + __umul24(ln.c16, (uint32_t)N) + ln.s16;
  // planes 2 and 3 from a second base: opaque, so plane 3 stays an immediate
  // offset from it rather than a third address
  uint32_t a2 = a + 2 * iw::kPlaneBytes;
  asm volatile("" : "+v"(a2));
  v[0] = lds_at(a);
  v[1] = lds_at(a + iw::kPlaneBytes);
  v[2] = lds_at(a2);
  v[3] = lds_at(a2 + iw::kPlaneBytes);
  const uint32_t c = ln.s16 + ln.qm16;
  ln.s16 = min(c, c - ln.m16);
}

__device__ __forceinline__ void lw_fence(float4 (&a)[4]) {
  asm volatile("" : "+v"(a[0].x), "+v"(a[0].y), "+v"(a[0].z), "+v"(a[0].w), "+v"(a[1].x),
               "+v"(a[1].y), "+v"(a[1].z), "+v"(a[1].w)::"memory");
  asm volatile("" : "+v"(a[2].x), "+v"(a[2].y), "+v"(a[2].z), "+v"(a[2].w), "+v"(a[3].x),
               "+v"(a[3].y), "+v"(a[3].z), "+v"(a[3].w)::"memory");
}

// Sum step N (in order 0 .. Q-1), then issue step N + 1 into its registers.
template <int Q, int N>
__device__ __forceinline__ void lw_pipe(float4 (&a)[4], float4 (&buf)[4], uint32_t pb,
                                        LrLane& ln) {
  if constexpr (N < Q) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (N == 0)
        a[p] = buf[p];
      else
        add4(a[p], buf[p]);
    }
    lw_fence(a);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (N + 1 < Q) lw_issue<N + 1>(buf, pb, ln);
    __builtin_amdgcn_sched_barrier(0);
    lw_pipe<Q, N + 1>(a, buf, pb, ln);
  }
}

template <int Q>
__device__ __forceinline__ void lw_line_sums(float4 (&a)[4], uint32_t pb, LrLane ln) {
  float4 buf[4];
  lw_issue<0>(buf, pb, ln);
  __builtin_amdgcn_sched_barrier(0);
  lw_pipe<Q, 0>(a, buf, pb, ln);
}

// The lane state of line li of the lines of their own: R of them a direction,
// after the P full groups' 16 P lines.  Lanes past NOL walk column 0 and store
// nothing.
template <int Q, int P, int R, int NOL, int kCW>
__device__ __forceinline__ LrLane own_lane(int li, int& code) {
  const bool valid = li < NOL;
  const int dir = valid ? li / R : 0;
  const int bl = 16 * P + (valid ? li - dir * R : 0);
  const bool sl = dir < Q;
  LrLane ln;
  ln.s16 = 16u * (uint32_t)(sl ? bl : kCW * bl);
  ln.qm16 = sl ? 16u * (uint32_t)(Q - dir) : 0u;
  ln.m16 = sl ? 16u * (uint32_t)Q : 0x80000000u;
  ln.c16 = 16u * (uint32_t)(sl ? kCW : 1);
  code = valid ? (sl ? (dir + 1) * Q + bl : bl) : -1;
  return ln;
}

template <int Q, bool HasG>
__global__ __launch_bounds__(iw::kThreads, 1) void incidence_wave_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const int* __restrict__ code,
    float* __restrict__ U, int B, int64_t rp, int64_t ld, int nslices, int64_t total,
    int64_t per_xcd) {
  using namespace iw;
  constexpr int q = Q;
  constexpr int N0 = Q * Q;
  constexpr int nlines = Q * (Q + 1);
  // Past 16 lines a direction, fewer than ten lines after its last full group
  // go to lanes of their own (LrLane, all four planes) rather than a group
  // with idle lanes; those tasks all fall in one slot k = kOwnK of every wave.
  constexpr int R = Q % kGroup;
  constexpr bool kOwn = Q > kGroup && R > 0 && R < 10;
  constexpr int P = kOwn ? Q / kGroup : (Q + kGroup - 1) / kGroup;   // groups per direction
  constexpr int G = (Q + 1) * P;                     // groups per item
  constexpr int NTG = (G + 1) / 2;                   // group tasks (two groups) per item
  constexpr int NOL = kOwn ? (Q + 1) * R : 0;        // lines of their own
  constexpr int NT = NTG + (NOL + 63) / 64;          // wave tasks per item
  constexpr int kOwnK = NTG / kWaves;
  static_assert(!kOwn || (NT - 1) / kWaves == kOwnK, "lines of their own in one task slot");
  constexpr int NR = (Q + 15) / 16;                  // runs of sixteen steps
  extern __shared__ float4 smem[];
  short* line_type = reinterpret_cast<short*>(smem + (size_t)kPlanes * kPlane);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());

  const int xcd = blockIdx.x % inc::kXCD;
  const int64_t nk = gridDim.x / inc::kXCD;
  const int64_t first = (int64_t)xcd * per_xcd + blockIdx.x / inc::kXCD;
  const int64_t end = min<int64_t>(total, (int64_t)(xcd + 1) * per_xcd);
  if (first >= end) return;

  for (int c = tid; c < nlines; c += kThreads) line_type[c] = -1;
  __syncthreads();
  for (int h = tid; h < B; h += kThreads) {
    const int c = code[h];
    if (c >= 0 && c < nlines) line_type[c] = (short)h;
  }

  // The chunk map of this thread (LgSlot) is recomputed on every item rather
  // than kept live: ps0 passes through an empty asm so it is not hoisted.
  const uint32_t ps0 = 16u * (uint32_t)(tid >> 6) + (uint32_t)(tid & 15);
  const int kx = (tid >> 4) & 3;
  const uint32_t ld4 = (uint32_t)ld * 4u;   // bytes from one F or U row to the next
  float4 pf[kPF];
  uint32_t src[kPF];
  auto chunk_src = [&](uint32_t ps) {
    const uint32_t x1 = LgSlot<Q>::div(ps), x0 = ps - Q * x1;
    return __umul24(x0 * Q + x1, ld4) + 16u * kx;   // 4 (x ld + 4 kx)
  };
  auto prefetch = [&](int64_t item) {
    const int64_t bi = item / nslices;
    const int64_t e0 = (item - bi * nslices) * kE;
    const char* Fb = reinterpret_cast<const char*>(F + bi * (int64_t)N0 * ld + e0);
    const bool in = e0 + 4 * kx < rp;
#pragma unroll
    for (int u = 0; u < kPF; ++u)
      pf[u] = (ps0 + 256u * u < (uint32_t)N0 && in)
                  ? *reinterpret_cast<const float4*>(Fb + src[u])
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  };
#pragma unroll
  for (int u = 0; u < kPF; ++u) src[u] = chunk_src(ps0 + 256u * u);
  prefetch(first);

  // Row roles: group A or B of the wave's task, plane pair (0, 1) or (2, 3).
  const int j = lane & 15;
  const int gsel = lane >> 5;
  const int pp = (lane >> 4) & 1;
  const int splane = (pp << 1) | gsel;               // plane this lane stores (after swap_halves)
  const char* pbase = reinterpret_cast<const char*>(smem) + (size_t)(2 * pp) * kPlaneBytes;
  const int lane16 = 16 * j, laneCW16 = 16 * kCW * j;
  const uint32_t splane16 = 16u * splane;

  // The lane state of each of the wave's tasks is the same for every item, so
  // it is worked out once: tasks wv, wv + 16, ... (kTasks at most); for each,
  // the lane part of the read address, the row parts ot[] of the q steps, and
  // the byte offsets in an item's U rows of the two lines this lane stores
  // after the half exchange (kNoLine: none).
  constexpr int kTasks = (NT + kWaves - 1) / kWaves;
  constexpr uint32_t kNoLine = ~0u;
  int tvb[kTasks], tot[kTasks][NR];
  uint32_t tsA[kTasks], tsB[kTasks];
  lds_barrier();                                     // line table complete
#pragma unroll
  for (int k = 0; k < kTasks; ++k) {
    const int task = wv + kWaves * k;                // past NT: dead, never summed
    if (kOwn && k == kOwnK && task >= NTG) {
      // a line of its own: s_0 in tvb, qm in tot[0] (c1 and m follow from
      // qm, zero only for vertical lines), its U row's byte offset in tsA
      int lc;
      const LrLane ln = own_lane<Q, P, R, NOL, kCW>(64 * (task - NTG) + lane, lc);
      const int h = lc >= 0 ? line_type[lc] : -1;
      tvb[k] = (int)ln.s16;
      tot[k][0] = (int)ln.qm16;
      tsA[k] = h >= 0 ? (uint32_t)h * ld4 : kNoLine;
      continue;
    }
    // The task's groups 2 task (rows 0-1) and 2 task + 1 (rows 2-3) are
    // worked out on the scalar unit; each lane then takes its own.
    LgGroup<Q, P> gA(2 * task), gB(2 * task + 1);
    gA.opaque();                                     // select the values, not their
    gB.opaque();                                     // derivation, per lane
    const int b0 = gsel ? gB.b0 : gA.b0;
    const int s0 = gsel ? gB.s0 : gA.s0;
    const int qm = gsel ? gB.qm : gA.qm;
    const int d16 = gsel ? gB.d16 : gA.d16;
    const int lcb = gsel ? gB.lcb : gA.lcb;
    const int nvalid = gsel ? gB.nvalid : gA.nvalid;
    const bool sloped = (gsel ? gB.sloped : gA.sloped) != 0;
    const bool valid = j < nvalid;
    // sloped: lane part 16 j; row part of step t = 16 (kCW t + s_t),
    //   s_t = (b0 - m t) mod q = (b0 + qm t) mod q, taken by lane l for
    //   t = 16 run + l.
    // vertical (and the dead group of an odd G, s0 = qm = 0): lane part
    //   16 (kCW col + j), row part of step t = 16 t, col clamped into the
    //   columns for lanes past q.
    const int bl = b0 + j;
    const int col = valid ? bl : (bl >= kGroup ? bl - kGroup : 0);
    tvb[k] = lane16 + (sloped ? 0 : (int)__umul24(16 * kCW, col));
    {
      int s = (int)LgMod<Q>::mod((unsigned)s0 + __umul24(qm, j));
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        tot[k][r] = (sloped ? 256 * kCW * r + laneCW16 : 256 * r + lane16) + 16 * s;
        const unsigned c = (unsigned)(s + d16);
        s = (int)min(c, c - (unsigned)q);
      }
    }
    int hA = valid ? line_type[min(lcb + j, nlines - 1)] : -1, hB = hA;
    swap_halves(hA, hB);                             // the lines stored after the exchange
    // a lane stores at byte h * 4 ld + 16 splane of its type row h (below 2^32:
    // checked on the host)
    tsA[k] = hA >= 0 ? (uint32_t)hA * ld4 + splane16 : kNoLine;
    tsB[k] = hB >= 0 ? (uint32_t)hB * ld4 + splane16 : kNoLine;
  }

  for (int64_t item = first; item < end; item += nk) {
    {
      uint32_t p0 = ps0;
      asm volatile("" : "+v"(p0));
#pragma unroll
      for (int u = 0; u < kPF; ++u) {
        const uint32_t ps = p0 + 256u * u;
        const uint32_t x1 = LgSlot<Q>::div(ps), x0 = ps - Q * x1;
        if (ps < (uint32_t)N0) {
          float4* e = smem + (kx * kPlane + kCW * x1 + x0);
#pragma unroll
          for (int c = 0; c < (Q + 15 + Q - 1) / Q; ++c)
            if (x0 + c * Q < (uint32_t)(Q + 15)) e[c * Q] = pf[u];
        }
        src[u] = __umul24(x0 * Q + x1, ld4) + 16u * kx;
      }
    }
    lds_barrier();                                   // panel (and line table) complete
    const int64_t b = item / nslices;
    const int64_t e0 = (item - b * nslices) * kE;
    if (item + nk < end) prefetch(item + nk);        // lands while this item is summed
    const bool live = e0 + 4 * splane < rp;          // rp % 4 == 0: whole planes
    // The U rows of this item start at Ubase; a lane stores at byte
    // h * 4 ld + 16 splane of its type row h (below 2^32: checked on the host).
    const char* Ubase = reinterpret_cast<const char*>(U + b * (int64_t)B * ld + e0);

#pragma unroll
    for (int k = 0; k < kTasks; ++k) {
      if (wv + kWaves * k >= NT) continue;
      if (kOwn && k == kOwnK && wv + kWaves * k >= NTG) {
        // s_0 passes through an empty asm each item: the walk depends on no
        // load, and hoisted out of the item loop its q addresses would all
        // stay live (and spill)
        LrLane ln;
        ln.s16 = (uint32_t)tvb[k];
        ln.qm16 = (uint32_t)tot[k][0];
        asm volatile("" : "+v"(ln.s16), "+v"(ln.qm16));
        ln.m16 = ln.qm16 ? 16u * Q : 0x80000000u;
        ln.c16 = ln.qm16 ? 16u * kCW : 16u;
        float4 a[4];
        lw_line_sums<Q>(a, (uint32_t)(size_t)(lds_cfloat*)(smem), ln);
        if (tsA[k] != kNoLine) {
          char* urow = const_cast<char*>(Ubase) + tsA[k];
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            if (e0 + 4 * p < rp) {                   // rp % 4 == 0: whole planes
              if (HasG) add4(a[p], *reinterpret_cast<const float4*>(Fg + b * rp + e0 + 4 * p));
              *reinterpret_cast<float4*>(urow + 16 * p) = a[p];
            }
          }
        }
        continue;
      }
      float4 a0, a1;
      lg_line_sums<Q>(a0, a1, pbase + tvb[k], tot[k]);
      // Rows 0-3 hold planes (0, 1) and (2, 3) of group A, then of group B, in
      // (a0, a1).  One exchange of 32-lane halves leaves group A's four planes in
      // a0 and group B's in a1 (rows 0-3: planes 0, 2, 1, 3), so each store
      // writes a line's 64 bytes from four lanes of one instruction.
      swap_halves(a0.x, a1.x);
      swap_halves(a0.y, a1.y);
      swap_halves(a0.z, a1.z);
      swap_halves(a0.w, a1.w);
      if (live) {
        if (HasG) {
          const float4 g = *reinterpret_cast<const float4*>(Fg + b * rp + e0 + 4 * splane);
          add4(a0, g);
          add4(a1, g);
        }
        if (tsA[k] != kNoLine) *reinterpret_cast<float4*>(const_cast<char*>(Ubase) + tsA[k]) = a0;
        if (tsB[k] != kNoLine) *reinterpret_cast<float4*>(const_cast<char*>(Ubase) + tsB[k]) = a1;
      }
    }
    lds_barrier();                                   // every wave is done with the panel
  }
}

template <int Q>
static int launch_wave_q(const float* F, const float* F_glob, const int* code, float* U, int nb,
                         int B, int64_t rp, int64_t ld, hipStream_t stream) {
  using namespace iw;
  const int nslices = (int)((rp + kE - 1) / kE);
  const int64_t total = (int64_t)nb * nslices;
  int dev = 0, ncu = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t per_xcd = (total + inc::kXCD - 1) / inc::kXCD;
  const int64_t per_xcd_wgs = std::max<int64_t>(1, std::min<int64_t>(ncu / inc::kXCD, per_xcd));
  const unsigned grid = (unsigned)(per_xcd_wgs * inc::kXCD);
  const size_t smem = (size_t)wave_lds_bytes(Q);
  static bool attr_set[2] = {false, false};
  auto kern = F_glob ? incidence_wave_kernel<Q, true> : incidence_wave_kernel<Q, false>;
  if (!attr_set[F_glob ? 1 : 0]) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              inc::kPlaneLdsBudget);
    attr_set[F_glob ? 1 : 0] = true;
  }
  smat::launch(kern, dim3(grid), dim3(kThreads), smem, stream, F, F_glob, code, U, B, rp, ld,
                     nslices, total, per_xcd);
  return launch_status("smat_incidence_plane");
}

// The line-group kernel is compiled for the prime field sizes it holds
// (q <= 41); returns SMAT_EUNSUPPORTED for any other q.
static int launch_wave(const float* F, const float* F_glob, const int* code, int q, float* U,
                       int nb, int N0, int B, int64_t rp, int64_t ld, hipStream_t stream) {
  (void)N0;
  switch (q) {
#define SMAT_WAVE_Q(QV) \
  case QV:              \
    return launch_wave_q<QV>(F, F_glob, code, U, nb, B, rp, ld, stream);
    SMAT_WAVE_Q(2) SMAT_WAVE_Q(3) SMAT_WAVE_Q(5) SMAT_WAVE_Q(7) SMAT_WAVE_Q(11)
    SMAT_WAVE_Q(13) SMAT_WAVE_Q(17) SMAT_WAVE_Q(19) SMAT_WAVE_Q(23) SMAT_WAVE_Q(29)
    SMAT_WAVE_Q(31) SMAT_WAVE_Q(37) SMAT_WAVE_Q(41)
#undef SMAT_WAVE_Q
    default:
      return SMAT_EUNSUPPORTED;
  }
}

static bool wave_kernel_has_q(int q) {
  switch (q) {
    case 2: case 3: case 5: case 7: case 11: case 13: case 17: case 19: case 23: case 29:
    case 31: case 37: case 41:
      return true;
    default:
      return false;
  }
}

// ---------------------------------------------------------------------------
// Row-group kernel (d = 3, larger q): one line group per row, one plane a lane
// ---------------------------------------------------------------------------

// For 43 <= q <= 83 four 16-byte planes of the N0 points no longer fit in LDS
// beside their column copies, so an item is one sequence's N0 x 4-float slice
// of F: one plane, stored as in the line-group kernel (entry kCW*x1 + i holds
// point (i mod q, x1) for i < q + 15, kCW = q + 15 rounded up to even).  Each
// sixteen-lane row of a wave owns its own group of sixteen consecutive lines
// of one direction and reads, at step t, the same entries as a line-group row
// (sloped: kCW*t + s_t + j; vertical: kCW*b + j + t), one 16-byte read and
// four adds a step after the DPP-broadcast address add.  The four rows of a
// wave are four consecutive groups: the two rows of a half-wave read the same
// bank phase except at a step whose offsets wrap past q (ds_read_b128 serves
// rows at different phases at about half its full rate).
namespace ir {
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kE = 4;             // floats of r*p per item (one plane)
constexpr int kPF = 7;            // panel chunks each thread prefetches (N0 <= 7168)
constexpr int kQMin = 43, kQMax = 83;
template <int Q>
struct Shape {
  static constexpr int kCW = (Q + 15 + 1) / 2 * 2;              // even: vertical stride odd
  static constexpr int kEntries = (kCW * Q + 15) / 16 * 16;
  static constexpr int kLdsBytes = kEntries * 16 + ((Q * (Q + 1) * 2 + 15) / 16) * 16;
  static_assert(kLdsBytes <= 160 * 1024, "panel and line table fit the LDS");
};
}  // namespace ir

// Step N: one plane at the lane part plus the row part of step N.
template <int N>
__device__ __forceinline__ void lr_issue(float4& v, const char* vb, const int* ot) {
  v = *reinterpret_cast<const float4*>(vb + row_bcast<N % 16>(ot[N / 16]));
}

// Batch K of steps 4K .. 4K+3, into buffer K mod 3.
template <int Q, int K>
__device__ __forceinline__ void lr_issue_batch(float4 (&buf)[3][4], const char* vb, const int* ot) {
  if constexpr (4 * K < Q) lr_issue<4 * K>(buf[K % 3][0], vb, ot);
  if constexpr (4 * K + 1 < Q) lr_issue<4 * K + 1>(buf[K % 3][1], vb, ot);
  if constexpr (4 * K + 2 < Q) lr_issue<4 * K + 2>(buf[K % 3][2], vb, ot);
  if constexpr (4 * K + 3 < Q) lr_issue<4 * K + 3>(buf[K % 3][3], vb, ot);
}

__device__ __forceinline__ void lr_fence(float4& a) {
  asm volatile("" : "+v"(a.x), "+v"(a.y), "+v"(a.z), "+v"(a.w)::"memory");
}

// Sum batch K (steps in order 0 .. Q-1), then issue batch K + 3 into its registers.
template <int Q, int K>
__device__ __forceinline__ void lr_pipe(float4& a, float4 (&buf)[3][4], const char* vb,
                                        const int* ot) {
  if constexpr (4 * K < Q) {
    if constexpr (K == 0)
      a = buf[0][0];
    else
      add4(a, buf[K % 3][0]);
    if constexpr (4 * K + 1 < Q) add4(a, buf[K % 3][1]);
    if constexpr (4 * K + 2 < Q) add4(a, buf[K % 3][2]);
    if constexpr (4 * K + 3 < Q) add4(a, buf[K % 3][3]);
    lr_fence(a);
    __builtin_amdgcn_sched_barrier(0);
    lr_issue_batch<Q, K + 3>(buf, vb, ot);
    __builtin_amdgcn_sched_barrier(0);
    lr_pipe<Q, K + 1>(a, buf, vb, ot);
  }
}

template <int Q>
__device__ __forceinline__ float4 lr_line_sum(const char* vb, const int* ot) {
  float4 buf[3][4];
  float4 a;
  lr_issue_batch<Q, 0>(buf, vb, ot);
  lr_issue_batch<Q, 1>(buf, vb, ot);
  lr_issue_batch<Q, 2>(buf, vb, ot);
  __builtin_amdgcn_sched_barrier(0);
  lr_pipe<Q, 0>(a, buf, vb, ot);
  return a;
}

// The row-group kernel's lines of their own (LrLane), one plane a lane.

template <int N>
__device__ __forceinline__ void lo_issue(float4& v, const char* pb, LrLane& ln) {
  v = *reinterpret_cast<const float4*>(pb + (__umul24(ln.c16, (uint32_t)N) + ln.s16));
  const uint32_t c = ln.s16 + ln.qm16;
  ln.s16 = min(c, c - ln.m16);
}

template <int Q, int K>
__device__ __forceinline__ void lo_issue_batch(float4 (&buf)[3][4], const char* pb, LrLane& ln) {
  if constexpr (4 * K < Q) lo_issue<4 * K>(buf[K % 3][0], pb, ln);
  if constexpr (4 * K + 1 < Q) lo_issue<4 * K + 1>(buf[K % 3][1], pb, ln);
  if constexpr (4 * K + 2 < Q) lo_issue<4 * K + 2>(buf[K % 3][2], pb, ln);
  if constexpr (4 * K + 3 < Q) lo_issue<4 * K + 3>(buf[K % 3][3], pb, ln);
}

template <int Q, int K>
__device__ __forceinline__ void lo_pipe(float4& a, float4 (&buf)[3][4], const char* pb,
                                        LrLane& ln) {
  if constexpr (4 * K < Q) {
    if constexpr (K == 0)
      a = buf[0][0];
    else
      add4(a, buf[K % 3][0]);
    if constexpr (4 * K + 1 < Q) add4(a, buf[K % 3][1]);
    if constexpr (4 * K + 2 < Q) add4(a, buf[K % 3][2]);
    if constexpr (4 * K + 3 < Q) add4(a, buf[K % 3][3]);
    lr_fence(a);
    __builtin_amdgcn_sched_barrier(0);
    lo_issue_batch<Q, K + 3>(buf, pb, ln);
    __builtin_amdgcn_sched_barrier(0);
    lo_pipe<Q, K + 1>(a, buf, pb, ln);
  }
}

template <int Q>
__device__ __forceinline__ float4 lo_line_sum(const char* pb, LrLane ln) {
  float4 buf[3][4];
  float4 a;
  lo_issue_batch<Q, 0>(buf, pb, ln);
  lo_issue_batch<Q, 1>(buf, pb, ln);
  lo_issue_batch<Q, 2>(buf, pb, ln);
  __builtin_amdgcn_sched_barrier(0);
  lo_pipe<Q, 0>(a, buf, pb, ln);
  return a;
}

// Slot ps of the panel: ps = 64 * (wave + 16 u) + lane, x1 = ps / q, x0 = ps mod q.
template <int Q>
using LrSlot = LgDiv<Q, 64 * ir::kWaves * ir::kPF>;

static bool row_kernel_fits(int q, int N0, int B, int64_t ld) {
  return q >= ir::kQMin && q <= ir::kQMax && N0 == q * q &&
         (int64_t)N0 <= (int64_t)ir::kPF * ir::kThreads && (int64_t)N0 * ld < (1ll << 30) &&
         (int64_t)B * ld < (1ll << 30);
}

template <int Q, bool HasG>
__global__ __launch_bounds__(ir::kThreads, 1) void incidence_row_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const int* __restrict__ code,
    float* __restrict__ U, int B, int64_t rp, int64_t ld, int nslices, int64_t total,
    int64_t per_xcd) {
  using namespace ir;
  typedef Shape<Q> Sh;
  constexpr int q = Q;
  constexpr int N0 = Q * Q;
  constexpr int kCW = Sh::kCW;
  constexpr int nlines = Q * (Q + 1);
  // Fewer than ten lines past a direction's last full group go to lanes of
  // their own (LrLane) rather than a group with idle lanes.
  constexpr int R = Q % 16;
  constexpr bool kOwn = R > 0 && R < 10;
  constexpr int P = kOwn ? Q / 16 : (Q + 15) / 16;   // groups per direction
  constexpr int G = (Q + 1) * P;                     // groups per item
  constexpr int NTG = (G + 3) / 4;                   // group tasks (four groups) per item
  constexpr int NOL = kOwn ? (Q + 1) * R : 0;        // lines of their own
  constexpr int NT = NTG + (NOL + 63) / 64;          // wave tasks per item
  constexpr int NR = (Q + 15) / 16;                  // runs of sixteen steps
  extern __shared__ float4 smem[];
  short* line_type = reinterpret_cast<short*>(smem + Sh::kEntries);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());

  const int xcd = blockIdx.x % inc::kXCD;
  const int64_t nk = gridDim.x / inc::kXCD;
  const int64_t first = (int64_t)xcd * per_xcd + blockIdx.x / inc::kXCD;
  const int64_t end = min<int64_t>(total, (int64_t)(xcd + 1) * per_xcd);
  if (first >= end) return;

  for (int c = tid; c < nlines; c += kThreads) line_type[c] = -1;
  __syncthreads();
  for (int h = tid; h < B; h += kThreads) {
    const int c = code[h];
    if (c >= 0 && c < nlines) line_type[c] = (short)h;
  }

  // Chunk u of this thread: slot ps0 + 1024 u, 16 bytes of one point; the map
  // is recomputed per item (ps0 passes through an empty asm).
  const uint32_t ps0 = (uint32_t)tid;
  const uint32_t ld4 = (uint32_t)ld * 4u;   // bytes from one F or U row to the next
  float4 pf[kPF];
  uint32_t src[kPF];
  auto prefetch = [&](int64_t item) {
    const int64_t b = item / nslices;
    const int64_t e0 = (item - b * nslices) * kE;
    const char* Fb = reinterpret_cast<const char*>(F + b * (int64_t)N0 * ld + e0);
#pragma unroll
    for (int u = 0; u < kPF; ++u)
      pf[u] = ps0 + 1024u * u < (uint32_t)N0 ? *reinterpret_cast<const float4*>(Fb + src[u])
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
  };
#pragma unroll
  for (int u = 0; u < kPF; ++u) {
    const uint32_t ps = ps0 + 1024u * u;
    const uint32_t x1 = LrSlot<Q>::div(ps), x0 = ps - Q * x1;
    src[u] = __umul24(x0 * Q + x1, ld4);             // 4 x ld, x = x0*q + x1
  }
  prefetch(first);

  const int j = lane & 15;
  const int row = lane >> 4;                         // group of the wave's task
  const int lane16 = 16 * j, laneCW16 = 16 * kCW * j;
  const char* pbase = reinterpret_cast<const char*>(smem);

  for (int64_t item = first; item < end; item += nk) {
    {
      uint32_t p0 = ps0;
      asm volatile("" : "+v"(p0));
#pragma unroll
      for (int u = 0; u < kPF; ++u) {
        const uint32_t ps = p0 + 1024u * u;
        const uint32_t x1 = LrSlot<Q>::div(ps), x0 = ps - Q * x1;
        if (ps < (uint32_t)N0) {
          float4* e = smem + (kCW * x1 + x0);
#pragma unroll
          for (int c = 0; c < (Q + 15 + Q - 1) / Q; ++c)
            if (x0 + c * Q < (uint32_t)(Q + 15)) e[c * Q] = pf[u];
        }
        src[u] = __umul24(x0 * Q + x1, ld4);
      }
    }
    lds_barrier();                                   // panel (and line table) complete
    const int64_t b = item / nslices;
    const int64_t e0 = (item - b * nslices) * kE;
    if (item + nk < end) prefetch(item + nk);        // lands while this item is summed
    const bool live = e0 < rp;                       // rp % 4 == 0: whole planes
    const char* Ubase = reinterpret_cast<const char*>(U + b * (int64_t)B * ld + e0);
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
    if (HasG && live) g = *reinterpret_cast<const float4*>(Fg + b * rp + e0);

    for (int task = wv; task < NT; task += kWaves) {
      if (kOwn && task >= NTG) {
        // lines of their own: lane l takes line 64 (task - NTG) + l of the
        // (direction, k) list, line b = 16 P + k of the direction
        int lc;
        const LrLane ln = own_lane<Q, P, R, NOL, kCW>(64 * (task - NTG) + lane, lc);
        float4 a = lo_line_sum<Q>(pbase, ln);
        const int h = lc >= 0 ? line_type[lc] : -1;
        if (live && h >= 0) {
          if (HasG) add4(a, g);
          *reinterpret_cast<float4*>(const_cast<char*>(Ubase) + (uint32_t)h * ld4) = a;
        }
        continue;
      }
      const LgGroup<Q, P> gr(4 * task + row);        // the lane's own group (per row)
      const bool valid = j < gr.nvalid;
      const int bl = gr.b0 + j;
      const int col = valid ? bl : (bl >= 16 ? bl - 16 : 0);
      const char* vb = pbase + lane16 + (gr.sloped ? 0 : (int)__umul24(16 * kCW, col));
      int ot[NR];
      {
        int s = (int)LgMod<Q>::mod((unsigned)gr.s0 + __umul24(gr.qm, j));
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          ot[r] = (gr.sloped ? 256 * kCW * r + laneCW16 : 256 * r + lane16) + 16 * s;
          const unsigned c = (unsigned)(s + gr.d16);
          s = (int)min(c, c - (unsigned)q);
        }
      }
      float4 a = lr_line_sum<Q>(vb, ot);
      const int h = valid ? line_type[min(gr.lcb + j, nlines - 1)] : -1;
      if (live && h >= 0) {
        if (HasG) add4(a, g);
        *reinterpret_cast<float4*>(const_cast<char*>(Ubase) + (uint32_t)h * ld4) = a;
      }
    }
    lds_barrier();                                   // every wave is done with the panel
  }
}

template <int Q>
static int launch_row_q(const float* F, const float* F_glob, const int* code, float* U, int nb,
                        int B, int64_t rp, int64_t ld, hipStream_t stream) {
  using namespace ir;
  const int nslices = (int)((rp + kE - 1) / kE);
  const int64_t total = (int64_t)nb * nslices;
  int dev = 0, ncu = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t per_xcd = (total + inc::kXCD - 1) / inc::kXCD;
  const int64_t per_xcd_wgs = std::max<int64_t>(1, std::min<int64_t>(ncu / inc::kXCD, per_xcd));
  const unsigned grid = (unsigned)(per_xcd_wgs * inc::kXCD);
  const size_t smem = (size_t)Shape<Q>::kLdsBytes;
  static bool attr_set[2] = {false, false};
  auto kern = F_glob ? incidence_row_kernel<Q, true> : incidence_row_kernel<Q, false>;
  if (!attr_set[F_glob ? 1 : 0]) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)smem);
    attr_set[F_glob ? 1 : 0] = true;
  }
  smat::launch(kern, dim3(grid), dim3(kThreads), smem, stream, F, F_glob, code, U, B, rp, ld,
                     nslices, total, per_xcd);
  return launch_status("smat_incidence_plane");
}

// The row-group kernel is compiled for the primes 43 .. 83; returns
// SMAT_EUNSUPPORTED for any other q.
static int launch_row(const float* F, const float* F_glob, const int* code, int q, float* U,
                      int nb, int B, int64_t rp, int64_t ld, hipStream_t stream) {
  switch (q) {
#define SMAT_ROW_Q(QV) \
  case QV:             \
    return launch_row_q<QV>(F, F_glob, code, U, nb, B, rp, ld, stream);
    SMAT_ROW_Q(43) SMAT_ROW_Q(47) SMAT_ROW_Q(53) SMAT_ROW_Q(59) SMAT_ROW_Q(61) SMAT_ROW_Q(67)
    SMAT_ROW_Q(71) SMAT_ROW_Q(73) SMAT_ROW_Q(79) SMAT_ROW_Q(83)
#undef SMAT_ROW_Q
    default:
      return SMAT_EUNSUPPORTED;
  }
}

static bool row_kernel_has_q(int q) {
  switch (q) {
    case 43: case 47: case 53: case 59: case 61: case 67: case 71: case 73: case 79: case 83:
      return true;
    default:
      return false;
  }
}
// ---------------------------------------------------------------------------
// L2 kernel
// ---------------------------------------------------------------------------

template <typename Idx, bool Vec>
__global__ __launch_bounds__(inc::kThreads) void incidence_l2_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const Idx* __restrict__ idx,
    const int64_t* __restrict__ indptr, int deg, float* __restrict__ U, int N0, int B, int64_t rp,
    int nslices, int nhg, int64_t total_wg, int64_t per_xcd) {
  using namespace inc;
  const int64_t L = blockIdx.x;
  const int64_t work = (L % kXCD) * per_xcd + L / kXCD;
  if (work >= total_wg) return;
  const int64_t group = work / nhg;          // (b, slice)
  const int hg = (int)(work - group * nhg);
  const int64_t b = group / nslices;
  const int slice = (int)(group - b * nslices);

  const int lane = lane_id(), w = wave_id();
  const int64_t e0 = (int64_t)slice * kSlice + 4 * lane;
  const float* Fb = F + b * (int64_t)N0 * rp;
  const float* Fgb = Fg ? Fg + b * rp : nullptr;
  float* Ub = U + b * (int64_t)B * rp;

#pragma unroll
  for (int kp = 0; kp < kPlanesPerWave; ++kp) {
    const int h = hg * kPlanesPerWG + w * kPlanesPerWave + kp;
    if (h >= B) continue;
    int64_t lo, hi;
    if (indptr) {
      lo = indptr[h];
      hi = indptr[h + 1];
    } else {
      lo = (int64_t)h * deg;
      hi = lo + deg;
    }
    if (Vec) {
      if (e0 < rp) {   // rp % 4 == 0 on this path, so the 4 floats are in range
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        int64_t t = lo;
        for (; t + kUnroll <= hi; t += kUnroll) {
          float4 v[kUnroll];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u)
            v[u] = *reinterpret_cast<const float4*>(Fb + (int64_t)idx[t + u] * rp + e0);
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) add4(acc, v[u]);
        }
        for (; t < hi; ++t) add4(acc, *reinterpret_cast<const float4*>(Fb + (int64_t)idx[t] * rp + e0));
        if (Fgb) add4(acc, *reinterpret_cast<const float4*>(Fgb + e0));
        *reinterpret_cast<float4*>(Ub + (int64_t)h * rp + e0) = acc;
      }
    } else {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int64_t t = lo; t < hi; ++t) {
        const int64_t x = (int64_t)idx[t];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (e0 + j < rp) acc[j] += Fb[x * rp + e0 + j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (e0 + j < rp) {
          float v = acc[j];
          if (Fgb) v += Fgb[e0 + j];
          Ub[(int64_t)h * rp + e0 + j] = v;
        }
      }
    }
  }
}

// Widest slice whose padded panel fits the LDS budget (0: none fits).
static int lds_slice_width(int N0) {
  for (int E : {16, 8, 4}) {
    const int64_t bytes = (int64_t)N0 * E * 4;
    if (bytes <= inc::kLdsBudget) return E;
  }
  return 0;
}

template <typename Idx, int E, int DMAX>
static int launch_lds(const float* F, const float* F_glob, const void* idx, const int64_t* indptr,
                      int deg, float* U, int nb, int N0, int B, int64_t rp, hipStream_t stream) {
  using namespace inc;
  const int nslices = (int)((rp + E - 1) / E);
  const int64_t total = (int64_t)nb * nslices;
  const int64_t per_xcd = (total + kXCD - 1) / kXCD;
  const int64_t grid = per_xcd * kXCD;
  const size_t smem = (size_t)N0 * E * 4;
  auto kern = incidence_lds_kernel<Idx, E, DMAX>;
  static bool attr_set = false;     // the LDS ceiling is per kernel; raise it once
  if (!attr_set) {
    hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                        inc::kLdsBudget);
    attr_set = true;
  }
  smat::launch(kern, dim3((unsigned)grid), dim3(kThreads), smem, stream, F, F_glob,
                     (const Idx*)idx, indptr, deg, U, N0, B, rp, nslices, total, per_xcd);
  return launch_status("smat_incidence");
}

template <typename Idx, int E>
static int launch_lds_deg(const float* F, const float* F_glob, const void* idx,
                          const int64_t* indptr, int deg, float* U, int nb, int N0, int B,
                          int64_t rp, hipStream_t stream) {
  if (indptr == nullptr && deg <= 32)
    return launch_lds<Idx, E, 32>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream);
  if (indptr == nullptr && deg <= 48)
    return launch_lds<Idx, E, 48>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream);
  return launch_lds<Idx, E, 80>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream);
}

int incidence_dispatch(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                       const int64_t* indptr, int deg, float* U, int nb, int N0, int B, int64_t rp,
                       hipStream_t stream) {
  using namespace inc;
  if (nb == 0 || B == 0 || rp == 0) return SMAT_OK;
  const bool aligned = (rp % 4 == 0) && aligned16(F) && aligned16(U) &&
                       (!F_glob || aligned16(F_glob));
  const int E = lds_slice_width(N0);
  if (aligned && E > 0 && variant(SMAT_VARIANT_INCIDENCE) == 0) {
#define SMAT_LDS(IDX)                                                                       \
  (E == 16 ? launch_lds_deg<IDX, 16>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream) \
   : E == 8 ? launch_lds_deg<IDX, 8>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream) \
            : launch_lds_deg<IDX, 4>(F, F_glob, idx, indptr, deg, U, nb, N0, B, rp, stream))
    return idx_is_64 ? SMAT_LDS(int64_t) : SMAT_LDS(int32_t);
#undef SMAT_LDS
  }
  const int nslices = (int)((rp + kSlice - 1) / kSlice);
  const int nhg = (B + kPlanesPerWG - 1) / kPlanesPerWG;
  const int64_t total = (int64_t)nb * nslices * nhg;
  const int64_t per_xcd = (total + kXCD - 1) / kXCD;
  const int64_t grid = per_xcd * kXCD;
  if (grid >= (1ll << 31)) {
    set_error("smat_incidence: problem too large (%lld workgroups)", (long long)grid);
    return SMAT_EUNSUPPORTED;
  }
#define SMAT_INC_LAUNCH(IDX, VEC)                                                              \
  smat::launch((incidence_l2_kernel<IDX, VEC>), dim3((unsigned)grid), dim3(kThreads), 0, \
                     stream, F, F_glob, (const IDX*)idx, indptr, deg, U, N0, B, rp, nslices,   \
                     nhg, total, per_xcd)
  if (idx_is_64) {
    if (aligned) SMAT_INC_LAUNCH(int64_t, true); else SMAT_INC_LAUNCH(int64_t, false);
  } else {
    if (aligned) SMAT_INC_LAUNCH(int32_t, true); else SMAT_INC_LAUNCH(int32_t, false);
  }
#undef SMAT_INC_LAUNCH
  return launch_status("smat_incidence");
}

// F and U rows of rp floats laid out ld floats apart with ld / 16 odd.  The
// line-group and row-group kernels move each row in 64-byte pieces, and the
// spacing of the pieces sets the rate HBM serves them at: at 8 sequences,
// q = 41, the kernel takes 606-618 us with ld = rp = 16512 (1032 x 16), 545-560
// us with ld = 16528, 16560, 16592, 16624 and 636-641 us with ld a multiple of
// 128 floats (MI355X, measured).
int64_t incidence_spread_ld(int64_t rp) {
  int64_t ld = (rp + 15) / 16 * 16;
  if ((ld / 16) % 2 == 0) ld += 16;
  return ld;
}

static bool plane_groups_run(int q, int N0, int B, int64_t ld) {
  if (variant(SMAT_VARIANT_INCIDENCE_PLANE) != 0) return false;
  return (wave_kernel_fits(q, N0, B, ld) && wave_kernel_has_q(q)) ||
         (row_kernel_fits(q, N0, B, ld) && row_kernel_has_q(q));
}

// The row stride a one-call forward lays F and U out with: the spread stride
// when the line-group or row-group kernel runs the incidence, else rp.
int64_t incidence_plane_ld(int q, int N0, int B, int64_t rp) {
  const int64_t ld = incidence_spread_ld(rp);
  return rp % 4 == 0 && plane_groups_run(q, N0, B, ld) ? ld : rp;
}

// F: (nb, N0) rows and U: (nb, B) rows of rp floats, ld floats apart; ld may
// exceed rp only where the line-group or row-group kernel runs.
int incidence_plane_dispatch(const float* F, const float* F_glob, const int* code, int q,
                             float* U, int nb, int N0, int B, int64_t rp, int64_t ld,
                             hipStream_t stream) {
  if (nb == 0 || B == 0 || rp == 0) return SMAT_OK;
  const bool aligned = (rp % 4 == 0) && (ld % 4 == 0) && aligned16(F) && aligned16(U) &&
                       (!F_glob || aligned16(F_glob));
  if (!aligned || (int64_t)q * q != N0 || q > 181 || ld < rp) {
    set_error("smat_incidence_plane: needs rp %% 4 == 0, ld >= rp, aligned tables and N0 = q^2 "
              "(q=%d N0=%d rp=%lld ld=%lld)", q, N0, (long long)rp, (long long)ld);
    return SMAT_EUNSUPPORTED;
  }
  if (wave_kernel_fits(q, N0, B, ld) && wave_kernel_has_q(q) &&
      variant(SMAT_VARIANT_INCIDENCE_PLANE) == 0)
    return launch_wave(F, F_glob, code, q, U, nb, N0, B, rp, ld, stream);
  if (row_kernel_fits(q, N0, B, ld) && row_kernel_has_q(q) &&
      variant(SMAT_VARIANT_INCIDENCE_PLANE) == 0)
    return launch_row(F, F_glob, code, q, U, nb, B, rp, ld, stream);
  if (ld != rp) {
    set_error("smat_incidence_plane: row stride %lld != %lld needs the line-group or row-group "
              "kernel (q=%d)", (long long)ld, (long long)rp, q);
    return SMAT_EUNSUPPORTED;
  }
  // Two workgroups per CU at E = 8 (one stages its panel while the other sums)
  // measured ahead of one at E = 16; wider panels fall back to one per CU.
  const int64_t entries = (int64_t)q * (q + 15);
  const int64_t budget = inc::kPlaneLdsBudget;
#define SMAT_PLANE_TRY(E_, PL_, MB_)                                                   \
  if (entries <= PL_ && MB_ * plane_lds_bytes(q, E_, PL_) <= budget)                   \
    return launch_plane<E_, PL_, MB_>(F, F_glob, code, q, U, nb, N0, B, rp, stream);
  SMAT_PLANE_TRY(8, 2304, 2)
  SMAT_PLANE_TRY(16, 2304, 1)
  SMAT_PLANE_TRY(8, 4608, 1)
  SMAT_PLANE_TRY(4, 9216, 1)
#undef SMAT_PLANE_TRY
  set_error("smat_incidence_plane: the F panel of q=%d does not fit LDS", q);
  return SMAT_EUNSUPPORTED;
}

}  // namespace smat

extern "C" int smat_incidence(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                              const int64_t* indptr, int deg, float* U, int nb, int N0, int B,
                              int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && idx && U, SMAT_EINVAL, "smat_incidence: null pointer");
  SMAT_REQUIRE(nb >= 0 && N0 >= 1 && B >= 0 && rp >= 0, SMAT_EINVAL, "smat_incidence: bad sizes");
  SMAT_REQUIRE(indptr || deg >= 0, SMAT_EINVAL, "smat_incidence: need indptr or deg >= 0");
  return incidence_dispatch(F, F_glob, idx, idx_is_64, indptr, deg, U, nb, N0, B, rp,
                            (hipStream_t)stream);
}

extern "C" int smat_incidence_plane(const float* F, const float* F_glob, const int* code, int q,
                                    float* U, int nb, int N0, int B, int64_t rp, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(F && code && U, SMAT_EINVAL, "smat_incidence_plane: null pointer");
  SMAT_REQUIRE(nb >= 0 && q >= 2 && B >= 0 && rp >= 0, SMAT_EINVAL,
               "smat_incidence_plane: bad sizes");
  return incidence_plane_dispatch(F, F_glob, code, q, U, nb, N0, B, rp, rp,
                                  (hipStream_t)stream);
}
