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
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(1024), smem, stream, F, F_glob, code, q,
                     U, N0, B, rp, nslices, total, per_xcd);
  return launch_status("smat_incidence_plane");
}

// ---------------------------------------------------------------------------
// Wave-per-direction kernel (d = 3): persistent, one line group per wave
// ---------------------------------------------------------------------------

// ds_read_b128 serves a 32-lane half of a wave at the full rate when both of its
// sixteen-lane rows read sixteen consecutive 16-byte units that start at the
// same offset modulo 16 units; rows that start at different offsets take about
// twice as long.  The plane kernel above hands its rows to different lines, so
// most of its reads are of the slow kind.  Here a wave owns sixteen
// consecutive lines b0 .. b0+15 of ONE direction m, and its four rows are the
// four 16-byte planes of those lines (E = 16 floats): at step t every row reads
// entries kCW*t + s_t + j, j = lane & 15, with one s_t = (b0 - m t) mod q for
// the whole wave.  Columns are kCW = 56 entries apart (>= q + 15: the first 15
// points of a column are stored again after its end, so the sixteen entries
// never wrap).  Lane l of every row holds the offset of step c0 + l of the
// current run of sixteen steps, and a step takes it with a DPP row broadcast
// folded into the address add: one vector instruction besides the four sums.
// Lines b >= q of the last group of a direction read in bounds and are not
// stored.  Vertical lines (e = 0, the column x1 = b) read entry kCW*b + t + j
// from lane j: lanes are kCW + 1 entries apart, an odd stride, so sixteen
// distinct phases, and the steps are immediate offsets.
//
// The panel (4 planes x kCW*q entries, 147 KB at q = 41) leaves no room for a
// second one, so the workgroup is persistent and prefetches the next item's
// panel into registers while it sums the current one: HBM latency stays off
// the critical path without a second LDS buffer.
namespace iw {
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kE = 16;            // floats of r*p per item (four planes)
constexpr int kPlanes = kE / 4;
constexpr int kPF = 7;            // panel chunks each thread prefetches (N0 <= 1792)
constexpr int kU = 8;             // steps issued together
constexpr int kGroup = 16;        // lines per wave task
constexpr int kCW = 56;           // entries per column: >= q + 15, even (see below)
}  // namespace iw

// Lane n of each sixteen-lane row of v, broadcast to the whole row (DPP row_newbcast).
template <int N>
__device__ __forceinline__ int row_bcast(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x150 + N, 0xf, 0xf, false);
}

// Eight steps of a sloped line: step H + n reads the byte offset that lane H + n
// of the row holds in otab.  The eight reads are issued together and waited for
// once.
template <int H>
__device__ __forceinline__ void wave_steps8(float4& acc, const char* vb, int otab) {
  float4 v[8];
  v[0] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 0>(otab));
  v[1] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 1>(otab));
  v[2] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 2>(otab));
  v[3] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 3>(otab));
  v[4] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 4>(otab));
  v[5] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 5>(otab));
  v[6] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 6>(otab));
  v[7] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 7>(otab));
  __builtin_amdgcn_s_waitcnt(0xC07F);                // lgkmcnt(0): one wait for the eight
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < 8; ++u) add4(acc, v[u]);
}

// Sixteen steps of a sloped line with the reads pipelined: four are in flight
// while the previous four are summed (same registers as wave_steps8).
template <int H>
__device__ __forceinline__ void wave_read4(float4* v, const char* vb, int otab) {
  v[0] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 0>(otab));
  v[1] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 1>(otab));
  v[2] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 2>(otab));
  v[3] = *reinterpret_cast<const float4*>(vb + row_bcast<H + 3>(otab));
}
__device__ __forceinline__ void wave_add4(float4& acc, const float4* v) {
  add4(acc, v[0]);
  add4(acc, v[1]);
  add4(acc, v[2]);
  add4(acc, v[3]);
}
__device__ __forceinline__ void wave_steps16(float4& acc, const char* vb, int otab) {
  float4 a[4], b[4];
  wave_read4<0>(a, vb, otab);
  wave_read4<4>(b, vb, otab);
  __builtin_amdgcn_s_waitcnt(0xC47F);                // lgkmcnt(4): a has landed
  __builtin_amdgcn_sched_barrier(0);
  wave_add4(acc, a);
  __builtin_amdgcn_sched_barrier(0);
  wave_read4<8>(a, vb, otab);
  __builtin_amdgcn_s_waitcnt(0xC47F);
  __builtin_amdgcn_sched_barrier(0);
  wave_add4(acc, b);
  __builtin_amdgcn_sched_barrier(0);
  wave_read4<12>(b, vb, otab);
  __builtin_amdgcn_s_waitcnt(0xC47F);
  __builtin_amdgcn_sched_barrier(0);
  wave_add4(acc, a);
  __builtin_amdgcn_s_waitcnt(0xC07F);                // lgkmcnt(0)
  __builtin_amdgcn_sched_barrier(0);
  wave_add4(acc, b);
}

// The steps H .. cnt-1 (cnt - H < 8) of a partial block.
template <int H>
__device__ __forceinline__ void wave_steps_tail(float4& acc, const char* vb, int otab, int cnt) {
#define SMAT_TAIL_STEP(n) \
  if (H + n < cnt) add4(acc, *reinterpret_cast<const float4*>(vb + row_bcast<H + n>(otab)));
  SMAT_TAIL_STEP(0) SMAT_TAIL_STEP(1) SMAT_TAIL_STEP(2) SMAT_TAIL_STEP(3)
  SMAT_TAIL_STEP(4) SMAT_TAIL_STEP(5) SMAT_TAIL_STEP(6)
#undef SMAT_TAIL_STEP
}

static int64_t wave_plane_entries(int q) {
  return ((int64_t)iw::kCW * q + 15) / 16 * 16;
}
static int64_t wave_lds_bytes(int q) {
  return iw::kPlanes * wave_plane_entries(q) * 16 + (((int64_t)q * (q + 1) * 2 + 15) & ~15);
}

template <bool HasG>
__global__ __launch_bounds__(iw::kThreads, 1) void incidence_wave_kernel(
    const float* __restrict__ F, const float* __restrict__ Fg, const int* __restrict__ code,
    int q, float* __restrict__ U, int N0, int B, int64_t rp, int nslices, int64_t total,
    int64_t per_xcd, int plane) {
  using namespace iw;
  extern __shared__ float4 smem[];
  const int W = q + 15;
  const int nlines = q * (q + 1);
  short* line_type = reinterpret_cast<short*>(smem + (size_t)kPlanes * plane);
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

  // Panel chunk u of this thread: point x = idx >> 2, plane k = idx & 3, stored
  // at entry W*x1 + x0 of plane k and again every q entries up to W.
  // Chunk u of this thread: plane kx = row of the lane, and slot
  // ps = 16 * (wave + 16 u) + (lane & 15) in column-major point order
  // (x1 = ps / q, x0 = ps mod q), so the sixteen lanes of a row write sixteen
  // consecutive LDS entries of one plane.  Its F offset (N0 * rp < 2^31,
  // checked on the host) is x*rp + 4*kx for the point x = x0*q + x1; its LDS
  // entry and the number of copies (entries x0, x0 + q, ... < W) are packed as
  // entry | copies << 24.
  const int kx = (tid >> 4) & 3;
  int dst[kPF], src[kPF];
#pragma unroll
  for (int u = 0; u < kPF; ++u) {
    const int ps = 16 * ((tid >> 6) + kWaves * u) + (tid & 15);
    const int x1 = ps / q, x0 = ps - x1 * q;
    const int ncopy = ps < N0 ? (W - x0 + q - 1) / q : 0;
    dst[u] = (kx * plane + kCW * x1 + x0) | (ncopy << 24);
    src[u] = (x0 * q + x1) * (int)rp + 4 * kx;
  }
  float4 pf[kPF];
  auto prefetch = [&](int64_t item) {
    const int64_t b = item / nslices;
    const int64_t e0 = (item - b * nslices) * kE;
    const float* Fb = F + b * (int64_t)N0 * rp + e0;
    const bool in = e0 + 4 * kx < rp;
#pragma unroll
    for (int u = 0; u < kPF; ++u)
      pf[u] = ((dst[u] >> 24) > 0 && in) ? *reinterpret_cast<const float4*>(Fb + src[u])
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  prefetch(first);

  const int j = lane & 15, kpl = lane >> 4;
  const float inv_q = 1.0f / (float)q;
  const int P = (q + kGroup - 1) / kGroup;           // groups per direction
  const int G = (q + 1) * P;
  const int dir0 = wv / P, part0 = wv - dir0 * P;
  const int ddir = kWaves / P, dpart = kWaves - ddir * P;
  const char* pbase = reinterpret_cast<const char*>(smem) + (size_t)kpl * plane * 16;

  for (int64_t item = first; item < end; item += nk) {
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      const int e = dst[u] & 0xffffff, nc = dst[u] >> 24;
      for (int c = 0; c < nc; ++c) smem[e + c * q] = pf[u];
    }
    lds_barrier();                                   // panel (and line table) complete
    const int64_t b = item / nslices;
    const int64_t e0 = (item - b * nslices) * kE;
    const bool live = e0 + 4 * kpl < rp;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
    if (HasG && live) g = *reinterpret_cast<const float4*>(Fg + b * rp + e0 + 4 * kpl);
    if (item + nk < end) prefetch(item + nk);        // lands while this item is summed
    float* Ub = U + b * (int64_t)B * rp + e0 + 4 * kpl;

    // group grp = wv + kWaves*i is part `part` of direction `dir`; both are
    // advanced without a division (kWaves = P*ddir + dpart)
    int dir = dir0, part = part0;
    for (int grp = wv; grp < G; grp += kWaves) {
      const int b0 = part * kGroup;
      const int bl = b0 + j;
      const bool valid = bl < q;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      int lc;
      if (dir < q) {
        // Step t reads entry kCW*t + s_t + j, s_t = (b0 + (q - m) t) mod q.  Lane l
        // of every row holds the byte offset of step c0 + l of the current run of
        // sixteen steps; each step broadcasts its lane within the row (DPP) into
        // the address add, so a step costs one vector add besides the sums.
        const int m = dir;
        lc = (m + 1) * q + bl;
        const char* vb = pbase + 16 * j;
        // lane j: s = s_{c0+j}, advanced by d16 = -16m mod q per run
        const int v = b0 + (q - m) * j;              // < 2^24: exact in float
        int sj = v - q * (int)((float)v * inv_q);
        sj += sj < 0 ? q : 0;
        sj -= sj >= q ? q : 0;
        const unsigned d16 = (unsigned)((16 * (q - m)) % q);
        int colpart = 16 * kCW * j;
        for (int c0 = 0; c0 < q; c0 += 16) {
          const int otab = colpart + 16 * sj;
          if (c0 + 16 <= q) {
            wave_steps16(acc, vb, otab);
          } else if (c0 + 8 <= q) {
            wave_steps8<0>(acc, vb, otab);
            if (c0 + 8 < q) wave_steps_tail<8>(acc, vb, otab, q - c0);
          } else {
            wave_steps_tail<0>(acc, vb, otab, q - c0);
          }
          const unsigned c = (unsigned)sj + d16;
          sj = (int)min(c, c - (unsigned)q);
          colpart += 16 * 16 * kCW;
        }
      } else {
        lc = bl;
        const int col = valid ? bl : (bl >= kGroup ? bl - kGroup : 0);
        const char* vb = pbase + 16 * (kCW * col + j);
        int t = 0;
        for (; t + kU <= q; t += kU) {
          float4 v[kU];
#pragma unroll
          for (int u = 0; u < kU; ++u) v[u] = *reinterpret_cast<const float4*>(vb + 16 * (t + u));
          __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < kU; ++u) add4(acc, v[u]);
        }
        for (; t < q; ++t) add4(acc, *reinterpret_cast<const float4*>(vb + 16 * t));
      }
      const int h = valid ? line_type[lc] : -1;
      if (h >= 0 && live) {
        if (HasG) add4(acc, g);
        *reinterpret_cast<float4*>(Ub + (int64_t)h * rp) = acc;
      }
      part += dpart;
      dir += ddir;
      if (part >= P) {
        part -= P;
        ++dir;
      }
    }
    lds_barrier();                                   // every wave is done with the panel
  }
}

static bool wave_kernel_fits(int q, int N0, int64_t rp) {
  return q + 15 <= iw::kCW && (int64_t)N0 * 4 <= (int64_t)iw::kPF * iw::kThreads &&
         (int64_t)N0 * rp < (1ll << 31) &&
         wave_lds_bytes(q) <= inc::kPlaneLdsBudget && q >= 2 && q * (q + 1) < 32768;
}

static int launch_wave(const float* F, const float* F_glob, const int* code, int q, float* U,
                       int nb, int N0, int B, int64_t rp, hipStream_t stream) {
  using namespace iw;
  const int nslices = (int)((rp + kE - 1) / kE);
  const int64_t total = (int64_t)nb * nslices;
  int dev = 0, ncu = 256;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t per_xcd = (total + inc::kXCD - 1) / inc::kXCD;
  const int64_t per_xcd_wgs = std::max<int64_t>(1, std::min<int64_t>(ncu / inc::kXCD, per_xcd));
  const unsigned grid = (unsigned)(per_xcd_wgs * inc::kXCD);
  const int plane = (int)wave_plane_entries(q);
  const size_t smem = (size_t)wave_lds_bytes(q);
  static bool attr_set[2] = {false, false};
  auto kern = F_glob ? incidence_wave_kernel<true> : incidence_wave_kernel<false>;
  if (!attr_set[F_glob ? 1 : 0]) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                              inc::kPlaneLdsBudget);
    attr_set[F_glob ? 1 : 0] = true;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), smem, stream, F, F_glob, code, q, U, N0,
                     B, rp, nslices, total, per_xcd, plane);
  return launch_status("smat_incidence_plane");
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
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kThreads), smem, stream, F, F_glob,
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
  hipLaunchKernelGGL((incidence_l2_kernel<IDX, VEC>), dim3((unsigned)grid), dim3(kThreads), 0, \
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

int incidence_plane_dispatch(const float* F, const float* F_glob, const int* code, int q,
                             float* U, int nb, int N0, int B, int64_t rp, hipStream_t stream) {
  if (nb == 0 || B == 0 || rp == 0) return SMAT_OK;
  const bool aligned = (rp % 4 == 0) && aligned16(F) && aligned16(U) &&
                       (!F_glob || aligned16(F_glob));
  if (!aligned || (int64_t)q * q != N0 || q > 181) {
    set_error("smat_incidence_plane: needs rp %% 4 == 0, aligned tables and N0 = q^2 "
              "(q=%d N0=%d rp=%lld)", q, N0, (long long)rp);
    return SMAT_EUNSUPPORTED;
  }
  if (wave_kernel_fits(q, N0, rp) && variant(SMAT_VARIANT_INCIDENCE_PLANE) == 0)
    return launch_wave(F, F_glob, code, q, U, nb, N0, B, rp, stream);
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
  return incidence_plane_dispatch(F, F_glob, code, q, U, nb, N0, B, rp, (hipStream_t)stream);
}
