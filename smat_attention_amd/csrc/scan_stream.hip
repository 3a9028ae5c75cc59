// The causal pass of the schedule for the common head shape -- 16-bit inputs,
// r = 128 features, p = 129 value columns (head_dim 128 plus the ones column),
// T and n multiples of 64 -- streamed through LDS.  Same contract as the
// normalising mode of scan_fused_kernel (src/smat/attention.py:134-192 and
// :446-453): segmented chunked scan with one reset at n, the long-range term
// Y added to recent rows, division by the normaliser column, optional gate.
//
//   * One workgroup of eight waves walks one group of chunks; the group's
//     incoming state comes from the same prepass (Gram sums per group, shifted
//     exclusive scan over groups) as scan_fused_kernel.
//   * Tokens advance 64 per step.  The Phi, Psi and Vb rows of the next step
//     are copied HBM -> LDS by global_load_lds_dwordx4 while the current step
//     computes: double-buffered, no registers and no VALU spent on staging.
//   * Wave w owns value columns 16w .. 16w+15.  It keeps S[:, cols] (128 x 16,
//     fp32) in MFMA accumulators and produces the transposed output
//         O^T[cols][t] = S^T Phi^T + Vb^T A^T ,
//     because (k-slot bijection) the accumulator tiles of S[a][c], split into
//     hi + lo 16-bit parts, are exactly the A operand of S^T Phi^T -- S never
//     goes through LDS -- and the O^T accumulator layout gives each lane four
//     consecutive columns of one row: 16-byte output stores.
//   * Columns 128..143 (the normaliser column and padding) are a ninth
//     column tile whose state every wave keeps; waves 0..3 each produce the
//     normaliser of one 16-row tile and share it through LDS.
//   * The within-step scores A^T = Psi Phi^T (the causal 16 x 16 tiles of the
//     64 x 64 block) are computed once, split over the waves, masked, rounded
//     to the input dtype as the reference does, and shared through LDS.
//   * Psi and Vb feed the MFMAs along the token axis through the gfx950
//     transposing LDS read ds_read_b64_tr_b16: within each 16-lane group,
//     lane i receives element (i & 3) of the 8 bytes addressed by lane
//     4j + (i >> 2) as its element j.
//
// LDS layout.  The LDS has 64 banks of 4 bytes.  A 16-byte read is served
// in four phases of 16 lanes: lanes 32h + 4j .. 32h + 4j + 3 go in phase
// (h, parity of j) for j = 0..7.  An 8-byte read, transposing or not, is
// served in two phases of 32 consecutive lanes.  A phase is conflict-free
// when its lanes' bytes fall in distinct banks (lanes reading the same
// address share the access).  Phi, Psi and Vb columns 0..127 are tiles of
// 64 rows of 256 bytes (sixteen 16-byte chunks); chunk k of row t is stored
// at slot k ^ swz16(t).  That one XOR satisfies all three reads of a tile: a
// row-wise 16-byte fragment read (16 rows, chunk 4 kk + lane/16), a
// row-wise 8-byte read (16 rows x 2 halves), and a transposing read (8 rows
// x 2 chunks x 2 halves).  Vb columns 128..135 (the normaliser column and
// padding) are a separate tile of 64 rows of 16 bytes.  The score share is
// 64 rows of 128 bytes with chunk k of row t at k ^ swz8(t).  The normaliser
// partials are 64 rows of 32 bytes whose two halves swap in rows 8..15 of
// every 16, so a phase's 16 rows cover the 256 bytes of the banks once.
#include <stdlib.h>

#include <type_traits>

#include "feat_map.hpp"
#include "smat_host.hpp"

namespace smat {

namespace ss {
constexpr int kThreads = 512;
constexpr int kStep = 64;                      // tokens per step
constexpr int kRowChunks = 16;                 // 16-byte chunks per Phi/Psi/Vb row
constexpr int kTileChunks = kStep * kRowChunks;    // 1024
constexpr int kVbTileChunks = kTileChunks + kStep; // + columns 128..135, one chunk a row
constexpr int kPhiLoads = kTileChunks / 64;        // wave-wide DMA loads per tile: 16
constexpr int kVbLoads = kVbTileChunks / 64;       // 17
constexpr int kLoads = 2 * kPhiLoads + kVbLoads;   // 49 per step, over eight waves
}  // namespace ss

#define SMAT_LDS __attribute__((address_space(3)))
typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz16(int t) {
  return (((t & 7) << 1) | ((t >> 3) & 1)) ^ (t & 8);
}
__device__ __forceinline__ int swz8(int t) { return (t >> 1) & 7; }
// Float index of wave w's normaliser partial of row t: 8 floats a row, the two
// 4-float halves swapped in rows 8..15 of every 16.
__device__ __forceinline__ int norm_slot(int t, int w) {
  return t * 8 + 4 * ((w >> 2) ^ ((t >> 3) & 1)) + (w & 3);
}

// Global loads the compiler does not track: their values may be used only
// after a wait_vmcnt that covers them and an opaque redefinition (asm "+v"),
// so no compiler-placed wait -- which would be vmcnt(0) with DMA loads and
// stores pending beside them -- drains the DMA issued after them.  "memory"
// keeps them in program order with the DMA, which the counts rely on.
__device__ __forceinline__ f32x4 load4_untracked(const void* p) {
  f32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=&v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ float load1_untracked(const void* p) {
  float v;
  asm volatile("global_load_dword %0, %1, off" : "=&v"(v) : "v"(p) : "memory");
  return v;
}
// A 16-bit element, zero-extended into a 32-bit register, untracked likewise.
__device__ __forceinline__ uint32_t load_u16_untracked(const void* p) {
  uint32_t v;
  asm volatile("global_load_ushort %0, %1, off" : "=&v"(v) : "v"(p) : "memory");
  return v;
}

// 8 bytes of a swizzled 256-byte row (t, chunk k, half h).
template <typename In>
__device__ __forceinline__ typename Traits<In>::half_frag row_half(const uint4* tile, int t, int k,
                                                                    int h) {
  const char* p = reinterpret_cast<const char*>(tile + t * ss::kRowChunks + (k ^ swz16(t))) + 8 * h;
  return *reinterpret_cast<const typename Traits<In>::half_frag*>(p);
}
// 16 bytes (one chunk) of a swizzled 256-byte row.
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag row_chunk(const uint4* tile, int t, int k) {
  return *reinterpret_cast<const typename Traits<In>::frag*>(tile + t * ss::kRowChunks +
                                                              (k ^ swz16(t)));
}

template <typename In>
__device__ __forceinline__ typename Traits<In>::half_frag tr_read(const char* addr) {
  short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (SMAT_LDS short4v*)(SMAT_LDS char*)(addr));
  return __builtin_bit_cast(typename Traits<In>::half_frag, v);
}

template <typename In>
__device__ __forceinline__ typename Traits<In>::frag join(typename Traits<In>::half_frag lo,
                                                          typename Traits<In>::half_frag hi) {
  typename Traits<In>::frag f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = lo[j];
    f[4 + j] = hi[j];
  }
  return f;
}

// A fragment of Psi^T (rows a = 16*at + lane%16, k-slots = tokens
// 32*ks + 8*grp + j) from a swizzled Psi tile, by two transposing reads.
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag psi_tr(const uint4* tile, int at, int ks,
                                                            int lane) {
  const int r16 = lane & 15, g = lane >> 4;
  typename Traits<In>::half_frag h2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = 32 * ks + 8 * g + 4 * h + (r16 >> 2);
    const int k = 2 * at + ((r16 & 3) >> 1);
    const char* p =
        reinterpret_cast<const char*>(tile + row * ss::kRowChunks + (k ^ swz16(row))) +
        8 * (r16 & 1);
    h2[h] = tr_read<In>(p);
  }
  return join<In>(h2[0], h2[1]);
}

// Fragment of Vb along tokens (column 16*ct + lane%16, k-slots = tokens
// 32*ks + 8*grp + j): the B operand of the state update and the A operand
// (Vb^T) of the within-step product.  Column tiles 0..7 are read like Psi's;
// tile 8 (columns 128..143) comes from the 16-byte rows of columns 128..135,
// and its lanes 8..15 repeat columns 128..135 in place of 136..143, which
// no caller keeps.
template <typename In>
__device__ __forceinline__ typename Traits<In>::frag vb_tr(const uint4* tile, int ct, int ks,
                                                           int lane) {
  if (ct < 8) return psi_tr<In>(tile, ct, ks, lane);
  const int r16 = lane & 15, g = lane >> 4;
  typename Traits<In>::half_frag h2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = 32 * ks + 8 * g + 4 * h + (r16 >> 2);
    const char* p = reinterpret_cast<const char*>(tile + ss::kTileChunks + row) + 8 * (r16 & 1);
    h2[h] = tr_read<In>(p);
  }
  return join<In>(h2[0], h2[1]);
}

// The DMA of one step's Phi, Psi and Vb rows [ts, ts + 64) into one buffer.
// Load I of the 49 goes to wave I % 8 as its slot u = I / 8: slots 0-1 are
// Phi's loads 0-15, slots 2-3 Psi's, slots 4-5 Vb's columns 0..127, and slot
// 6 (wave 0 only) Vb's columns 128..135, lane = row (wave 0 issues seven
// loads, the others six).  Each load moves 64 x 16 bytes to 1 KB of
// consecutive LDS; which global chunk a lane fetches implements the swizzle.
// That choice does not depend on the step, so a lane's byte offset from the
// step's first row is computed once per slot (dma_offsets); a step adds it
// to the wave-uniform row base of the slot's tensor.
struct DmaOffsets {
  uint32_t off[7];
};

template <typename In>
__device__ __forceinline__ void dma_offsets(DmaOffsets& d, const ScanArgs& a, int w, int lane) {
#pragma unroll
  for (int u = 0; u < 7; ++u) {
    const int I = w + 8 * u;
    int64_t e = 0;                                   // element offset from row ts
    if (u < 6) {
      const int li = I & 15;
      const int row = 4 * li + (lane >> 4);
      const int k = (lane & 15) ^ swz16(row);
      e = (int64_t)row * (u < 2 ? a.q_st : u < 4 ? a.k_st : a.v_st) + 8 * k;
    } else if (I < ss::kLoads) {
      e = (int64_t)lane * a.v_st + 128;              // columns 128..135 of row = lane
    }
    d.off[u] = (uint32_t)(e * (int64_t)sizeof(In));
  }
}

// FEAT: the rows are Q, K and V (the feature map runs in LDS afterwards), and
// the ninth Vb tile is the constant [1, 0, ...] written once: six loads a wave.
template <typename In, bool FEAT, bool UNTRACKED>
__device__ __forceinline__ void issue_step(uint4* dphi, uint4* dpsi, uint4* dvb, const In* phib,
                                           const In* psib, const In* vbb, int64_t ts,
                                           const ScanArgs& a, int w, const DmaOffsets& d) {
  const char* bphi = reinterpret_cast<const char*>(phib + ts * a.q_st);
  const char* bpsi = reinterpret_cast<const char*>(psib + ts * a.k_st);
  const char* bvb = reinterpret_cast<const char*>(vbb + ts * a.v_st);
#pragma unroll
  for (int u = 0; u < (FEAT ? 6 : 7); ++u) {
    const int I = w + 8 * u;
    if (I < ss::kLoads) {
      const char* base = u < 2 ? bphi : u < 4 ? bpsi : bvb;
      uint4* dst = u < 2 ? dphi + 64 * I
                 : u < 4 ? dpsi + 64 * (I - ss::kPhiLoads)
                         : dvb + 64 * (I - 2 * ss::kPhiLoads);
      lds_dma16<UNTRACKED>(reinterpret_cast<const void*>(base + d.off[u]), dst);
    }
  }
}

struct YRegs {
  float4 y[4];      // Y[t][16w + 4g .. +3] for the step's four row tiles
  float y8[4];      // Y[t][p - 1]
  float gv[4];      // gate
};

// Twelve loads, always issued (dummy in-bounds addresses when a term is
// absent), so the compiler's waits on them count a fixed number of loads.
// Per-lane byte offsets of the step's Y and output rows from row ts (the
// lane's rows 16 tt + lane % 16 at columns 16 w + 4 g), computed once; a step
// adds them to wave-uniform row bases.  y8 is the normaliser column's offset
// from the lane's Y chunk.
struct RowOffsets {
  uint32_t y[4], o[4];
  int y8;
};

__device__ __forceinline__ void row_offsets(RowOffsets& R, const ScanArgs& a, int w, int lane) {
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    R.y[tt] = (uint32_t)(((int64_t)(16 * tt + r16) * a.y_st + 16 * w + 4 * g) * 4);
    R.o[tt] = (uint32_t)(((int64_t)(16 * tt + r16) * a.o_st + 16 * w + 4 * g) * 4);
  }
  R.y8 = (a.p - 1 - 16 * w - 4 * g) * 4;
}

__device__ __forceinline__ void issue_y(YRegs& R, const float* Yb, const float* gb,
                                       const float* dummy, int64_t ts, const ScanArgs& a,
                                       const RowOffsets& ro, int lane) {
  const int r16 = lane & 15;
  const bool rec = Yb != nullptr && ts >= a.n;
  const char* yb = rec ? reinterpret_cast<const char*>(Yb + (ts - a.n) * a.y_st) : nullptr;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const char* yc = rec ? yb + ro.y[tt] : reinterpret_cast<const char*>(dummy);
    R.y[tt] = *reinterpret_cast<const float4*>(yc);
    R.y8[tt] = rec ? *reinterpret_cast<const float*>(yc + ro.y8) : 0.f;
    R.gv[tt] = gb ? gb[ts + 16 * tt + r16] : 1.f;
  }
}

__device__ __forceinline__ f32x4 mma16(f32x4 c, bf16x4 a, bf16x4 b) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a),
                                                   __builtin_bit_cast(s4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(f32x4 c, f16x4 a, f16x4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// FEAT = 1: phi, psi and vb are Q, K and V rows (v_st may be 128); each
// step's Phi and Psi tiles are formed from the DMA'd Q and K tiles into two
// more tiles, phiF and psiF (feat_rows, W in registers), the key gate applied
// to Psi.  A step's reads of phiF and psiF end before the barrier after its
// state update, so the next step's features overwrite them safely.
// FEAT = 2: psi holds Psi rows already (gate applied), only Phi is formed,
// in place over the DMA'd Q tile, with three row buffers.
template <typename In, int FEAT, int NBUF, bool TERMS>
__global__ __launch_bounds__(ss::kThreads, 1) void scan_stream_kernel(
    const In* __restrict__ phi, const In* __restrict__ psi, const In* __restrict__ vb,
    const float* __restrict__ Sg, const float* __restrict__ Y, const float* __restrict__ gate,
    float* __restrict__ out, ScanArgs a, FeatArgs fa) {
  using namespace ss;
  typedef typename Traits<In>::frag Frag;
  typedef typename Traits<In>::half_frag Half;
  __shared__ __attribute__((aligned(16))) uint4 phi0[kTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 psi0[kTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 vb0[kVbTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 phi1[kTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 psi1[kTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 vb1[kVbTileChunks];
  // NBUF = 3 (no Psi formed here): a third buffer (160 768 bytes of LDS in
  // all) keeps the rows of steps s + 1 and s + 2 in flight while step s
  // computes.
  // Y and the gate are then loaded untracked and waited for by count.
  // TERMS = false compiles Y and the gate out (launches with neither): their
  // pointers and flags would otherwise spill scalar registers every step.
  static_assert(NBUF == 2 || (NBUF == 3 && FEAT != 1), "three buffers only without Psi formed here");
  __shared__ __attribute__((aligned(16))) uint4 phi2[NBUF == 3 ? kTileChunks : 1];
  __shared__ __attribute__((aligned(16))) uint4 psi2[NBUF == 3 ? kTileChunks : 1];
  __shared__ __attribute__((aligned(16))) uint4 vb2[NBUF == 3 ? kVbTileChunks : 1];
  __shared__ __attribute__((aligned(16))) uint4 share[kStep * 8];
  // normaliser partials: wave w's share of H[t][p-1] at normp[norm_slot(t, w)]
  __shared__ __attribute__((aligned(16))) float normp[kStep * 8];
  __shared__ __attribute__((aligned(16))) uint4 phiF[FEAT && NBUF == 2 ? kTileChunks : 1];
  __shared__ __attribute__((aligned(16))) uint4 psiF[FEAT == 1 ? kTileChunks : 1];

  // Groups run last sequence first, last group first: the prepass just read
  // the same Psi and Vb rows in the opposite order, so the first groups here
  // find theirs in the memory-side cache (556 -> 531 us for the causal pass
  // at 8 x 131072 tokens).
  const int grp = gridDim.x - 1 - blockIdx.x;
  const int64_t b = gridDim.y - 1 - blockIdx.y;
  // The wave index in a scalar register: every condition on it below is a
  // scalar branch.  (Under a vector condition the compiler masks EXEC around
  // an MFMA without branching past it, and MFMAs execute regardless of EXEC.)
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  // Eight waves: the DMA's loads 0..47 are then unconditional, and the
  // compiler's count of loads issued after the Y loads is exact.
  __builtin_assume(w >= 0 && w < 8);
  const int lane = lane_id();
  const int r16 = lane & 15, g = lane >> 4;

  int c0, c1;
  if (grp < a.ng0) {
    c0 = grp * a.K;
    c1 = min(c0 + a.K, a.nc0);
  } else {
    c0 = a.nc0 + (grp - a.ng0) * a.K;
    c1 = min(c0 + a.K, a.nc);
  }
  const int64_t tk0 = (int64_t)c0 * a.C;
  const int64_t tk1 = min((int64_t)c1 * a.C, (int64_t)a.T);
  const int nsteps = (int)((tk1 - tk0) / kStep);

  const In* phib = phi + b * a.q_sb;
  const In* psib = psi + b * a.k_sb;
  const In* vbb = vb + b * a.v_sb;
  const float* Yb = (TERMS && Y) ? Y + b * a.y_sb : nullptr;
  const float* gb = (TERMS && gate) ? gate + b * a.g_sb : nullptr;
  float* outb = out + b * a.o_sb;
  const float* Sb = Sg + ((int64_t)b * gridDim.x + grp) * (int64_t)128 * a.p;

  DmaOffsets dmo;
  dma_offsets<In>(dmo, a, w, lane);
  RowOffsets rof;
  row_offsets(rof, a, w, lane);
  if (nsteps > 0) issue_step<In, FEAT != 0, NBUF == 3>(phi0, psi0, vb0, phib, psib, vbb, tk0, a, w, dmo);
  Frag wa[4];
  const In* hb = nullptr;
  if constexpr (FEAT) {
    feat_w_load<In>(wa, (const In*)fa.W, w, lane);
    feat_ones_tile<In>(vb0 + kTileChunks, threadIdx.x, kThreads);
    feat_ones_tile<In>(vb1 + kTileChunks, threadIdx.x, kThreads);
    if (NBUF == 3) feat_ones_tile<In>(vb2 + kTileChunks, threadIdx.x, kThreads);
    if (FEAT == 1) hb = fa.h ? (const In*)fa.h + b * fa.h_sb : nullptr;
  }

  // incoming state: S[a][16w + lane%16] for all a, and the normaliser column
  // block S[a][128 + lane%16] for this wave's rows a in [16w, 16w + 16)
  const int cn = a.p - 1 - 128;            // normaliser's row in the ninth tile
  f32x4 accS[8], accS8;
#pragma unroll
  for (int at = 0; at < 8; ++at)
#pragma unroll
    for (int i = 0; i < 4; ++i) accS[at][i] = Sb[(int64_t)(16 * at + 4 * g + i) * a.p + 16 * w + r16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c8 = 128 + r16;
    const float v8 = Sb[(int64_t)(16 * w + 4 * g + i) * a.p + (c8 < a.p ? c8 : 0)];
    accS8[i] = c8 < a.p ? v8 : 0.f;
  }
  // Consume the state (and W) loads here, so that no wait for them is placed
  // inside the loop.  With three buffers the copies are untracked and the
  // compiler's wait here is vmcnt(0), which lands step 0's rows too; step
  // 1's copy goes out after it.
#pragma unroll
  for (int at = 0; at < 8; ++at) asm volatile("" : "+v"(accS[at]));
  asm volatile("" : "+v"(accS8));
  if constexpr (FEAT) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(wa[kb]));
  }
  if (NBUF == 3 && nsteps > 1)
    issue_step<In, FEAT != 0, true>(phi1, psi1, vb1, phib, psib, vbb, tk0 + kStep, a, w, dmo);

  auto step = [&](auto BUFC, int s) {
    constexpr int BUF = decltype(BUFC)::value;
    const uint4* tphi = FEAT && NBUF == 2 ? phiF : BUF == 2 ? phi2 : BUF ? phi1 : phi0;
    const uint4* tpsi = FEAT == 1 ? psiF : BUF == 2 ? psi2 : BUF ? psi1 : psi0;
    const uint4* tvb = BUF == 2 ? vb2 : BUF ? vb1 : vb0;
    const int64_t ts = tk0 + (int64_t)s * kStep;
    // An opaque copy of the lane index per step: the LDS addresses derived
    // from it are recomputed inside the step instead of being hoisted out of
    // the loop, where the ~60 distinct swizzled addresses would pin as many
    // registers for the whole kernel.
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int r16 = lane & 15, g = lane >> 4;
    float hv[4] = {1.f, 1.f, 1.f, 1.f};    // FEAT = 1: the key gate of the lane's four rows
    if constexpr (FEAT == 1) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) hv[tt] = hb ? to_f32(hb[ts + 16 * tt + r16]) : 1.f;
    }
    static_assert(kLoads / 8 == 6 && kLoads % 8 == 1, "seven loads on wave 0, six on the rest");
    if constexpr (NBUF == 3) {
      // Issued after this step's DMA: the previous step's output stores and the
      // next step's DMA, seven loads on wave 0 and six on the rest (six on every
      // wave with the feature map).  Loads complete in order, so waiting down
      // to that many lands this step's rows.
      if (s + 1 < nsteps) {
        if (!FEAT && w == 0)
          wait_vmcnt<7>();
        else
          wait_vmcnt<6>();
      } else {
        wait_vmcnt<0>();
      }
    } else if (s + 1 < nsteps) {
      issue_step<In, FEAT != 0, NBUF == 3>(BUF ? phi0 : phi1, BUF ? psi0 : psi1, BUF ? vb0 : vb1, phib, psib,
                           vbb, ts + kStep, a, w, dmo);
      // the gate loads (issued first) are older than this step's six DMA loads
      if (!FEAT && w == 0)
        wait_vmcnt<7>();
      else
        wait_vmcnt<6>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();      // every wave's DMA of this step has landed
    if constexpr (FEAT && NBUF == 3) {
      // in place: feat_rows reads every wave's rows, then waits, then writes
      const auto sw = [](int t) { return swz16(t); };
      uint4* tq = BUF == 2 ? phi2 : BUF ? phi1 : phi0;
      feat_rows<In, 4>(tq, tq, 0, true, wa, w, fa.kind, false, hv, lane, sw);
      lds_barrier();    // the step's Phi tile is complete
    } else if constexpr (FEAT) {
      const auto sw = [](int t) { return swz16(t); };
      feat_rows<In, 4>(BUF ? phi1 : phi0, phiF, 0, true, wa, w, fa.kind, false, hv, lane, sw);
      if constexpr (FEAT == 1)
        feat_rows<In, 4>(BUF ? psi1 : psi0, psiF, 0, true, wa, w, fa.kind, hb != nullptr, hv, lane,
                         sw);
      lds_barrier();    // the step's Phi (and Psi) tiles are complete
    }
    YRegs yr;
    if constexpr (NBUF == 2) issue_y(yr, Yb, gb, Sb, ts, a, rof, lane);
    // Three buffers: the step's Y rows and gates, untracked; the only vector
    // memory issued after them before (e) is the DMA of step s + 2.
    const bool rec = Yb != nullptr && ts >= a.n;
    f32x4 ya[4];
    float y8a[4], ga[4];
    if constexpr (NBUF == 3) {
      if (rec) {
        const char* yb = reinterpret_cast<const char*>(Yb + (ts - a.n) * a.y_st);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          ya[tt] = load4_untracked(yb + rof.y[tt]);
          y8a[tt] = load1_untracked(yb + rof.y[tt] + rof.y8);
        }
      }
      if (gb) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) ga[tt] = load1_untracked(gb + ts + 16 * tt + r16);
      }
    }

    // (a) this wave's share of the causal score tiles A^T = Psi Phi^T
    //     entries 0..9: (ut, tt) with ut <= tt; 10, 11: zero tiles (1,0), (3,2).
    //     Wave w takes entry w and, for w < 4, entry w + 8: waves 0, 1 two
    //     products, whose fragments are all read first and whose MFMA chains
    //     interleave; waves 2, 3 a product and a zero tile.
    {
      auto entry = [](int e, int& ut, int& tt) {
        if (e < 10) {
          tt = e < 1 ? 0 : e < 3 ? 1 : e < 6 ? 2 : 3;
          ut = e - (tt * (tt + 1)) / 2;
        } else {
          ut = e == 10 ? 1 : 3;
          tt = e == 10 ? 0 : 2;
        }
      };
      // acc[i] = A^T[t' = 16ut + 4g + i][t = 16tt + r16] = A[t][t'], masked,
      // rounded to the input type and stored to the share
      auto put = [&](const f32x4& acc, int ut, int tt) {
        Half hv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool keep = ut < tt || 4 * g + i <= r16;
          hv[i] = from_f32<In>(keep ? acc[i] : 0.f);
        }
        const int t = 16 * tt + r16;
        const int k = 2 * ut + (g >> 1);
        char* p = reinterpret_cast<char*>(share + t * 8 + (k ^ swz8(t))) + 8 * (g & 1);
        *reinterpret_cast<Half*>(p) = hv;
      };
      int ut0, tt0, ut1, tt1;
      entry(w, ut0, tt0);
      entry(w + 8, ut1, tt1);
      Frag fa0[4], fb0[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        fa0[kk] = row_chunk<In>(tpsi, 16 * ut0 + r16, 4 * kk + g);
        fb0[kk] = row_chunk<In>(tphi, 16 * tt0 + r16, 4 * kk + g);
      }
      f32x4 acc0 = zero4();
      if (w < 2) {
        Frag fa1[4], fb1[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          fa1[kk] = row_chunk<In>(tpsi, 16 * ut1 + r16, 4 * kk + g);
          fb1[kk] = row_chunk<In>(tphi, 16 * tt1 + r16, 4 * kk + g);
        }
        f32x4 acc1 = zero4();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          acc0 = mma(acc0, fa0[kk], fb0[kk]);
          acc1 = mma(acc1, fa1[kk], fb1[kk]);
        }
        put(acc1, ut1, tt1);
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc0 = mma(acc0, fa0[kk], fb0[kk]);
        if (w < 4) put(zero4(), ut1, tt1);
      }
      put(acc0, ut0, tt0);
    }

    // Three buffers: step s + 2's rows go to the buffer step s - 1 used, free
    // since that step's last barrier.  Issued after the score reads: before
    // them, the compiler waits for the whole DMA in one of the three steps.
    if constexpr (NBUF == 3) {
      constexpr int NB = (BUF + 2) % 3;
      if (s + 2 < nsteps)
        issue_step<In, FEAT != 0, NBUF == 3>(NB == 2 ? phi2 : NB ? phi1 : phi0, NB == 2 ? psi2 : NB ? psi1 : psi0,
                             NB == 2 ? vb2 : NB ? vb1 : vb0, phib, psib, vbb, ts + 2 * kStep, a,
                             w, dmo);
    }

    // (b) O^T = S^T Phi^T with the state before this step; the normaliser
    //     column's share of this wave's 16 state rows
    f32x4 accO[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) accO[tt] = zero4();
    // Row t = 16 tt + r16 of the Phi tile, one opaque base per tt.  Rows t and
    // t + 16 sit at the same swizzle 4096 bytes apart; seen as such, their two
    // 8-byte reads are fused into one ds_read2st64_b64, which the LDS serves at
    // half the rate of two ds_read_b64 and with this pattern's lanes in
    // conflict.  With opaque bases every read stays a ds_read_b64.
    const char* prow[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      uint32_t off = (uint32_t)(16 * tt + r16) * (ss::kRowChunks * 16);
      asm volatile("" : "+v"(off));
      prow[tt] = reinterpret_cast<const char*>(tphi) + off;
    }
    const int sw = swz16(r16);
    auto phi_half = [&](int tt, int k) {
      return *reinterpret_cast<const Half*>(prow[tt] + ((k ^ sw) * 16 + 8 * (g & 1)));
    };
    // The Phi fragments of k-block kk + 1 are read while block kk's state is
    // split and multiplied, and the hi parts of the four row tiles go before
    // the lo parts, so no MFMA waits on the one before it.
    Frag bfs[2][4];
    auto read_bf = [&](Frag(&dst)[4], int kk) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        dst[tt] = join<In>(phi_half(tt, 4 * kk + (g >> 1)), phi_half(tt, 4 * kk + 2 + (g >> 1)));
    };
    read_bf(bfs[0], 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) read_bf(bfs[(kk + 1) & 1], kk + 1);
      Half h0, l0, h1, l1;
      split4<In>(accS[2 * kk], h0, l0);
      split4<In>(accS[2 * kk + 1], h1, l1);
      const Frag shi = join<In>(h0, h1), slo = join<In>(l0, l1);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) accO[tt] = mma(accO[tt], shi, bfs[kk & 1][tt]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) accO[tt] = mma(accO[tt], slo, bfs[kk & 1][tt]);
    }
    float own = 0.f;                       // wave w < 4: its row tile's value, finished in (d)
    {
      Half s8hi, s8lo, bfn[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) bfn[tt] = phi_half(tt, 2 * w + (g >> 1));
      split4<In>(accS8, s8hi, s8lo);
      f32x4 pn[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) pn[tt] = mma16(zero4(), s8hi, bfn[tt]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) pn[tt] = mma16(pn[tt], s8lo, bfn[tt]);
      if (g == (cn >> 2)) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          if (tt == w)
            own = pn[tt][cn & 3];
          else
            normp[norm_slot(16 * tt + r16, w)] = pn[tt][cn & 3];
        }
      }
    }

    // (c) S += Psi^T Vb over the step's 64 tokens
    // The ninth tile's rows of this wave take the Psi fragment of row tile w
    // once more, outside the loop: a branch on at == w inside it would split
    // the loop into blocks the compiler cannot move a read across.
    // The sixteen (ks, at) products run in order with the Psi fragments of the
    // next two read ahead (sched barriers keep the compiler from sinking the
    // reads to their MFMAs).
    Frag vbw[2], vb8[2], pa[3];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      vbw[ks] = vb_tr<In>(tvb, w, ks, lane);
      vb8[ks] = vb_tr<In>(tvb, 8, ks, lane);
    }
    pa[0] = psi_tr<In>(tpsi, 0, 0, lane);
    pa[1] = psi_tr<In>(tpsi, 1, 0, lane);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i + 2 < 16) pa[(i + 2) % 3] = psi_tr<In>(tpsi, (i + 2) & 7, (i + 2) >> 3, lane);
      __builtin_amdgcn_sched_barrier(0);
      accS[i & 7] = mma(accS[i & 7], pa[i % 3], vbw[i >> 3]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) accS8 = mma(accS8, psi_tr<In>(tpsi, w, ks, lane), vb8[ks]);
    lds_barrier();       // the score share is complete

    // (d) O^T += Vb^T A^T within the step; waves 0..3 add the row sums of A
    //     (the ones column) to their row tile's normaliser
    auto share_bf = [&](int t, int ks) {
      return *reinterpret_cast<const Frag*>(share + t * 8 + ((4 * ks + g) ^ swz8(t)));
    };
    {
      Frag sh[4][2];    // the six causal score fragments, read before their MFMAs
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int ks = 0; ks <= (tt >> 1); ++ks) sh[tt][ks] = share_bf(16 * tt + r16, ks);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int tt = 2 * ks; tt < 4; ++tt) accO[tt] = mma(accO[tt], vbw[ks], sh[tt][ks]);
    }
    if (w < 4) {        // row tile w's normaliser: the row sums of its score tiles
      const int t = 16 * w + r16;
      f32x4 p8 = mma(zero4(), vb8[0], share_bf(t, 0));
      if (w >= 2) p8 = mma(p8, vb8[1], share_bf(t, 1));
      if (g == (cn >> 2)) normp[norm_slot(t, w)] = own + p8[cn & 3];
    }
    lds_barrier();

    // (e) long-range term, normalise, store four columns per lane per row tile
    if constexpr (NBUF == 3) {
      if (rec || gb) {
        // everything issued after the Y and gate loads: step s + 2's DMA
        if (s + 2 < nsteps) {
          if (!FEAT && w == 0)
            wait_vmcnt<7>();
          else
            wait_vmcnt<6>();
        } else {
          wait_vmcnt<0>();
        }
        asm volatile("" : "+v"(ya[0]), "+v"(ya[1]), "+v"(ya[2]), "+v"(ya[3]), "+v"(y8a[0]),
                     "+v"(y8a[1]), "+v"(y8a[2]), "+v"(y8a[3]));
        asm volatile("" : "+v"(ga[0]), "+v"(ga[1]), "+v"(ga[2]), "+v"(ga[3]));
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = 16 * tt + r16;
      const float4 n0 = *reinterpret_cast<const float4*>(normp + norm_slot(t, 0));
      const float4 n1 = *reinterpret_cast<const float4*>(normp + norm_slot(t, 4));
      float den = ((n0.x + n0.y) + (n0.z + n0.w)) + ((n1.x + n1.y) + (n1.z + n1.w));
      float4 o;
      o.x = accO[tt][0];
      o.y = accO[tt][1];
      o.z = accO[tt][2];
      o.w = accO[tt][3];
      if (rec) {
        if constexpr (NBUF == 3) {
          den += y8a[tt];
          o.x += ya[tt][0];
          o.y += ya[tt][1];
          o.z += ya[tt][2];
          o.w += ya[tt][3];
        } else {
          den += yr.y8[tt];
          o.x += yr.y[tt].x;
          o.y += yr.y[tt].y;
          o.z += yr.y[tt].z;
          o.w += yr.y[tt].w;
        }
      }
      const float num = NBUF == 3 ? (gb ? ga[tt] : 1.f) : yr.gv[tt];   // the gate (1 without)
      // the reciprocal (1 ulp) in place of the IEEE division's ten-instruction
      // sequence; the product below rounds once more either way
      const float inv = num * __builtin_amdgcn_rcpf(den);
      o.x *= inv;
      o.y *= inv;
      o.z *= inv;
      o.w *= inv;
      *reinterpret_cast<float4*>(reinterpret_cast<char*>(outb + ts * a.o_st) + rof.o[tt]) = o;
    }
  };

  if constexpr (NBUF == 3) {
    for (int s = 0; s < nsteps; s += 3) {
      step(std::integral_constant<int, 0>{}, s);
      if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
      if (s + 2 < nsteps) step(std::integral_constant<int, 2>{}, s + 2);
    }
  } else {
    for (int s = 0; s < nsteps; s += 2) {
      step(std::integral_constant<int, 0>{}, s);
      if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
    }
  }
}

// ---------------------------------------------------------------------------
// Gram sums G = sum_t Psi_t^T Vb_t over a token progression (the chunk-group
// prepass of the causal pass, and the profile pool), same machinery: rows
// of 64 tokens at a time copied HBM -> LDS by DMA (double-buffered), read
// along tokens by transposing LDS reads, wave w accumulating G[:, 16w ..
// 16w+15] and rows [16w, 16w+16) of the ninth column tile.  Rows past the end
// of a progression are fetched from its first token (in bounds) and zeroed in
// the Vb fragment, so they add nothing.
// ---------------------------------------------------------------------------

// Issue one step's DMA: Psi (16 loads) and Vb (17) for rows
// tok(row) = start + stride * (base + row), row < 64; wave 0 issues five
// loads, the others four.
// FEAT: K and V rows; the ninth Vb tile is constant, so 32 loads, four a wave.
// Token of term idx: LIST (mode 2) reads it from the item's column list; the
// other modes compute it, with no index loads whose waits (vmcnt(0), placed by
// the compiler at every join after them) would drain the DMA in flight.
template <bool LIST>
__device__ __forceinline__ int64_t gram_token_of(const GramItems& it, int item, int64_t start,
                                                 int64_t stride, int idx) {
  if constexpr (LIST)
    return gram_token(it, item, start, stride, idx);
  else
    return start + (int64_t)idx * stride;
}

template <typename In, bool FEAT, bool LIST>
__device__ __forceinline__ void issue_gram(uint4* dpsi, uint4* dvb, const In* psib,
                                           const In* vbb, const GramItems& it, int item,
                                           int64_t start, int64_t stride, int base, int count,
                                           int64_t k_st, int64_t v_st, int w, int lane) {
  constexpr int kL = ss::kPhiLoads + ss::kVbLoads - (FEAT ? 1 : 0);     // 33 or 32
#pragma unroll
  for (int u = 0; u < 5; ++u) {
    const int I = w + 8 * u;
    if (I < kL) {
      const In* src;
      uint4* dst;
      if (I < ss::kPhiLoads) {
        const int row = 4 * I + (lane >> 4);
        const int k = (lane & 15) ^ swz16(row);
        const int64_t tok =
            gram_token_of<LIST>(it, item, start, stride, base + row < count ? base + row : 0);
        src = psib + tok * k_st + 8 * k;
        dst = dpsi + 64 * I;
      } else {
        // Vb columns 0..127 swizzled like Psi, then columns 128..135, lane = row
        const int li = I - ss::kPhiLoads;
        const int row = li < ss::kPhiLoads ? 4 * li + (lane >> 4) : lane;
        const int col = li < ss::kPhiLoads ? 8 * ((lane & 15) ^ swz16(row)) : 128;
        const int64_t tok =
            gram_token_of<LIST>(it, item, start, stride, base + row < count ? base + row : 0);
        src = vbb + tok * v_st + col;
        dst = dvb + 64 * li;
      }
      // untracked except with the list's token loads, whose own compiler
      // waits drain the copies anyway
      lds_dma16<!LIST>(reinterpret_cast<const void*>(src), dst);
    }
  }
}

// ONE: every item of the launch has at most kStep terms (the profile pool at
// long T: (n - n_P) / N0 tokens a profile), so one buffer suffices.  Its
// 35 KB of LDS let three workgroups share a CU instead of two, which is what
// a launch of one-step items -- a load latency, a few MFMAs and a 66 KB
// store each -- is limited by.
// FEAT: psi and vb are K and V rows; each step's Psi tile is formed in place
// from the DMA'd K tile (feat_rows, W in registers, two halves of 32 rows),
// times the key gate.
template <typename In, bool ONE, bool FEAT, bool LIST>
__global__ __launch_bounds__(ss::kThreads, (ONE && !FEAT) ? 3 : 2) void gram_stream_kernel(
    const In* __restrict__ psi, const In* __restrict__ vb, float* __restrict__ G,
    float* __restrict__ G_last, GramItems it, int p, int64_t k_sb, int64_t k_st, int64_t v_sb,
    int64_t v_st, int64_t g_sb, int64_t g_si, int64_t gl_sb, FeatArgs fa) {
  using namespace ss;
  typedef typename Traits<In>::frag Frag;
  // psi0 and vb0 are one array: after the last step it stages the output
  __shared__ __attribute__((aligned(16))) uint4 stage0[kTileChunks + kVbTileChunks];
  static_assert((kTileChunks + kVbTileChunks) * 16 >= 64 * 129 * 4, "stage holds 64 rows of G");
  uint4* psi0 = stage0;
  uint4* vb0 = stage0 + kTileChunks;
  __shared__ __attribute__((aligned(16))) uint4 psi1[ONE ? 1 : kTileChunks];
  __shared__ __attribute__((aligned(16))) uint4 vb1[ONE ? 1 : kVbTileChunks];

  // Profiles (mode 1) run point by point across the sequences, so the last
  // rows of F written -- the ones the memory-side cache still holds when the
  // incidence starts -- are spread over all sequences, whose slices the
  // incidence walks on separate XCDs.
  int item = blockIdx.x;
  int64_t b = blockIdx.y;
  if (it.mode == 1) {
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    b = lin % gridDim.y;
    item = (int)(lin / gridDim.y);
  }
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  __builtin_assume(w >= 0 && w < 8);                 // eight waves
  int64_t start, stride;
  int count;
  gram_item(it, item, start, stride, count);
  const In* psib = psi + b * k_sb;
  const In* vbb = vb + b * v_sb;
  float* Gout = (it.mode == 1 && item == it.N0) ? G_last + b * gl_sb : G + b * g_sb + item * g_si;
  const int nsteps = (count + kStep - 1) / kStep;

  f32x4 accS[8], accS8 = zero4();
#pragma unroll
  for (int at = 0; at < 8; ++at) accS[at] = zero4();
  if (nsteps > 0)
    issue_gram<In, FEAT, LIST>(psi0, vb0, psib, vbb, it, item, start, stride, 0, count, k_st, v_st, w,
                         lane_id());
  Frag wa[4];
  const In* hb = nullptr;
  if constexpr (FEAT) {
    feat_w_load<In>(wa, (const In*)fa.W, w, lane_id());
    feat_ones_tile<In>(vb0 + kTileChunks, threadIdx.x, kThreads);
    if (!ONE) feat_ones_tile<In>(vb1 + kTileChunks, threadIdx.x, kThreads);
    hb = fa.h ? (const In*)fa.h + b * fa.h_sb : nullptr;
    // consumed here (the compiler's wait also lands step 0's rows), so no
    // wait for W sits inside the loop
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(wa[kb]));
  }

  auto step = [&](auto BUFC, int s) {
    constexpr int BUF = decltype(BUFC)::value;
    const uint4* tpsi = BUF ? psi1 : psi0;
    const uint4* tvb = BUF ? vb1 : vb0;
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int g = lane >> 4;
    // FEAT: the key gate of the lane's four rows, loaded untracked before the
    // next step's copy and consumed after the wait that covers it
    uint32_t hraw[4] = {0, 0, 0, 0};
    if constexpr (FEAT) {
      const int r16 = lane & 15;
      if (hb) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          const int row = s * kStep + 16 * tt + r16;
          hraw[tt] = load_u16_untracked(
              hb + gram_token_of<LIST>(it, item, start, stride, row < count ? row : 0));
        }
      }
    }
    if (!ONE && s + 1 < nsteps) {
      issue_gram<In, FEAT, LIST>(BUF ? psi0 : psi1, BUF ? vb0 : vb1, psib, vbb, it, item, start, stride,
                           (s + 1) * kStep, count, k_st, v_st, w, lane);
      static_assert(kPhiLoads + kVbLoads == 33, "five loads on wave 0, four on the rest");
      // the gate loads (issued first) are older than this step's DMA loads
      if (!FEAT && w == 0)
        wait_vmcnt<5>();
      else
        wait_vmcnt<4>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if constexpr (FEAT) {
      float hv[4] = {1.f, 1.f, 1.f, 1.f};
      if (hb) {
        asm volatile("" : "+v"(hraw[0]), "+v"(hraw[1]), "+v"(hraw[2]), "+v"(hraw[3]));
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) hv[tt] = to_f32(__builtin_bit_cast(In, (uint16_t)hraw[tt]));
      }
      uint4* fpsi = BUF ? psi1 : psi0;
      const auto sw = [](int t) { return swz16(t); };
      const float h01[2] = {hv[0], hv[1]}, h23[2] = {hv[2], hv[3]};
      feat_rows<In, 2>(fpsi, fpsi, 0, true, wa, w, fa.kind, hb != nullptr, h01, lane, sw);
      feat_rows<In, 2>(fpsi, fpsi, 2, true, wa, w, fa.kind, hb != nullptr, h23, lane, sw);
      lds_barrier();    // the step's Psi tile is complete
      if (fa.psi_out != nullptr) {
        // the tile's rows to psi_out: thread (t, c) of 64 rows x 8 pairs of
        // 16-byte chunks, un-swizzled, for the rows that hold tokens
        const int t = threadIdx.x >> 3, c = 2 * (threadIdx.x & 7);
        const int row = s * kStep + t;
        if (row < count) {
          const int64_t tok = gram_token_of<LIST>(it, item, start, stride, row);
          uint4* dst = reinterpret_cast<uint4*>((In*)fa.psi_out + b * fa.psi_sb + tok * 128);
          dst[c] = fpsi[t * kRowChunks + (c ^ swz16(t))];
          dst[c + 1] = fpsi[t * kRowChunks + ((c + 1) ^ swz16(t))];
        }
      }
    }
    const int nvalid = count - s * kStep;        // rows of this step holding tokens
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Frag vbw = vb_tr<In>(tvb, w, ks, lane);
      Frag vb8 = vb_tr<In>(tvb, 8, ks, lane);
      if (nvalid < kStep) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool ok = 32 * ks + 8 * g + e < nvalid;
          vbw[e] = ok ? vbw[e] : from_f32<In>(0.f);
          vb8[e] = ok ? vb8[e] : from_f32<In>(0.f);
        }
      }
#pragma unroll
      for (int at = 0; at < 8; ++at) {
        const Frag pa = psi_tr<In>(tpsi, at, ks, lane);
        accS[at] = mma(accS[at], pa, vbw);
        if (at == w) accS8 = mma(accS8, pa, vb8);
      }
    }
    lds_barrier();     // this buffer is free for the DMA issued next step
  };
  if constexpr (ONE) {
    if (nsteps > 0) step(std::integral_constant<int, 0>{}, 0);     // nsteps <= 1
  } else {
    for (int s = 0; s < nsteps; s += 2) {
      step(std::integral_constant<int, 0>{}, s);
      if (s + 1 < nsteps) step(std::integral_constant<int, 1>{}, s + 1);
    }
  }

  const int lane = lane_id();
  const int r16 = lane & 15, g = lane >> 4;
  if (p == 129 && (reinterpret_cast<uintptr_t>(Gout) & 15) == 0) {
    // The r x p result is one contiguous block.  Stage it 64 rows (33 KB) at
    // a time in the idle tile buffer and store each half as consecutive
    // 16-byte stores: whole cache lines, instead of 64-byte runs of
    // 516-byte rows.  Non-temporal: the table (888 MB for the long-prefill
    // pool) is far larger than the last-level cache and is read back only by
    // the next kernel.
    float* st = reinterpret_cast<float*>(stage0);
    constexpr int kHalf = 64 * 129;                  // floats
    for (int h = 0; h < 2; ++h) {
      lds_barrier();                                 // the tile buffer is free
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st[(16 * q4 + 4 * g + i) * 129 + 16 * w + r16] = accS[4 * h + q4][i];
      if ((w >> 2) == h && r16 == 0) {               // column 128: rows 16 w + 4 g + i
#pragma unroll
        for (int i = 0; i < 4; ++i) st[(16 * (w & 3) + 4 * g + i) * 129 + 128] = accS8[i];
      }
      lds_barrier();
      const float4* src = reinterpret_cast<const float4*>(st);
      float4* dst = reinterpret_cast<float4*>(Gout + h * kHalf);
      for (int e = threadIdx.x; e < kHalf / 4; e += kThreads) {
        const float4 v = src[e];
        __builtin_nontemporal_store(v.x, &dst[e].x);
        __builtin_nontemporal_store(v.y, &dst[e].y);
        __builtin_nontemporal_store(v.z, &dst[e].z);
        __builtin_nontemporal_store(v.w, &dst[e].w);
      }
    }
    return;
  }
#pragma unroll
  for (int at = 0; at < 8; ++at)
#pragma unroll
    for (int i = 0; i < 4; ++i) Gout[(int64_t)(16 * at + 4 * g + i) * p + 16 * w + r16] = accS[at][i];
  if (128 + r16 < p) {
#pragma unroll
    for (int i = 0; i < 4; ++i) Gout[(int64_t)(16 * w + 4 * g + i) * p + 128 + r16] = accS8[i];
  }
}

bool gram_stream_ok(int dtype, const void* psi, const void* vb, int r, int p, int64_t k_sb,
                    int64_t k_st, int64_t v_sb, int64_t v_st, const GramItems& it, int nitems,
                    int nb) {
  if (dtype != SMAT_BF16 && dtype != SMAT_F16) return false;
  if (r != 128 || p != 129 || it.nsplit > 1) return false;
  if ((int64_t)nitems * nb < 256) return false;        // few, long items: the split-K kernel
  if (!rows_vec_ok(psi, k_sb, k_st, 2) || !rows_vec_ok(vb, v_sb, v_st, 2) || v_st < 136)
    return false;
  return variant(SMAT_VARIANT_GRAM) == 0;
}

template <typename In, bool FEAT>
static void gram_stream_kernel_launch(const void* psi, const void* vb, float* G, float* G_last,
                                      const GramItems& it, dim3 grid, bool one, int p,
                                      int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                                      int64_t g_sb, int64_t g_si, int64_t gl_sb,
                                      const FeatArgs& fa, hipStream_t stream) {
  const In* k = (const In*)psi;
  const In* v = (const In*)vb;
  const dim3 blk(ss::kThreads);
  // the feature map runs for profiles and chunk groups only: no list form
  if (!FEAT && it.mode == 2) {
    if (one)
      smat::launch((gram_stream_kernel<In, true, false, true>), grid, blk, 0, stream, k, v,
                         G, G_last, it, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb, fa);
    else
      smat::launch((gram_stream_kernel<In, false, false, true>), grid, blk, 0, stream, k, v,
                         G, G_last, it, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb, fa);
  } else if (one) {
    smat::launch((gram_stream_kernel<In, true, FEAT, false>), grid, blk, 0, stream, k, v, G,
                       G_last, it, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb, fa);
  } else {
    smat::launch((gram_stream_kernel<In, false, FEAT, false>), grid, blk, 0, stream, k, v,
                       G, G_last, it, p, k_sb, k_st, v_sb, v_st, g_sb, g_si, gl_sb, fa);
  }
}

template <bool FEAT>
static int gram_stream_go(int dtype, const void* psi, const void* vb, float* G, float* G_last,
                          const GramItems& it, int nitems, int nb, int p, int64_t k_sb,
                          int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                          int64_t gl_sb, const FeatArgs& fa, hipStream_t stream,
                          const char* who) {
  dim3 grid((unsigned)nitems, (unsigned)nb);
  // the longest item: a profile has ceil((n - n_P) / N0) terms, the global
  // channel (item N0, when launched) n_P
  bool one = false;
  if (it.mode == 1) {
    int64_t maxc = it.N0 > 0 ? ((int64_t)it.n - it.n_P + it.N0 - 1) / it.N0 : 0;
    if (nitems > it.N0) maxc = maxc > it.n_P ? maxc : it.n_P;
    one = maxc <= ss::kStep;
  }
  if (dtype == SMAT_BF16)
    gram_stream_kernel_launch<bf16, FEAT>(psi, vb, G, G_last, it, grid, one, p, k_sb, k_st, v_sb,
                                          v_st, g_sb, g_si, gl_sb, fa, stream);
  else
    gram_stream_kernel_launch<f16, FEAT>(psi, vb, G, G_last, it, grid, one, p, k_sb, k_st, v_sb,
                                         v_st, g_sb, g_si, gl_sb, fa, stream);
  return launch_status(who);
}

int gram_stream_launch(int dtype, const void* psi, const void* vb, float* G, float* G_last,
                       const GramItems& it, int nitems, int nb, int p, int64_t k_sb,
                       int64_t k_st, int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                       int64_t gl_sb, hipStream_t stream, const char* who) {
  return gram_stream_go<false>(dtype, psi, vb, G, G_last, it, nitems, nb, p, k_sb, k_st, v_sb,
                               v_st, g_sb, g_si, gl_sb, FeatArgs{}, stream, who);
}

// The Gram sums with the feature map in place: k, v are K and V rows
// (d_qk = d_v = 128, 16-byte aligned rows); any item count (no split-K).
int gram_stream_launch_feat(int dtype, const void* k, const void* v, float* G, float* G_last,
                            const GramItems& it, int nitems, int nb, int64_t k_sb, int64_t k_st,
                            int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                            int64_t gl_sb, const FeatArgs& fa, hipStream_t stream,
                            const char* who) {
  if (nitems == 0 || nb == 0) return SMAT_OK;
  if (it.mode == 2) {                  // compiled for profiles and chunk groups only
    set_error("%s: the feature map is not fused into list Gram sums", who);
    return SMAT_EUNSUPPORTED;
  }
  return gram_stream_go<true>(dtype, k, v, G, G_last, it, nitems, nb, 129, k_sb, k_st, v_sb, v_st,
                              g_sb, g_si, gl_sb, fa, stream, who);
}

// The shapes this kernel serves; everything else runs scan_fused_kernel.
bool scan_stream_ok(int dtype, const void* phi, const void* psi, const void* vb, const float* Y,
                    const float* out, const ScanArgs& a) {
  if (dtype != SMAT_BF16 && dtype != SMAT_F16) return false;
  if (a.write_H || a.r != 128 || a.p != 129) return false;
  if (a.C % ss::kStep || a.T % ss::kStep || a.n % ss::kStep) return false;
  if (!rows_vec_ok(phi, a.q_sb, a.q_st, 2) || !rows_vec_ok(psi, a.k_sb, a.k_st, 2) ||
      !rows_vec_ok(vb, a.v_sb, a.v_st, 2) || a.v_st < 136)
    return false;
  if (!rows_vec_ok(out, a.o_sb, a.o_st, 4)) return false;
  if (Y && !rows_vec_ok(Y, a.y_sb, a.y_st, 4)) return false;
  // per-lane row offsets are 32-bit bytes over 64 rows
  constexpr int64_t kMaxSt = 1 << 20;
  if (a.q_st >= kMaxSt || a.k_st >= kMaxSt || a.v_st >= kMaxSt || a.o_st >= kMaxSt ||
      a.y_st >= kMaxSt)
    return false;
  return variant(SMAT_VARIANT_SCAN) == 0;
}

template <typename In, int FEAT>
static void scan_stream_kernel_launch(const void* phi, const void* psi, const void* vb,
                                      const float* Sg, const float* Y, const float* gate,
                                      float* out, dim3 grid, const ScanArgs& a, const FeatArgs& fa,
                                      hipStream_t stream) {
  const In* q = (const In*)phi;
  const In* k = (const In*)psi;
  const In* v = (const In*)vb;
  if constexpr (FEAT != 0)
    smat::launch((scan_stream_kernel<In, FEAT, FEAT == 2 ? 3 : 2, true>), grid,
                 dim3(ss::kThreads), 0, stream, q, k, v, Sg, Y, gate, out, a, fa);
  else if (Y || gate)
    smat::launch((scan_stream_kernel<In, 0, 3, true>), grid, dim3(ss::kThreads), 0,
                       stream, q, k, v, Sg, Y, gate, out, a, fa);
  else
    smat::launch((scan_stream_kernel<In, 0, 3, false>), grid, dim3(ss::kThreads), 0,
                       stream, q, k, v, Sg, Y, gate, out, a, fa);
}

template <int FEAT>
static int scan_stream_go(int dtype, const void* phi, const void* psi, const void* vb,
                          const float* Sg, const float* Y, const float* gate, float* out, int nb,
                          int ng, const ScanArgs& a, const FeatArgs& fa, hipStream_t stream) {
  dim3 grid((unsigned)ng, (unsigned)nb);
  if (dtype == SMAT_BF16)
    scan_stream_kernel_launch<bf16, FEAT>(phi, psi, vb, Sg, Y, gate, out, grid, a, fa, stream);
  else
    scan_stream_kernel_launch<f16, FEAT>(phi, psi, vb, Sg, Y, gate, out, grid, a, fa, stream);
  return launch_status("smat_causal_scan");
}

int scan_stream_launch(int dtype, const void* phi, const void* psi, const void* vb,
                       const float* Sg, const float* Y, const float* gate, float* out, int nb,
                       int ng, const ScanArgs& a, hipStream_t stream) {
  return scan_stream_go<0>(dtype, phi, psi, vb, Sg, Y, gate, out, nb, ng, a, FeatArgs{},
                           stream);
}

// The streaming causal pass with the feature map in place: q and v are Q
// and V rows (the shapes scan_stream_ok accepts, with V rows of 128); k is
// K rows, or the Psi rows (key gate applied) when psi_formed.
int scan_stream_launch_feat(int dtype, const void* q, const void* k, const void* v,
                            const float* Sg, const float* Y, const float* gate, float* out,
                            int nb, int ng, const ScanArgs& a, const FeatArgs& fa,
                            bool psi_formed, hipStream_t stream) {
  if (psi_formed) return scan_stream_go<2>(dtype, q, k, v, Sg, Y, gate, out, nb, ng, a, fa, stream);
  return scan_stream_go<1>(dtype, q, k, v, Sg, Y, gate, out, nb, ng, a, fa, stream);
}

}  // namespace smat
