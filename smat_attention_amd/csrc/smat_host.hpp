// Host-side helpers shared by the C-ABI entry points: argument checks, the
// per-thread error message, and dtype dispatch.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/smat_hip.h"
#include "smat_common.hpp"

namespace smat {

void set_error(const char* fmt, ...);
void clear_error();

// Kernel variant selected for `which` (SMAT_VARIANT_*, smat_set_variant);
// 0 is the default kernel.  Set only by the explicit test hook, never from
// the environment.
int variant(int which);

// Checked at every entry point before any launch.
#define SMAT_REQUIRE(cond, code, ...)            \
  do {                                           \
    if (!(cond)) {                               \
      ::smat::set_error(__VA_ARGS__);            \
      return (code);                             \
    }                                            \
  } while (0)

// Stage marks of the one-call forwards (smat_set_stage_events): the events a
// launch made now binds to its kernel's start and end, or nulls when no marked
// stage is active on this thread.  Every launch of a marked stage binds the
// stage's event to its end (the stage's last launch wins); no start events.
void stage_launch_events(hipEvent_t* start, hipEvent_t* stop);

// Every kernel launch of the forward's kernels goes through here: with stage
// events active, hipExtLaunchKernelGGL has the launch itself record them, so a
// stage is timed as its kernels run, with no marker between them.
template <typename... Formals, typename... Actuals>
inline void launch(void (*kern)(Formals...), dim3 grid, dim3 block, uint32_t shmem,
                   hipStream_t st, Actuals... args) {
  hipEvent_t a = nullptr, b = nullptr;
  stage_launch_events(&a, &b);
  hipExtLaunchKernelGGL(kern, grid, block, shmem, st, a, b, 0u, args...);
}

inline int launch_status(const char* who) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", who, hipGetErrorString(e));
    return SMAT_ELAUNCH;
  }
  return SMAT_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// True when rows of `elem_bytes`-sized elements starting at p with row stride
// `ld` (elements) and batch stride `sb` can be read in 16-byte groups.
inline bool rows_vec_ok(const void* p, int64_t sb, int64_t ld, int elem_bytes) {
  const int64_t per16 = 16 / elem_bytes;
  return aligned16(p) && (ld % per16 == 0) && (sb % per16 == 0);
}

// True when the 8-element tile loaders (tile8_load / tile8_issue / load8v with
// VEC) may read rows starting at p: rows 16-byte aligned and row and batch
// strides multiples of 8 elements.  Those loaders read a row's last group
// [c0, c0 + 8) whole, up to round_up(ncols, 8), which stays inside the row's
// stride only when the stride is a multiple of 8 elements.  For 16-bit
// elements this is rows_vec_ok; fp32 rows need 32-byte strides (a row of 36
// floats would let the group at column 32 read 4 floats into the next row,
// and past the allocation on the last row).
inline bool rows_vec8_ok(const void* p, int64_t sb, int64_t ld) {
  return aligned16(p) && (ld % 8 == 0) && (sb % 8 == 0);
}

inline int elem_bytes(int dtype) { return dtype == SMAT_F32 ? 4 : 2; }

// Upper bounds of the MFMA tilings.
// Arguments of the causal-pass kernels (scan_fused.hip, scan_stream.hip): chunks
// of C tokens grouped K at a time inside each segment; ng0 groups cover the
// first segment [0, n).
struct ScanArgs {
  int T, n, C, K, nc, nc0, ng0, r, p;
  int64_t q_sb, q_st, k_sb, k_st, v_sb, v_st;
  int64_t y_sb, y_st;   // Y rows are recent rows t - n
  int64_t o_sb, o_st;
  int64_t g_sb;
  int write_H;          // 1: out is H (nb, T, p) unnormalised, no Y / gate
};

// Token progressions summed by the Gram kernels (gram.hip, scan_stream.hip).
struct GramItems {
  int mode;        // 0: chunk groups, 1: profiles (+ optional global channel)
  // mode 0: chunks of width C over T tokens; segment 0 has nc0 chunks; a group
  // is K consecutive chunks inside one segment.
  int T, C, K, nc0, nc, ng0;
  // mode 1: profiles x < N0 over [n_P, n); item N0 is the global channel.
  int n_P, n, N0;
  // split-K: each progression is cut into nsplit runs of `per` terms (a
  // multiple of the 32-token block); run s writes partial s, and a second
  // kernel sums the partials in run order, so the result is deterministic.
  int nsplit, per;
  // mode 2: item i sums the landmark columns cols[i*kappa .. i*kappa + counts[i])
  // (tokens n_P + col): the unpooled (direct) long-range sums of row types.
  // With offs set (CSR), item i's columns are cols[offs[i] .. offs[i+1]).
  const int32_t* cols;
  const int32_t* counts;
  int kappa;
  const int64_t* offs;
};

__device__ __forceinline__ void gram_item(const GramItems& it, int i, int64_t& start,
                                          int64_t& stride, int& count) {
  if (it.mode == 0) {
    int c0, c1;
    if (i < it.ng0) {
      c0 = i * it.K;
      c1 = min(c0 + it.K, it.nc0);
    } else {
      c0 = it.nc0 + (i - it.ng0) * it.K;
      c1 = min(c0 + it.K, it.nc);
    }
    start = (int64_t)c0 * it.C;
    stride = 1;
    const int64_t end = min((int64_t)c1 * it.C, (int64_t)it.T);
    count = (int)max((int64_t)0, end - start);
  } else if (it.mode == 2) {
    start = it.n_P;
    stride = 1;
    count = it.offs ? (int)(it.offs[i + 1] - it.offs[i]) : it.counts[i];
  } else {
    if (i < it.N0) {
      const int nX = it.n - it.n_P;
      start = it.n_P + i;
      stride = it.N0;
      count = (i < nX) ? (nX - i + it.N0 - 1) / it.N0 : 0;
    } else {
      start = 0;
      stride = 1;
      count = it.n_P;
    }
  }
}

// Token of term `idx` of item `item` (start, stride from gram_item).
__device__ __forceinline__ int64_t gram_token(const GramItems& it, int item, int64_t start,
                                              int64_t stride, int idx) {
  if (it.mode == 2)
    return start + it.cols[(it.offs ? it.offs[item] : (int64_t)item * it.kappa) + idx];
  return start + (int64_t)idx * stride;
}

constexpr int kMaxR = 128;
constexpr int kMaxP = 144;
constexpr int kMaxC = 256;

}  // namespace smat
