// The whole forward schedule of smat_attention (src/smat/attention.py:391-455)
// for a geometric mask, as one C call that enqueues the kernels on one stream:
//
//   pool (+ global channel)  ->  incidence  ->  type-major query  ->
//   chunk summaries  ->  segmented shifted scan  ->  chunk-local pass  ->
//   normalise (long-range term added for recent rows, optional gate)
//
// The two passes are summed before the single division, as in the reference.
// Scratch lives in the caller's workspace; this file also holds the error
// state and version string of the library.
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "feat_map.hpp"
#include "smat_host.hpp"

namespace smat {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

static std::atomic<int> g_variant[SMAT_NUM_VARIANTS];

int variant(int which) {
  return (which >= 0 && which < SMAT_NUM_VARIANTS)
             ? g_variant[which].load(std::memory_order_relaxed)
             : 0;
}

// defined in the other translation units
int pool_dispatch(int dtype, const void* psi, const void* vb, float* F, float* F_glob, int nb,
                  int n_P, int n, int N0, int r, int p, int64_t k_sb, int64_t k_st, int64_t v_sb,
                  int64_t v_st, float* partials, int64_t partial_bytes, hipStream_t stream,
                  int64_t f_ld);
int64_t pool_workspace_bytes(int nb, int n_P, int n, int N0, int r, int p, bool glob);
int chunk_states_dispatch(int dtype, const void* psi, const void* vb, float* D, int nb, int T,
                          int C, int K, int n, int r, int p, int64_t k_sb, int64_t k_st,
                          int64_t v_sb, int64_t v_st, float* partials, int64_t partial_bytes,
                          hipStream_t stream, int* ngroups_out, int* ng0_out);
int segment_scan_dispatch(const float* D, float* Sin, int nb, int nc, int nc0, int64_t rp,
                          hipStream_t stream);
int chunk_local_dispatch(int dtype, const void* phi, const void* psi, const void* vb,
                         const float* sin, float* out, int64_t nbc, int C, int r, int p,
                         int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                         int64_t v_st, int64_t s_sb, int64_t s_sr, int64_t o_sb, int64_t o_st,
                         hipStream_t stream, const float* L = nullptr);
int incidence_dispatch(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                       const int64_t* indptr, int deg, float* U, int nb, int N0, int B, int64_t rp,
                       hipStream_t stream);
int incidence_plane_dispatch(const float* F, const float* F_glob, const int* code, int q,
                             float* U, int nb, int N0, int B, int64_t rp, int64_t ld,
                             hipStream_t stream);
int64_t incidence_spread_ld(int64_t rp);
int64_t incidence_plane_ld(int q, int N0, int B, int64_t rp);
int query_dispatch(int dtype, const void* phi, const float* U, float* Y, int nb, int T_R, int B,
                   int r, int p, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                   int64_t y_st, hipStream_t stream);
int normalise_dispatch(const float* H, const float* Y, const float* g, float* out, int nb, int T,
                       int n, int p, int64_t h_sb, int64_t h_st, int64_t y_sb, int64_t y_st,
                       int64_t o_sb, int64_t o_st, int64_t g_sb, hipStream_t stream,
                       float eps);

int gram_stream_launch_feat(int dtype, const void* k, const void* v, float* G, float* G_last,
                            const GramItems& it, int nitems, int nb, int64_t k_sb, int64_t k_st,
                            int64_t v_sb, int64_t v_st, int64_t g_sb, int64_t g_si,
                            int64_t gl_sb, const FeatArgs& fa, hipStream_t stream,
                            const char* who);
int query_stream_launch_feat(int dtype, const void* q, const float* U, float* Y, int nb, int T_R,
                             int B, int64_t u_ld, int64_t q_sb, int64_t q_st, int64_t y_sb,
                             int64_t y_st, const FeatArgs& fa, hipStream_t stream);
int causal_scan_run_feat(int dtype, const void* q, const void* k, const void* v, const float* Y,
                         const float* gate, float* out, int nb, int T, int n, int C,
                         int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                         int64_t v_st, int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st,
                         int64_t g_sb, const FeatArgs& fa, void* ws, int64_t ws_bytes,
                         void* psi_buf, float* F_out, int64_t f_sb, int phases,
                         hipStream_t stream);
int64_t causal_scan_workspace_bytes(int nb, int T, int C, int r, int p);
int causal_scan_dispatch(int dtype, const void* phi, const void* psi, const void* vb,
                         const float* Y, const float* gate, float* out, int nb, int T, int n,
                         int C, int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb,
                         int64_t k_st, int64_t v_sb, int64_t v_st, int64_t y_sb, int64_t y_st,
                         int64_t o_sb, int64_t o_st, int64_t g_sb, int write_H, void* ws,
                         int64_t ws_bytes, hipStream_t stream, float* F_out = nullptr,
                         int64_t f_sb = 0, int phases = 3);

// Workspace carve-up, each region 256-byte aligned.  The fused causal pass
// (chunk <= 128, no H requested) needs only its group states; the staged one
// keeps the per-chunk summaries, their scan and H.
struct FwdLayout {
  int64_t F, Fg, U, Y, D, Sin, H, part, scan, total;
  bool fused;
};

static inline int64_t al256(int64_t x) { return (x + 255) & ~(int64_t)255; }
// Row stride of the long-range term Y: 16-byte rows for vector access.
static inline int64_t y_stride(int p) { return (p + 3) & ~3; }

static FwdLayout fwd_layout(int nb, int T, int n, int N0, int B, int n_P, int C, int r, int p,
                            bool want_H) {
  FwdLayout L{};
  const int64_t rp = (int64_t)r * p;
  const int nc = (T + C - 1) / C;
  const int T_R = T - n;
  L.fused = (C <= 128) && !want_H;
  int64_t off = 0;
  // F and U rows are sized for the spread row stride, which the forward
  // takes when the line-group or row-group incidence runs (rp otherwise).
  const int64_t ld = incidence_spread_ld(rp);
  L.F = off;   off += al256((int64_t)nb * N0 * ld * 4);
  L.Fg = off;  off += n_P > 0 ? al256((int64_t)nb * rp * 4) : 0;
  L.U = off;   off += al256((int64_t)nb * B * ld * 4);
  L.Y = off;   off += al256((int64_t)nb * T_R * y_stride(p) * 4);
  if (L.fused) {
    L.scan = off; off += al256(causal_scan_workspace_bytes(nb, T, C, r, p));
  } else {
    L.D = off;   off += al256((int64_t)nb * nc * rp * 4);
    L.Sin = off; off += al256((int64_t)nb * nc * rp * 4);
    L.H = off;   off += al256((int64_t)nb * nc * C * p * 4);
  }
  L.part = off; off += al256(pool_workspace_bytes(nb, n_P, n, N0, r, p, n_P > 0));
  L.total = off;
  return L;
}

}  // namespace smat

// Stage marks of the one-call forwards (smat_set_stage_events): for stage s
// (0 pool, 1 incidence, 2 query, 3 causal pass) events[s], bound by the
// stage's kernel launches to the end of its last kernel (smat::launch), for
// the calling thread.
namespace smat {

constexpr int kMaxStageMarks = 8;
static thread_local hipEvent_t g_marks[kMaxStageMarks];
static thread_local int g_nmarks = 0;
static thread_local int g_stage = -1;          // the marked stage running now, or -1

void stage_launch_events(hipEvent_t* start, hipEvent_t* stop) {
  *start = nullptr;
  *stop = (g_stage >= 0 && g_stage < g_nmarks) ? g_marks[g_stage] : nullptr;
}

// Marks the kernels launched during its lifetime as stage `s`.
struct StageScope {
  explicit StageScope(int s) { g_stage = s; }
  ~StageScope() { g_stage = -1; }
};

}  // namespace smat

extern "C" const char* smat_last_error(void) { return smat::g_err; }

extern "C" int smat_set_stage_events(void* const* events, int n) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(n >= 0 && n <= kMaxStageMarks && (n == 0 || events), SMAT_EINVAL,
               "smat_set_stage_events: need 0 <= n <= %d events", kMaxStageMarks);
  for (int i = 0; i < kMaxStageMarks; ++i) g_marks[i] = i < n ? (hipEvent_t)events[i] : nullptr;
  g_nmarks = n;
  g_stage = -1;
  return SMAT_OK;
}

extern "C" const char* smat_version(void) { return "0.1 gfx950"; }

extern "C" int smat_set_variant(int which, int value) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(which >= 0 && which < SMAT_NUM_VARIANTS, SMAT_EINVAL,
               "smat_set_variant: unknown variant selector %d", which);
  SMAT_REQUIRE(value == 0 || value == 1, SMAT_EINVAL,
               "smat_set_variant: value must be 0 or 1, got %d", value);
  return g_variant[which].exchange(value);
}

extern "C" int64_t smat_forward_workspace_bytes(int nb, int T, int n, int N0, int B, int n_P,
                                                int C, int r, int p) {
  if (nb <= 0 || T <= 0 || C <= 0 || N0 <= 0 || B <= 0 || r <= 0 || p <= 0) return 0;
  const smat::FwdLayout a = smat::fwd_layout(nb, T, n, N0, B, n_P, C, r, p, false);
  const smat::FwdLayout b = smat::fwd_layout(nb, T, n, N0, B, n_P, C, r, p, true);
  return a.total > b.total ? a.total : b.total;
}

extern "C" int smat_forward(int dtype, const void* phi, const void* psi, const void* vb,
                            const void* idx, int idx_is_64, const int64_t* indptr, int deg,
                            const int* plane_code, int q,
                            float* out, float* H_out, const float* g, int nb, int T, int n,
                            int n_P, int N0, int B, int C, int r, int p, int64_t q_sb,
                            int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                            int64_t o_sb, int64_t o_st, int64_t g_sb, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(phi && psi && vb && out && workspace, SMAT_EINVAL, "smat_forward: null pointer");
  SMAT_REQUIRE(idx || (deg == 1 && B == N0 && n_P == 0), SMAT_EINVAL,
               "smat_forward: idx may be NULL only for the identity incidence (deg=1, B=N0, "
               "n_P=0; got deg=%d B=%d N0=%d n_P=%d)", deg, B, N0, n_P);
  SMAT_REQUIRE(dtype == SMAT_BF16 || dtype == SMAT_F16 || dtype == SMAT_F32, SMAT_EINVAL,
               "smat_forward: unknown dtype %d", dtype);
  SMAT_REQUIRE(nb >= 1 && T >= 1 && C >= 1 && C <= kMaxC, SMAT_EINVAL,
               "smat_forward: bad sizes (nb=%d T=%d C=%d)", nb, T, C);
  SMAT_REQUIRE(n >= 0 && n <= T && n % C == 0, SMAT_EINVAL,
               "smat_forward: landmark count n=%d must be a multiple of chunk=%d in [0, T]", n, C);
  SMAT_REQUIRE(n_P >= 0 && n_P <= n && N0 >= 1 && B >= 1, SMAT_EINVAL,
               "smat_forward: bad mask sizes (n_P=%d N0=%d B=%d)", n_P, N0, B);
  SMAT_REQUIRE(r >= 1 && r <= kMaxR && p >= 2 && p <= kMaxP, SMAT_EUNSUPPORTED,
               "smat_forward: r=%d p=%d beyond r<=%d, 2<=p<=%d", r, p, kMaxR, kMaxP);
  SMAT_REQUIRE(q_st >= r && k_st >= r && v_st >= p && o_st >= p - 1, SMAT_EINVAL,
               "smat_forward: a row stride is shorter than its row");
  SMAT_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, SMAT_EINVAL,
               "smat_forward: workspace must be 256-byte aligned");
  const FwdLayout L = fwd_layout(nb, T, n, N0, B, n_P, C, r, p, H_out != nullptr);
  SMAT_REQUIRE(workspace_bytes >= L.total, SMAT_EINVAL,
               "smat_forward: workspace of %lld bytes needed, %lld given", (long long)L.total,
               (long long)workspace_bytes);

  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  float* F = (float*)(ws + L.F);
  float* Fg = n_P > 0 ? (float*)(ws + L.Fg) : nullptr;
  float* U = (float*)(ws + L.U);
  float* Y = (float*)(ws + L.Y);
  float* part = (float*)(ws + L.part);
  const int64_t part_bytes = L.total - L.part;
  const int64_t rp = (int64_t)r * p;
  const int nc = (T + C - 1) / C;
  const int T_R = T - n;
  const int64_t yst = y_stride(p);
  int rc;

  // One profile holding every landmark token (d = 1, no global channel, the
  // identity incidence): its pool is the sum of the causal pass's group sums
  // over the tokens [0, n), so the causal pass's summaries run first and no
  // pool pass is made.
  // (the group sums are added as float4, so r*p is a multiple of 4)
  const bool pool_from_prepass =
      L.fused && T_R > 0 && !idx && N0 == 1 && n_P == 0 && n > 0 && rp % 4 == 0;

  // ---- long range: S^T, then C, then R ---------------------------------
  if (T_R > 0) {
    // With no profiled landmark columns (n == n_P) every U_h is the global
    // channel alone (or zero): the incidence runs with an empty row.
    const bool profiled = n > n_P;
    const char* phi_rec = (const char*)phi + (int64_t)n * q_st * elem_bytes(dtype);
    // row stride of F and U
    const int64_t ld = idx && plane_code && profiled ? incidence_plane_ld(q, N0, B, rp) : rp;
    {
      StageScope stage(0);
      if (pool_from_prepass)
        rc = causal_scan_dispatch(dtype, phi, psi, vb, nullptr, g, out, nb, T, n, C, r, p, q_sb,
                                  q_st, k_sb, k_st, v_sb, v_st, (int64_t)T_R * yst, yst, o_sb,
                                  o_st, g_sb, 0, ws + L.scan, L.part - L.scan, st, F, ld, 1);
      else
        rc = pool_dispatch(dtype, psi, vb, F, Fg, nb, n_P, n, N0, r, p, k_sb, k_st, v_sb, v_st,
                           part, part_bytes, st, ld);
    }
    if (rc) return rc;
    const float* Uq = U;
    {
      StageScope stage(1);
      if (!idx)                                      // identity incidence: U = F
        Uq = F;
      else if (plane_code && profiled)
        rc = incidence_plane_dispatch(F, Fg, plane_code, q, U, nb, N0, B, rp, ld, st);
      else
        rc = incidence_dispatch(F, Fg, idx, idx_is_64, profiled ? indptr : nullptr,
                                profiled ? deg : 0, U, nb, N0, B, rp, st);
    }
    if (rc) return rc;
    {
      StageScope stage(2);
      rc = query_dispatch(dtype, phi_rec, Uq, Y, nb, T_R, B, r, p, ld, q_sb, q_st,
                          (int64_t)T_R * yst, yst, st);
    }
    if (rc) return rc;
  }

  // ---- causal pass ------------------------------------------------------
  StageScope stage(3);
  if (L.fused) {
    // one kernel: segmented scan, + Y on recent rows, normalise, gate
    return causal_scan_dispatch(dtype, phi, psi, vb, T_R > 0 ? Y : nullptr, g, out, nb, T, n, C,
                                r, p, q_sb, q_st, k_sb, k_st, v_sb, v_st, (int64_t)T_R * yst, yst,
                                o_sb, o_st, g_sb, 0, ws + L.scan, L.part - L.scan, st, nullptr,
                                0, pool_from_prepass ? 2 : 3);
  }
  // staged: chunk summaries, segmented scan, chunk-local pass into H, normalise
  float* D = (float*)(ws + L.D);
  float* Sin = (float*)(ws + L.Sin);
  // H in (nb, nc*C, p) fp32: the caller's H_out is (nb, T, p), which is the
  // same layout for every row the chunk pass writes (rows >= T are skipped).
  float* H = H_out ? H_out : (float*)(ws + L.H);
  rc = chunk_states_dispatch(dtype, psi, vb, D, nb, T, C, 1, n, r, p, k_sb, k_st, v_sb, v_st,
                             nullptr, 0, st, nullptr, nullptr);
  if (rc) return rc;
  rc = segment_scan_dispatch(D, Sin, nb, nc, n / C, rp, st);
  if (rc) return rc;
  // Chunk b of sequence s covers rows [b*C, b*C + C).  When every sequence is
  // a whole number of chunks laid out back to back, all nb*nc chunks form one
  // batch; otherwise each sequence runs its full chunks and its ragged tail
  // chunk (rows [nfull*C, T), zero-padded like the reference) separately.
  const int nfull = T / C;
  const int64_t h_sb = H_out ? (int64_t)T * p : (int64_t)nc * C * p;
  const int eb = elem_bytes(dtype);
  if (T % C == 0 && q_sb == (int64_t)T * q_st && k_sb == (int64_t)T * k_st &&
      v_sb == (int64_t)T * v_st) {
    rc = chunk_local_dispatch(dtype, phi, psi, vb, Sin, H, (int64_t)nb * nc, C, r, p, C * q_st,
                              q_st, C * k_st, k_st, C * v_st, v_st, rp, p, (int64_t)C * p, p, st);
    if (rc) return rc;
  } else {
    for (int s = 0; s < nb; ++s) {
      const char* phs = (const char*)phi + s * q_sb * eb;
      const char* pss = (const char*)psi + s * k_sb * eb;
      const char* vbs = (const char*)vb + s * v_sb * eb;
      float* Hs = H + s * h_sb;
      const float* Ss = Sin + (int64_t)s * nc * rp;
      if (nfull > 0) {
        rc = chunk_local_dispatch(dtype, phs, pss, vbs, Ss, Hs, nfull, C, r, p, C * q_st, q_st,
                                  C * k_st, k_st, C * v_st, v_st, rp, p, (int64_t)C * p, p, st);
        if (rc) return rc;
      }
      if (nfull < nc) {
        const int Ct = T - nfull * C;
        const int64_t t0 = (int64_t)nfull * C;
        rc = chunk_local_dispatch(dtype, phs + t0 * q_st * eb, pss + t0 * k_st * eb,
                                  vbs + t0 * v_st * eb, Ss + (int64_t)nfull * rp, Hs + t0 * p, 1,
                                  Ct, r, p, 0, q_st, 0, k_st, 0, v_st, 0, p, 0, p, st);
        if (rc) return rc;
      }
    }
  }
  return normalise_dispatch(H, T_R > 0 ? Y : nullptr, g, out, nb, T, n, p, h_sb, p,
                            (int64_t)T_R * yst, yst, o_sb, o_st, g_sb, st, -1.f);
}

extern "C" int smat_featurise(int dtype, const void* q, const void* k, const void* v,
                              const void* W, const void* h, void* phi, void* psi, void* vb,
                              int nb, int T, int d_qk, int r, int d_v, int kind, int64_t q_sb,
                              int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                              int64_t v_st, int64_t h_sb, int64_t o_sb, int64_t o_st,
                              int64_t vb_sb, int64_t vb_st, void* stream);

namespace smat {
// More recent rows a row type than the streaming query's 64: the recent rows'
// Phi is featurised into the workspace and read by the general query kernel.
static bool fused_query_staged(int T, int n, int B) {
  return T > n && (T - n + B - 1) / B > 64;
}
// Beyond the forward's layout: the staged recent Phi rows (if any), then the
// Psi rows the prepass forms and the scan reads (nb x T rows of 128).
static int64_t fused_phi_bytes(int nb, int T, int n, int B) {
  return fused_query_staged(T, n, B) ? al256((int64_t)nb * (T - n) * 128 * 2) : 0;
}
static int64_t fused_workspace_bytes(int nb, int T, int n, int N0, int B, int n_P, int C) {
  const FwdLayout L = fwd_layout(nb, T, n, N0, B, n_P, C, 128, 129, false);
  return L.total + fused_phi_bytes(nb, T, n, B) + al256((int64_t)nb * T * 128 * 2);
}
}  // namespace smat

extern "C" int64_t smat_forward_fused_workspace_bytes(int nb, int T, int n, int N0, int B,
                                                      int n_P, int C) {
  if (nb <= 0 || T <= 0 || C <= 0 || N0 <= 0 || B <= 0 || n < 0 || n > T) return 0;
  return smat::fused_workspace_bytes(nb, T, n, N0, B, n_P, C);
}

// The forward of smat_forward computed from Q, K, V: the feature map
// Phi = map(Q W^T), Psi = h map(K W^T), Vb = [V, 1] (src/smat/attention.py:82-106)
// runs inside the pool, the query, the prepass and the scan, on tiles already
// in LDS, so Phi and Vb are never written to memory -- except, when a row
// type has more than 64 recent rows (beyond the streaming query), the recent
// rows' Phi, which is featurised into the workspace for the general query
// kernel.  Psi is formed once, by the causal pass's prepass, which stores it
// to the workspace for the scan.  Serves the head-dim-128 streaming shape: 16-bit inputs,
// d_qk = d_v = r = 128 (p = 129), T, n and the chunk multiples of 64
// (chunk <= 128), 16-byte aligned rows; anything else returns
// SMAT_EUNSUPPORTED (the caller featurises, then calls smat_forward).
extern "C" int smat_forward_fused(int dtype, const void* q, const void* k, const void* v,
                                  const void* W, const void* h, int kind, const void* idx,
                                  int idx_is_64, const int64_t* indptr, int deg,
                                  const int* plane_code, int field_q, float* out, const float* g,
                                  int nb, int T, int n, int n_P, int N0, int B, int C,
                                  int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                                  int64_t v_sb, int64_t v_st, int64_t h_sb, int64_t o_sb,
                                  int64_t o_st, int64_t g_sb, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  using namespace smat;
  clear_error();
  constexpr int r = 128, p = 129;
  SMAT_REQUIRE(q && k && v && W && out && workspace, SMAT_EINVAL,
               "smat_forward_fused: null pointer");
  SMAT_REQUIRE(idx || (deg == 1 && B == N0 && n_P == 0), SMAT_EINVAL,
               "smat_forward_fused: idx may be NULL only for the identity incidence");
  SMAT_REQUIRE(kind == 0 || kind == 1, SMAT_EINVAL, "smat_forward_fused: kind must be 0 or 1");
  SMAT_REQUIRE(nb >= 1 && T >= 1 && n >= 0 && n <= T && n_P >= 0 && n_P <= n && N0 >= 1 &&
                   B >= 1,
               SMAT_EINVAL, "smat_forward_fused: bad sizes (nb=%d T=%d n=%d n_P=%d N0=%d B=%d)",
               nb, T, n, n_P, N0, B);
  const int T_R = T - n;
  constexpr int64_t kMaxSt = 1 << 20;
  SMAT_REQUIRE(dtype == SMAT_BF16 || dtype == SMAT_F16, SMAT_EUNSUPPORTED,
               "smat_forward_fused: 16-bit inputs only");
  SMAT_REQUIRE(C >= 64 && C <= 128 && C % 64 == 0 && T % 64 == 0 && n % C == 0,
               SMAT_EUNSUPPORTED,
               "smat_forward_fused: T, n and the chunk (64 or 128) must be multiples of 64");
  SMAT_REQUIRE(q_st >= 128 && k_st >= 128 && v_st >= 128 && o_st >= 128 && q_st < kMaxSt &&
                   k_st < kMaxSt && v_st < kMaxSt && o_st < kMaxSt,
               SMAT_EUNSUPPORTED, "smat_forward_fused: row strides must be in [128, 2^20)");
  SMAT_REQUIRE(rows_vec_ok(q, q_sb, q_st, 2) && rows_vec_ok(k, k_sb, k_st, 2) &&
                   rows_vec_ok(v, v_sb, v_st, 2) && rows_vec_ok(out, o_sb, o_st, 4) &&
                   aligned16(W),
               SMAT_EUNSUPPORTED, "smat_forward_fused: rows and W must be 16-byte aligned");
  SMAT_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, SMAT_EINVAL,
               "smat_forward_fused: workspace must be 256-byte aligned");
  const FwdLayout L = fwd_layout(nb, T, n, N0, B, n_P, C, r, p, false);
  const int64_t need = fused_workspace_bytes(nb, T, n, N0, B, n_P, C);
  SMAT_REQUIRE(workspace_bytes >= need, SMAT_EINVAL,
               "smat_forward_fused: workspace of %lld bytes needed, %lld given",
               (long long)need, (long long)workspace_bytes);

  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  float* F = (float*)(ws + L.F);
  float* Fg = n_P > 0 ? (float*)(ws + L.Fg) : nullptr;
  float* U = (float*)(ws + L.U);
  float* Y = (float*)(ws + L.Y);
  const int64_t rp = (int64_t)r * p;
  const int64_t yst = y_stride(p);
  const FeatArgs fa{W, h, h_sb, kind};
  int rc;

  void* psi_rows = ws + L.total + fused_phi_bytes(nb, T, n, B);
  // One profile holding every landmark token (d = 1, no global channel, the
  // identity incidence): its pool is the sum of the causal pass's group sums
  // over the tokens [0, n), so the prepass runs first and no pool pass is made.
  const bool pool_from_prepass = T_R > 0 && !idx && N0 == 1 && n_P == 0 && n > 0;
  if (T_R > 0) {
    const bool profiled = n > n_P;
    // row stride of F and U
    const int64_t ld =
        idx && plane_code && profiled ? incidence_plane_ld(field_q, N0, B, rp) : rp;
    if (pool_from_prepass) {
      StageScope stage(0);
      rc = causal_scan_run_feat(dtype, q, k, v, nullptr, g, out, nb, T, n, C, q_sb, q_st, k_sb,
                                k_st, v_sb, v_st, (int64_t)T_R * yst, yst, o_sb, o_st, g_sb, fa,
                                ws + L.scan, L.part - L.scan, psi_rows, F, ld, 1, st);
    } else {
      GramItems it{};
      it.mode = 1;
      it.n_P = n_P;
      it.n = n;
      it.N0 = N0;
      it.nsplit = 1;
      it.per = 1 << 30;
      StageScope stage(0);
      rc = gram_stream_launch_feat(dtype, k, v, F, Fg, it, N0 + (Fg ? 1 : 0), nb, k_sb, k_st,
                                   v_sb, v_st, (int64_t)N0 * ld, ld, rp, fa, st,
                                   "smat_forward_fused");
    }
    if (rc) return rc;
    const float* Uq = U;
    {
      StageScope stage(1);
      if (!idx)
        Uq = F;
      else if (plane_code && profiled)
        rc = incidence_plane_dispatch(F, Fg, plane_code, field_q, U, nb, N0, B, rp, ld, st);
      else
        rc = incidence_dispatch(F, Fg, idx, idx_is_64, profiled ? indptr : nullptr,
                                profiled ? deg : 0, U, nb, N0, B, rp, st);
    }
    if (rc) return rc;
    const char* q_rec = (const char*)q + (int64_t)n * q_st * 2;
    {
      StageScope stage(2);
      if (fused_query_staged(T, n, B)) {
        void* phi_rec = ws + L.total;                // (nb, T_R, 128), rows of 128
        rc = smat_featurise(dtype, q_rec, nullptr, nullptr, W, nullptr, phi_rec, nullptr,
                            nullptr, nb, T_R, 128, 128, 0, kind, q_sb, q_st, 0, 0, 0, 0, 0,
                            (int64_t)T_R * 128, 128, 0, 0, stream);
        if (rc == SMAT_OK)
          rc = query_dispatch(dtype, phi_rec, Uq, Y, nb, T_R, B, r, p, ld, (int64_t)T_R * 128,
                              128, (int64_t)T_R * yst, yst, st);
      } else {
        rc = query_stream_launch_feat(dtype, q_rec, Uq, Y, nb, T_R, B, ld, q_sb, q_st,
                                      (int64_t)T_R * yst, yst, fa, st);
      }
    }
    if (rc) return rc;
  }
  StageScope stage(3);
  return causal_scan_run_feat(dtype, q, k, v, T_R > 0 ? Y : nullptr, g, out, nb, T, n, C, q_sb,
                              q_st, k_sb, k_st, v_sb, v_st, (int64_t)T_R * yst, yst, o_sb, o_st,
                              g_sb, fa, ws + L.scan, L.part - L.scan, psi_rows, nullptr, 0,
                              pool_from_prepass ? 2 : 3, st);
}
