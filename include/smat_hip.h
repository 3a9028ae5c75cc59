/*
 * smat_hip.h -- C ABI of libsmat_hip.so, the MI355X (gfx950) kernels of the
 * SMat chunkwise schedule.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers; the library never allocates or frees.
 *     Entry points that need scratch memory take a caller-provided workspace
 *     whose size a matching *_workspace_bytes() query returns.
 *   - A matrix argument is (pointer, batch stride, row stride) in ELEMENTS;
 *     its columns are contiguous.  Strides are int64_t.
 *   - `dtype` names the element type of the feature inputs (Phi, Psi, Vb):
 *     SMAT_BF16, SMAT_F16 or SMAT_F32.  Pooled tables, chunk states and
 *     outputs are fp32 (the reference accumulates and returns fp32 for these
 *     inputs, src/smat/attention.py:124-127).
 *   - `stream` is a hipStream_t (NULL: the null stream).  Work is enqueued
 *     only; nothing synchronises the host.
 *   - Return value: SMAT_OK, or a negative code; smat_last_error() then
 *     returns a message naming the entry point and the offending argument.
 *
 * Sizes supported by the MFMA kernels: r <= 128 (feature rank) and
 * p <= 144 (value width + 1); chunk C <= 256.  Larger shapes return
 * SMAT_EUNSUPPORTED rather than running.
 */
#ifndef SMAT_HIP_H
#define SMAT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMAT_OK 0
#define SMAT_EINVAL (-1)
#define SMAT_EUNSUPPORTED (-2)
#define SMAT_ELAUNCH (-3)

#define SMAT_BF16 0
#define SMAT_F16 1
#define SMAT_F32 2

/* Message for the last failing call on this host thread ("" if none). */
const char* smat_last_error(void);

/* Library version and the target it was built for, e.g. "0.1 gfx950". */
const char* smat_version(void);

/*
 * Test hook with no counterpart in the reference: select, process-wide, the
 * general kernel that a specialised one replaced, so that tests can compare
 * the two on the same inputs.  value 1 selects the general kernel, 0 (the
 * default) the specialised one; returns the previous value, or SMAT_EINVAL.
 *   SMAT_VARIANT_SCAN             general fused causal scan instead of the
 *                                 head_dim-128 streaming scan
 *   SMAT_VARIANT_GRAM             general Gram kernel instead of the
 *                                 head_dim-128 streaming pool / prepass
 *   SMAT_VARIANT_QUERY            general query kernel instead of the
 *                                 head_dim-128 streaming query
 *   SMAT_VARIANT_INCIDENCE        L2 gather kernel instead of the LDS panel
 *   SMAT_VARIANT_INCIDENCE_PLANE  line-per-lane generated-line kernel instead
 *                                 of the line-group one
 * Not for production use: a call changes the kernels of every later call.
 */
#define SMAT_VARIANT_SCAN 0
#define SMAT_VARIANT_GRAM 1
#define SMAT_VARIANT_QUERY 2
#define SMAT_VARIANT_INCIDENCE 3
#define SMAT_VARIANT_INCIDENCE_PLANE 4
#define SMAT_NUM_VARIANTS 5
int smat_set_variant(int which, int value);

/*
 * Fused within-chunk pass, one output block per chunk:
 *   out_b = Phi_b Sin_b + (tril(Phi_b Psi_b^T)) Vb_b
 * Phi_b, Psi_b: (C, r) of dtype; Vb_b: (C, p) of dtype; Sin_b: (r, p) fp32;
 * out_b: (C, p) fp32, for b in [0, nbc).  The score tile is rounded to dtype
 * before the product with Vb, as the reference does.
 * Replaces chunk_local, src/smat/kernels/triton_fwd.py:118-152 (kernel
 * :48-115), called at src/smat/attention.py:183,185.
 */
int smat_chunk_local(int dtype, const void* phi, const void* psi, const void* vb,
                     const float* sin, float* out, int64_t nbc, int C, int r, int p,
                     int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                     int64_t v_sb, int64_t v_st, int64_t s_sb, int64_t s_sr,
                     int64_t o_sb, int64_t o_st, void* stream);

/*
 * Chunk summaries D_c = Psi_c^T Vb_c (fp32, (nb, nc, r, p) contiguous) for the
 * chunks of width C of a (nb, T, .) sequence; a ragged last chunk is
 * zero-padded.  Replaces the torch GEMM of src/smat/attention.py:162.
 */
int smat_chunk_states(int dtype, const void* psi, const void* vb, float* D,
                      int nb, int T, int C, int r, int p,
                      int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                      void* stream);

/*
 * Segmented shifted exclusive scan over chunks, one reset at chunk nc0:
 *   Sin[c] = sum_{c' in seg(c), c' < c} D[c']   (seg: [0,nc0) and [nc0,nc))
 * D, Sin: (nb, nc, rp) fp32 contiguous; Sin may not alias D.  A shifted scan,
 * never cumsum-minus-self (src/smat/attention.py:163-179).
 */
int smat_segment_scan(const float* D, float* Sin, int nb, int nc, int nc0, int64_t rp,
                      void* stream);

/*
 * The decayed scan (S_t = a_t S_{t-1} + psi_t vb_t^T, y_t = Phi_t S_t, one
 * reset at chunk nc0), in two entry points over chunks of C rows.
 * Replaces decayed_segmented_scan, src/smat/model.py:41-82 (torch in the
 * reference: :60-68 within chunks, :71-80 across them).
 *
 * smat_decay_scan: Sin[c] = the state entering chunk c,
 *   S <- aC[c] S + D[c] after chunk c, S = 0 at c = nc0;
 * D, Sin: (nb, nc, rp) fp32 contiguous (Sin may not alias D); aC: (nb, nc)
 * fp32, the total decay exp(L_C) of each chunk.
 *
 * smat_chunk_local_decay: as smat_chunk_local with the within-chunk decay:
 *   out_b[m] = exp(L_m) Phi_m Sin_b + sum_{n <= m} exp(L_m - L_n) (Phi_m . Psi_n) Vb_n
 * L: (nbc, C) fp32 contiguous, L_m the running sum of the log-decays of chunk
 * b up to row m.  The masked weights are never formed.
 */
int smat_decay_scan(const float* D, const float* aC, float* Sin, int nb, int nc, int nc0,
                    int64_t rp, void* stream);

/*
 * The gradient of smat_decay_scan, walking the chunks backwards: given dSin
 * (the gradient of every state entering a chunk), dD[c] receives the gradient
 * of the summary D[c]: g = 0; for c = nc-1 .. 0: gn = (c + 1 == nc0 ? 0 : g);
 * dD[c] = gn; g = dSin[c] + aC[c] gn.  Shapes as smat_decay_scan.  Replaces
 * torch autograd through src/smat/model.py:71-80.
 */
int smat_decay_scan_reverse(const float* dSin, const float* aC, float* dD, int nb, int nc,
                            int nc0, int64_t rp, void* stream);
int smat_chunk_local_decay(int dtype, const void* phi, const void* psi, const void* vb,
                           const float* sin, const float* L, float* out, int64_t nbc, int C,
                           int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                           int64_t v_sb, int64_t v_st, int64_t s_sb, int64_t s_sr,
                           int64_t o_sb, int64_t o_st, void* stream);

/*
 * The causal pass fused: segmented chunked scan with one reset at n (chunk
 * C <= 128), then either (write_H = 1) H = [[L_n,0],[0,L_{T_R}]] Phi Psi^T Vb
 * into out (nb, T, p) fp32, or (write_H = 0) the normalised output
 *   out[t, c] = (H[t, c] + Y[t-n, c]) / (H[t, p-1] + Y[t-n, p-1]) * g[t]
 * into out (nb, T, p-1) fp32, the Y term only for t >= n (Y may be NULL, rows
 * y_st apart), g optional.  Reads Phi, Psi, Vb once; H never reaches memory in
 * the normalised mode.  Replaces segmented_causal_scan
 * (src/smat/attention.py:134-192) plus the cat/normalise of :446-453.
 * workspace: smat_causal_scan_workspace_bytes(...) bytes, 256-byte aligned.
 */
int64_t smat_causal_scan_workspace_bytes(int nb, int T, int C, int r, int p);
int smat_causal_scan(int dtype, const void* phi, const void* psi, const void* vb,
                     const float* Y, const float* g, float* out, int nb, int T, int n, int C,
                     int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                     int64_t v_sb, int64_t v_st, int64_t y_sb, int64_t y_st,
                     int64_t o_sb, int64_t o_st, int64_t g_sb, int write_H,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * smat_causal_scan without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  It has no counterpart in the reference.  Arguments and
 * results as smat_causal_scan; its scratch is a fixed array of
 * smat_causal_scan_noalloc_max_bytes() = 64 MiB per GPU, held by the library
 * from its load until the process ends.  When the default grouping of chunks
 * would need more, it sums longer groups of chunks (fewer summaries; the same
 * result up to fp32 rounding), and returns SMAT_EUNSUPPORTED when even one
 * group per segment does not fit (4 * nb * r * p * 4 bytes: nb up to 254
 * sequences at r = 128, p = 129).  It calls no hipMalloc or hipFree.  All
 * calls on one GPU share that GPU's array: calls that overlap there (other
 * streams, other host threads) race.
 */
int64_t smat_causal_scan_noalloc_max_bytes(void);
int smat_causal_scan_noalloc(int dtype, const void* phi, const void* psi, const void* vb,
                             const float* Y, const float* g, float* out, int nb, int T, int n,
                             int C, int r, int p, int64_t q_sb, int64_t q_st, int64_t k_sb,
                             int64_t k_st, int64_t v_sb, int64_t v_st, int64_t y_sb,
                             int64_t y_st, int64_t o_sb, int64_t o_st, int64_t g_sb,
                             int write_H, void* stream);

/*
 * Profile pooling  F_x = sum_{j in [n_P, n), (j - n_P) mod N0 = x} Psi_j^T Vb_j
 * (fp32, F: (nb, N0, r, p) contiguous).  If F_glob is not NULL and n_P > 0 it
 * also receives the global-channel term sum_{j < n_P} Psi_j^T Vb_j, (nb, r, p).
 * Replaces pool, src/smat/kernels/triton_fwd.py:281-311 (kernel :226-267),
 * and the rank-one term of src/smat/attention.py:422-425.  Few, long
 * progressions (small N0, e.g. d = 1 where N0 = 1) are split over several
 * workgroups and summed in a fixed order; that needs
 * smat_pool_workspace_bytes(...) bytes of workspace (0: none needed).
 */
int64_t smat_pool_workspace_bytes(int nb, int n_P, int n, int N0, int r, int p);
int smat_pool(int dtype, const void* psi, const void* vb, float* F, float* F_glob,
              int nb, int n_P, int n, int N0, int r, int p,
              int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
              void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Incidence  U_h = sum_{x in H_h} F_x (+ F_glob when not NULL), fp32.
 * F: (nb, N0, rp) contiguous; U: (nb, B, rp) contiguous.  Row h's points are
 * idx[h*deg .. h*deg+deg) when indptr is NULL (uniform degree), otherwise
 * idx[indptr[h] .. indptr[h+1]).  idx_is_64: 1 if idx holds int64, 0 int32.
 * Replaces incidence, src/smat/kernels/triton_fwd.py:191-216 (kernel
 * :162-188), and the ragged CSR loop of src/smat/attention.py:268-274.
 */
int smat_incidence(const float* F, const float* F_glob, const void* idx, int idx_is_64,
                   const int64_t* indptr, int deg, float* U, int nb, int N0, int B,
                   int64_t rp, void* stream);

/*
 * Incidence for the d = 3 geometric mask with the lines generated in-kernel:
 * row h is the line <a_e, x> = b of F_q^2 given by code[h] = e*q + b, where
 * a_0 = (0, 1), a_e = (1, e-1) for e >= 1, and point x = x0*q + x1.  Same
 * result as smat_incidence on that mask's table (up to fp32 summation order)
 * without reading the table.  F, U, F_glob as for smat_incidence; N0 = q*q.
 * Returns SMAT_EUNSUPPORTED when the F panel does not fit on chip.
 */
int smat_incidence_plane(const float* F, const float* F_glob, const int* code, int q,
                         float* U, int nb, int N0, int B, int64_t rp, void* stream);

/*
 * Type-major query  Y[i] = Phi_rec[i] U_{i mod B}, i in [0, T_R), fp32 out
 * (nb, T_R, p) with row stride y_st.  Phi_rec has dtype; U: (nb, B, r, p).
 * Replaces query_by_type, src/smat/attention.py:310-330.
 */
int smat_query(int dtype, const void* phi_rec, const float* U, float* Y,
               int nb, int T_R, int B, int r, int p,
               int64_t q_sb, int64_t q_st, int64_t y_sb, int64_t y_st, void* stream);

/*
 * Normalise  out[t, c] = (H[t, c] + Y[t-n, c]) / (H[t, p-1] + Y[t-n, p-1]) * g[t]
 * for c < p-1; the Y term only for t >= n (Y may be NULL), g optional (NULL).
 * H: (nb, T, p) fp32; out: (nb, T, p-1) fp32; g: (nb, T) fp32.
 * Replaces the cat + divide + gate of src/smat/attention.py:446-453.
 */
int smat_normalise(const float* H, const float* Y, const float* g, float* out,
                   int nb, int T, int n, int p,
                   int64_t h_sb, int64_t h_st, int64_t y_sb, int64_t y_st,
                   int64_t o_sb, int64_t o_st, int64_t g_sb, void* stream);

/*
 * Reverse segmented exclusive scan (backward pass): Sout[c] = sum of D[c']
 * over c' > c in the same segment ([0, nc0) or [nc0, nc)).  The state that
 * flows backwards through the chunks in the gradient of the causal scan.
 */
int smat_segment_scan_reverse(const float* D, float* Sout, int nb, int nc, int nc0, int64_t rp,
                              void* stream);

/*
 * Backward of out = H[..., :p-1] / H[..., p-1:] * g (g optional):
 * dH[t, c] = dout[t, c] g[t] / H[t, p-1] for c < p-1,
 * dH[t, p-1] = -sum_c dH[t, c] H[t, c] / H[t, p-1], and dg[t] (if dg is not
 * NULL) = sum_c dout[t, c] H[t, c] / H[t, p-1].  dout (nb, T, p-1), H and dH
 * (nb, T, p), each with its own (batch, row) strides, all fp32; dg (nb, T).
 */
int smat_normalise_backward(const float* dout, const float* H, const float* g, float* dH,
                            float* dg, int nb, int T, int p, int64_t o_sb, int64_t o_st,
                            int64_t h_sb, int64_t h_st, int64_t d_sb, int64_t d_st,
                            int64_t g_sb, void* stream);

/*
 * The layer's combine and division with the normaliser floored at eps:
 * N = H + [0; Y] (Y's rows added from row n on; Y (nb, T-n, p) may be NULL),
 * out[t, c] = N[t, c] / max(N[t, p-1], eps) for c < p-1.  H, Y fp32 (nb, T, p);
 * out (nb, T, p-1) of out_dtype (SMAT_F32, SMAT_BF16 or SMAT_F16: the fp32
 * quotient rounded to nearest even), each with its own (batch, row) strides.
 * Replaces torch.cat([H[:, :n], H[:, n:] + Ylr]), H[..., :-1] /
 * H[..., -1:].clamp_min(eps) and the cast .to(x.dtype) of src/smat/model.py:296-300
 * and :317 (eps = 1e-6 there).
 */
int smat_combine_normalise(int out_dtype, const float* H, const float* Y, void* out, int nb,
                           int T, int n, int p, float eps, int64_t h_sb, int64_t h_st,
                           int64_t y_sb, int64_t y_st, int64_t o_sb, int64_t o_st, void* stream);

/*
 * Backward of smat_combine_normalise: dN[t, c] = dout[t, c] / den (c < p-1),
 * dN[t, p-1] = -sum_c dN[t, c] N[t, c] / den, or 0 where N[t, p-1] < eps (the
 * floor passes no gradient), den = max(N[t, p-1], eps).  dN (nb, T, p) is the
 * gradient of H, and its rows from n on are the gradient of Y.  dout of
 * dout_dtype (SMAT_F32, SMAT_BF16 or SMAT_F16), widened to fp32.
 */
int smat_combine_normalise_backward(int dout_dtype, const void* dout, const float* H,
                                    const float* Y, float* dH, int nb, int T, int n, int p,
                                    float eps, int64_t o_sb, int64_t o_st, int64_t h_sb,
                                    int64_t h_st, int64_t y_sb, int64_t y_st, int64_t d_sb,
                                    int64_t d_st, void* stream);

/*
 * Strided batched GEMM on fp32 MFMA (backward pass building block):
 *   C[i] = A[i] . B[i]  (beta = 0)  or  C[i] += A[i] . B[i]  (beta = 1),
 * A[i]: M x K, B[i]: K x N, C[i]: M x N fp32, for i = (i1, i2) in
 * [0, n1) x [0, n2); element (m, k) of A[i] is A[i1*a1 + i2*a2 + m*am + k*ak],
 * likewise B with (b1, b2, bk, bn) and C with (c1, c2, cm, cn).  A and B may
 * be bf16, fp16 or fp32 (dtype_a, dtype_b), widened to fp32.  mask: 0 none,
 * 1 keep entries with m >= n (zero the rest), 2 keep m <= n.  n1*n2 < 65536.
 * The products of the backward pass the reference takes from torch autograd
 * and from the fused kernels of src/smat/kernels/triton_bwd.py:49-237.
 */
int smat_bgemm(int dtype_a, int dtype_b, const void* A, const void* B, float* C, int M, int N,
               int K, int n1, int n2, int64_t a1, int64_t a2, int64_t am, int64_t ak, int64_t b1,
               int64_t b2, int64_t bk, int64_t bn, int64_t c1, int64_t c2, int64_t cm,
               int64_t cn, int beta, int mask, void* stream);

/*
 * Fused backward of the intra-chunk causal scan, one workgroup per
 * (sequence, chunk) with the C x C scores A = tril(Phi Psi^T) and
 * dA = tril(dH Vb^T) kept on chip:
 *   dPhi = dA Psi + dH Sin^T,  dPsi = dA^T Phi + Vb Q^T,  dVb = A^T dH + Psi Q
 * for 16-bit Phi, Psi, Vb (nb x nc*C rows; dtype SMAT_BF16 or SMAT_F16), fp32
 * dH (nb x nc*C x p), the chunk-entry states Sin and the reverse-scan states Q
 * (both nb x nc x r x p, contiguous).  Writes dPhi, dPsi (row stride d_st)
 * and dVb (row stride e_st), strides in elements of out_dtype: SMAT_F32, or
 * dtype itself for gradients rounded to nearest even in the inputs' type;
 * every row of the nc chunks is written.  Serves r = 64, p = 65, C = 128 with
 * 16-byte aligned rows of Phi, Psi, dPhi and dPsi (SMAT_EUNSUPPORTED
 * otherwise).  Optional fp32 terms (NULL: none) are added before the store,
 * rows addressed by absolute index: add_phi (rows ap_st apart, sequences
 * ap_sb) on dPhi rows [add_split, add_end), add_psi (ak_*) and add_vb (av_*)
 * on dPsi and dVb rows [0, add_split) -- the long-range branch's gradients
 * (smat_lr_dphi, smat_pool_backward with accumulate = 0), so that the sum
 * is rounded once.  The products of
 * src/smat/kernels/triton_bwd.py:49-147 (_cl_bwd_dphi_kernel and
 * _cl_bwd_dpsi_dvb_kernel) with the chunk states of attention.py:134-192.
 */
int smat_chunk_backward(int dtype, int out_dtype, const void* phi, const void* psi,
                        const void* vb, const float* dH, const float* Sin, const float* Q,
                        void* dPhi, void* dPsi, void* dVb, int nb, int nc, int r, int p, int C,
                        int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st, int64_t v_sb,
                        int64_t v_st, int64_t h_sb, int64_t h_st, int64_t d_sb, int64_t d_st,
                        int64_t e_sb, int64_t e_st, const float* add_phi, const float* add_psi,
                        const float* add_vb, int64_t ap_sb, int64_t ap_st, int64_t ak_sb,
                        int64_t ak_st, int64_t av_sb, int64_t av_st, int64_t add_split,
                        int64_t add_end, void* stream);

/*
 * The per-chunk state gradient of the causal scan, Dr_c = Phi_c^T dH_c for
 * every (sequence, chunk): fp32 (nb x nc x r x p, contiguous, 16-byte
 * aligned), the input of the reverse scan (smat_segment_scan_reverse) that
 * gives smat_chunk_backward its Q.  16-bit Phi (rows 16-byte aligned), fp32
 * dH (nb x nc*C rows, row stride h_st >= p); products on 16-bit MFMA with dH
 * split hi/lo.  Serves r = 64, p = 65, C = 128 (SMAT_EUNSUPPORTED
 * otherwise).  Part of the gradient of src/smat/attention.py:134-192 (the
 * reference takes it from torch autograd).
 */
int smat_chunk_dstates(int dtype, const void* phi, const float* dH, float* Dr, int nb, int nc,
                       int r, int p, int C, int64_t q_sb, int64_t q_st, int64_t h_sb,
                       int64_t h_st, void* stream);

/*
 * Backward of the long-range branch (attention.py:196-330) at r = 64, p = 65
 * for 16-bit inputs (dtype SMAT_BF16 or SMAT_F16; SMAT_EUNSUPPORTED
 * otherwise); dY is dH on the recent rows, fp32.
 *
 * smat_lr_dphi: dPhi[n + h + k*B] += dH[n + h + k*B] U_h^T for every row type
 * h < B and k with h + k*B < T_R; U fp32 (nb x B x r x p, 16-byte aligned
 * matrices), dPhi fp32 rows 16-byte aligned.  The query's gradient, which
 * the reference takes from torch autograd of attention.py:287-330.
 *
 * smat_lr_dfeat: dF[x] = sum over t in tok[tptr[x] .. tptr[x+1]) of
 * Phi_t^T dH_t (r x p fp32, dF contiguous nb x nitems x r x p).  With
 * the list of point x holding the recent rows of every row type whose
 * hyperplane contains x, this is C^T dU with dU_h the query's parameter
 * gradient: the reference's dU (torch) and incidence backward
 * (src/smat/kernels/triton_bwd.py:262-276) in one pass.
 *
 * smat_pool_backward: for every profile x < N0 and its tokens
 * j = n_P + x + s*N0 < n, dPsi_j += Vb_j dF_x^T and dVb_j += Psi_j dF_x; when
 * n_P > 0, item N0 (dF row N0, the global channel) does tokens 0 .. n_P-1.
 * dF_x is read once for both (src/smat/kernels/triton_bwd.py:203-237).
 *
 * accumulate = 1 adds into dPhi / dPsi / dVb as written above; 0 stores the
 * term itself (every recent row has one row type and every landmark row one
 * profile or the global channel, so each of those rows is written once and
 * the others are left as they are).
 */
int smat_lr_dphi(int dtype, const float* dH, const float* U, float* dPhi, int nb, int T_R, int B,
                 int n, int r, int p, int64_t h_sb, int64_t h_st, int64_t u_sb, int64_t d_sb,
                 int64_t d_st, int accumulate, void* stream);
int smat_lr_dfeat(int dtype, const void* phi, const float* dH, const int32_t* tptr,
                  const int32_t* tok, float* dF, int nb, int nitems, int r, int p, int64_t q_sb,
                  int64_t q_st, int64_t h_sb, int64_t h_st, int64_t f_sb, void* stream);
int smat_pool_backward(int dtype, const void* psi, const void* vb, const float* dF, float* dPsi,
                       float* dVb, int nb, int N0, int n, int n_P, int r, int p, int64_t k_sb,
                       int64_t k_st, int64_t v_sb, int64_t v_st, int64_t f_sb, int64_t d_sb,
                       int64_t d_st, int64_t e_sb, int64_t e_st, int accumulate, void* stream);

/*
 * Gradients of ContentAssign's hard point read and pool (src/smat/assign.py:
 * 431-441 at anneal = 1, whose forward weights are the one-hot of pair 0) at
 * r = 64, p = 65 for 16-bit Phi/Psi/Vb (SMAT_EUNSUPPORTED otherwise).  ent
 * lists, for every (sequence b, cell x), the entries e = pair*L + token of
 * sequence b (L tokens, K pairs each) whose pair points at x, in ascending
 * order (so a cell's pair-0 entries come first):
 * ent[eoffs[b*N0 + x] .. eoffs[b*N0+x+1]), every (token, pair) once.
 *
 * smat_cell_read_backward: for y_i = Phi_i F[cell_i0] and upstream dY (fp32,
 * rows of stride y_st): dPhi_i = F[x] dY_i (pair 0), dw[i*K + k] =
 * Phi_i . (F[x] dY_i) for every entry, dF[x] = sum over pair-0 entries of
 * Phi_i^T dY_i.  Writes the dPhi row of every token with a pair-0 entry,
 * every dw and every dF (fp32).
 *
 * smat_cell_pool_backward: for F[x] = sum_{cell_j0 = x} Psi_j^T Vb_j and dF:
 * dPsi_j = Vb_j dF[x]^T and dVb_j = Psi_j dF[x] (pair 0), dw[j*K + k] =
 * Psi_j . (Vb_j dF[x]^T) for every entry (fp32).
 *
 * Both: dPhi, dPsi and dVb of out_dtype (SMAT_F32, or dtype for gradients
 * rounded to nearest even in the inputs' type; strides in its elements), with
 * batch and row strides of their own, so they may be rows of larger tensors.
 *
 * The reference's autograd of the dense read and pool; its fused pool
 * backward is src/smat/kernels/triton_bwd.py:203-237.
 */
/*
 * Backward of one feature map (attention.py:82-106) at d_qk = r = 64 for
 * 16-bit inputs (SMAT_EUNSUPPORTED otherwise): with y = x W^T (fp32) and G the
 * upstream gradient of the map's output,
 *   g = G * m'(y) * h,  dx = g W (in x's dtype),  dW = sum g^T x (fp32),
 *   dh = sum_f G * m(y) (in h's dtype, when h is not NULL),
 * m = elu + 1 (kind 0) or relu + 1e-3 (kind 1).  dWp is scratch for
 * smat_featurise_backward_parts(nb, T) partial 64 x 64 fp32 sums; dW
 * receives their total (beta = 1 adds it to dW).  The torch autograd of the
 * reference's featurise, one launch and a reduction.
 */
int64_t smat_featurise_backward_parts(int nb, int T);
int smat_featurise_backward(int dtype, const void* x, const void* G, const void* W, const void* h,
                            void* dx, float* dWp, float* dW, void* dh, int nb, int T, int d_qk,
                            int r, int kind, int beta, int64_t x_sb, int64_t x_st, int64_t g_sb,
                            int64_t g_st, int64_t h_sb, int64_t o_sb, int64_t o_st,
                            int64_t dh_sb, void* stream);

int smat_cell_read_backward(int dtype, int out_dtype, const void* phr, const float* dY,
                            const float* F, const int32_t* ent, const int64_t* eoffs, void* dPhi,
                            float* dF, float* dw, int nb, int N0, int K, int L, int r, int p,
                            int64_t q_sb,
                            int64_t q_st, int64_t y_sb, int64_t y_st, int64_t f_sb,
                            int64_t d_sb, int64_t d_st, int64_t w_sb, void* stream);
int smat_cell_pool_backward(int dtype, int out_dtype, const void* psi, const void* vb,
                            const float* dF, const int32_t* ent, const int64_t* eoffs, void* dPsi,
                            void* dVb, float* dw, int nb, int N0, int K, int L, int r, int p,
                            int64_t k_sb,
                            int64_t k_st, int64_t v_sb, int64_t v_st, int64_t f_sb,
                            int64_t d_sb, int64_t d_st, int64_t e_sb, int64_t e_st,
                            int64_t w_sb, void* stream);

/*
 * Whole forward schedule of smat_attention (src/smat/attention.py:391-455) for
 * a geometric mask: pool -> incidence (+ global channel) -> query ->
 * chunk states -> segmented scan -> chunk-local pass -> normalise.
 * idx/indptr/deg describe C as for smat_incidence; B, N0, n, n_P from the spec.
 * idx may be NULL when C is the identity (deg = 1, B = N0, row h = [h]: every
 * d = 2 geometric mask) and n_P = 0: the query then reads F as U and the
 * incidence pass is skipped (U = F exactly, as the gather would give).
 * plane_code/q, when plane_code is not NULL, select smat_incidence_plane's
 * generated lines instead of the table (d = 3 masks).
 * out: (nb, T, p-1) fp32 with row stride o_st; g optional.  H_out, if not
 * NULL, receives the unnormalised H (nb, T, p) fp32 contiguous.
 * workspace: smat_forward_workspace_bytes(...) bytes, 256-byte aligned.
 */
int64_t smat_forward_workspace_bytes(int nb, int T, int n, int N0, int B, int n_P,
                                     int C, int r, int p);

/*
 * Stage marks of smat_forward and smat_forward_fused, for the calling thread.
 * Stage s is 0 the pool, 1 the incidence, 2 the query, 3 the causal pass; with
 * n hipEvent_t handles set, each later call binds events[s] to the end of
 * stage s's last kernel through the launch itself (hipExtLaunchKernelGGL's
 * stop event: no marker packet between kernels), so the time from events[s-1]
 * to events[s] is stage s as the one-call forward runs it, kernels plus the
 * dispatch gaps between them (stage 0: from an event the caller records
 * before the call).  The device-side counterpart of the timer argument of
 * smat_attention (src/smat/attention.py:391-455, whose phases lr_pool,
 * lr_incidence, lr_query and scan + normalise these stages are).  Stages a
 * call does not run (no recent rows) record nothing.  n = 0 clears them; at
 * most 8.  The caller keeps the events alive while they are set.
 */
int smat_set_stage_events(void* const* events, int n);
int smat_forward(int dtype, const void* phi, const void* psi, const void* vb,
                 const void* idx, int idx_is_64, const int64_t* indptr, int deg,
                 const int* plane_code, int q,
                 float* out, float* H_out, const float* g,
                 int nb, int T, int n, int n_P, int N0, int B, int C, int r, int p,
                 int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                 int64_t v_sb, int64_t v_st, int64_t o_sb, int64_t o_st, int64_t g_sb,
                 void* workspace, int64_t workspace_bytes, void* stream);

/*
 * One cached-decode step for nb sequences (SmatDecoder.step,
 * src/smat/attention.py:522-528):
 *   S_out = S_in + Psi_t Vb_t^T;  o = Phi_t (S_out + U[type]);  out = o[:p-1] / o[p-1]
 * S_in, S_out: (nb, r, p) fp32, distinct buffers (the caller swaps them
 * between steps); U: (nb, B, r, p) fp32; the row type is step mod B.
 * Phi_t, Psi_t: (nb, r) and Vb_t: (nb, p) of dtype with batch strides;
 * out: (nb, p-1) fp32.  o_full, if not NULL, receives o (nb, p) fp32.
 */
int smat_decode_step(int dtype, const void* phi_t, const void* psi_t, const void* vb_t,
                     const float* S_in, float* S_out, const float* U, float* out,
                     float* o_full, int nb, int B, int r, int p, int64_t step,
                     int64_t q_sb, int64_t k_sb, int64_t v_sb, void* stream);

/*
 * Unpooled long-range sums  U_h = sum_{j in cols_h} Psi_{n_P+j}^T Vb_{n_P+j}
 * (fp32, U: (nb, B, r, p) contiguous), one row type per list: cols (B, kappa)
 * int32 landmark columns, row h holding its counts[h] columns first.
 * Replaces direct_long_range, src/smat/attention.py:333-362 (the reference
 * pads each list with n_X; this table is the same lists, compacted).
 */
int smat_direct(int dtype, const void* psi, const void* vb, const int32_t* cols,
                const int32_t* counts, int kappa, float* U, int nb, int B, int n_P,
                int r, int p, int64_t k_sb, int64_t k_st, int64_t v_sb, int64_t v_st,
                void* stream);

/*
 * Subset-sum (zeta) transform over N = 2^k profiles:
 *   Z_a = sum_{x subset of a} F_x,   F, Z: (nb, N, rp) fp32, Z may equal F.
 * Replaces zeta_transform, src/smat/attention.py:369-384.
 */
int smat_zeta(const float* F, float* Z, int nb, int N, int64_t rp, void* stream);

/*
 * Walsh incidence of the endpoint mask, C[h, a] = 1{popcount(h & a) even}:
 *   U = (sum_x F_x + H F) / 2, H the N x N Walsh matrix, N = 2^k;
 * F, U: (nb, N, rp) fp32, U may equal F.  Replaces walsh_incidence,
 * src/smat/attention.py:288-307.
 */
int smat_walsh(const float* F, float* U, int nb, int N, int64_t rp, void* stream);

/*
 * U_h <- U_h - sum_x F_x for every row type h (in place; F: (nb, N0, rp),
 * U: (nb, B, rp) fp32).  The negated complement Ubar = F_tot - U of the
 * subtractive schedule, src/smat/attention.py:458-482: querying the result
 * gives -Y_ex, which the normalisation adds.
 */
int smat_incidence_complement(const float* F, float* U, int nb, int N0, int B, int64_t rp,
                              void* stream);

/*
 * Feature map and value packing, src/smat/attention.py:82-106:
 * Phi = map(Q W^T), Psi = map(K W^T) * h, Vb = [V, 1] in the input dtype,
 * map = elu(x) + 1 (kind 0) or relu(x) + 1e-3 (kind 1), with torch's rounding
 * steps (product, map and gate each rounded to the dtype).  Q, K: (nb, T, d_qk)
 * rows, W: (r, d_qk) contiguous, h: (nb, T) or NULL, V: (nb, T, d_v).
 * Phi/Psi rows o_st apart, Vb rows vb_st > d_v apart (the pad is not written).
 * k (with psi) and v (with vb) may be NULL to skip those outputs.
 * d_qk <= 128, r <= 128.
 */
int smat_featurise(int dtype, const void* q, const void* k, const void* v, const void* W,
                   const void* h, void* phi, void* psi, void* vb, int nb, int T, int d_qk,
                   int r, int d_v, int kind, int64_t q_sb, int64_t q_st, int64_t k_sb,
                   int64_t k_st, int64_t v_sb, int64_t v_st, int64_t h_sb, int64_t o_sb,
                   int64_t o_st, int64_t vb_sb, int64_t vb_st, void* stream);

/*
 * Gram sums over token lists (CSR): G[i] = sum_{j in tokens[offs[i] .. offs[i+1])}
 * psi_j^T vb_j, fp32 (nitems, r, p) contiguous; psi / vb are row matrices with
 * row strides k_st / v_st (sequences flattened: token = sequence * T + t).
 * The pool by cell of a content-addressed assignment, src/smat/assign.py:431-436.
 */
int smat_gram_lists(int dtype, const void* psi, const void* vb, const int32_t* tokens,
                    const int64_t* offs, float* G, int nitems, int r, int p,
                    int64_t k_st, int64_t v_st, void* stream);

/*
 * Read by type over row lists (CSR): Y[i] = phi[i] U[h] for every row i in
 * rows[roffs[h] .. roffs[h+1]), h < ntypes.  maxcnt sizes the grid (about the
 * longest list; any value >= 0 is correct: longer lists are walked by the
 * same workgroups), so a caller need not read the list lengths back.
 * U: (ntypes, r, p) fp32, Y rows y_st apart.  The point / plane read of a
 * content-addressed assignment, src/smat/assign.py:437-439, 471-472.
 */
int smat_query_lists(int dtype, const void* phi, const float* U, float* Y,
                     const int32_t* rows, const int64_t* roffs, int ntypes, int maxcnt,
                     int r, int p, int64_t q_st, int64_t y_st, void* stream);

/*
 * smat_forward from Q, K, V with the feature map inside the kernels:
 * Phi = map(Q W^T), Psi = h * map(K W^T), Vb = [V, 1] (map: kind 0 elu + 1,
 * kind 1 relu + 1e-3, torch's rounding steps; h (nb, T) the optional key gate,
 * h_sb its batch stride) are formed in LDS by the pool, the query, the
 * prepass and the scan from the Q, K, V tiles they stream, so Phi and Vb
 * never reach memory (when a row type has more than 64 recent rows, the
 * recent rows' Phi alone is featurised into the workspace for the general
 * query); the causal pass's prepass stores the Psi rows it forms to the
 * workspace and the scan reads them.  W (128 x 128, features x d_qk) in the
 * input dtype.  The other
 * arguments are smat_forward's (no H_out); the workspace is
 * smat_forward_fused_workspace_bytes(nb, T, n, N0, B, n_P, C) bytes.  Serves
 * 16-bit inputs with d_qk = d_v = r = 128, T, n and C multiples of 64
 * (C <= 128) and 16-byte aligned rows; otherwise returns SMAT_EUNSUPPORTED.
 * Replaces featurise (src/smat/attention.py:82-106) followed by smat_attention
 * (:391-455): the fused featurisation that src/smat/kernels/triton_fwd.py
 * leaves to a separate torch pass.
 */
int64_t smat_forward_fused_workspace_bytes(int nb, int T, int n, int N0, int B, int n_P, int C);
int smat_forward_fused(int dtype, const void* q, const void* k, const void* v, const void* W,
                       const void* h, int kind, const void* idx, int idx_is_64,
                       const int64_t* indptr, int deg, const int* plane_code, int field_q,
                       float* out, const float* g, int nb, int T, int n, int n_P, int N0, int B,
                       int C, int64_t q_sb, int64_t q_st, int64_t k_sb, int64_t k_st,
                       int64_t v_sb, int64_t v_st, int64_t h_sb, int64_t o_sb, int64_t o_st,
                       int64_t g_sb, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Class lists (CSR) of every sequence by a counting sort: keys (nb, L) int64 in
 * [0, ncls) -> order (nb*L) int32, the items of sequence 0's class 0, class 1,
 * ..., then sequence 1's, each list in item order (the stable sort of
 * b*ncls + key); an item is b*seq_rows + row0 + l (global_index: the row of a
 * rows [row0, row0 + L) slice of sequences seq_rows rows long; seq_rows = L,
 * row0 = 0 numbers the items b*L + l) or l.  offs (nb*ncls + 1)
 * int64: list (b, c) is order[offs[b*ncls + c] .. offs[b*ncls + c + 1]).
 * workspace: smat_csr_workspace_bytes(nb, L, ncls) bytes.  ncls <= 8192,
 * nb*L < 2^31; keys outside [0, ncls) are clamped into it.  Nothing is read
 * back to the host.  Replaces the torch.argsort / bincount grouping of the
 * cell and type lists, src/smat/assign.py:431-439 and
 * src/smat/kernels/smat_pool_ops.py:158-182.
 */
int64_t smat_csr_workspace_bytes(int nb, int L, int ncls);
int smat_csr_lists(const int64_t* keys, int32_t* order, int64_t* offs, void* workspace, int nb,
                   int L, int ncls, int global_index, int64_t seq_rows, int64_t row0,
                   void* stream);

/*
 * Content hash of token rows u (nb, L, dm; dtype of u): for head h and
 * coordinate k < dim, z = (LN(u) . Wn[h,k]) gamma[h,k] + bias[h,k],
 * s = clamp(q Phi_N(z), 0, q - 1e-4), cell = sum_k floor(s_k) q^(dim-1-k).
 * Wn: (nh, dim, dm) unit rows, fp32.  Outputs s (nb*nh, L, dim) fp32 and
 * cells (nb*nh, L) int64.  Replaces the hard path of ContentAssign._cells,
 * src/smat/assign.py:246-295.
 */
int smat_cell_hash(int dtype, const void* u, const float* Wn, const float* gamma,
                   const float* bias, float* s_out, int64_t* cells, int nb, int L, int dm,
                   int nh, int dim, int q, int64_t u_sb, int64_t u_st, void* stream);

/*
 * The (cell, weight) pairs of the training path at anneal = 1, from the
 * projections z (nb, L, nh*dim) fp32, z = (LN(u) . Wn) gamma + bias: s
 * (nb*nh, L, dim) as smat_cell_hash, the chosen cells (nb*nh, L), the 2^dim
 * pair cells idx (nb*nh, L, 2^dim) (pair p takes the high bin
 * min(floor(s_k) + 1, q - 1) in coordinate k when bit k of p is set) and the
 * soft bin occupancy occ (nb*nh, dim, q): 1 - frac at the low bin plus frac at
 * the high bin, summed over the L tokens.  plant (L,) int64 or null: a cell
 * >= 0 replaces every pair of that token (the planted key columns).
 * dim <= 8, dim*q <= 4096, nh*dim <= 64.  Replaces the pair construction and
 * the occupancy of src/smat/assign.py:257-317 (anneal = 1, no token weights).
 */
int smat_hash_pairs(const float* z, const int64_t* plant, float* s_out, int64_t* cells,
                    int64_t* idx, float* occ, int nb, int L, int nh, int dim, int q,
                    void* stream);

/*
 * Gradient of z (nb, L, nh*dim) fp32 from the gradients of the pairs' weights
 * dw (nb*nh, L, 2^dim) and of the occupancy docc (nb*nh, dim, q), either null,
 * through the straight-through weights of src/smat/assign.py:262-295 at
 * anneal = 1 (forward one-hot on pair 0) and the clamped normal CDF:
 * dz_k = q phi(z_k) [in range] (dw[2^k] - dw[0] + docc[k][hi_k] - docc[k][lo_k]);
 * planted tokens (plant >= 0) take no dw term.  s_fwd is smat_hash_pairs' s.
 */
int smat_hash_pairs_backward(const float* z, const float* s_fwd, const int64_t* plant,
                             const float* dw, const float* docc, float* dz, int nb, int L,
                             int nh, int dim, int q, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SMAT_HIP_H */
