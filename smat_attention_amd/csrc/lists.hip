// Per-sequence class lists (CSR) by a counting sort: for keys (nb, L) in
// [0, ncls) -- the cell or row type of every token, or of every (token, pair)
// entry -- the items of each (sequence, class) in item order, and the offsets
// of each list.  This is the grouping the reference gets from torch.argsort /
// bincount over ``b * ncls + key`` before its list reads and pools
// (src/smat/assign.py:431-439, src/smat/kernels/smat_pool_ops.py:158-182).
//
// Three launches, none of which reads anything back to the host:
//   1. count: a histogram of each tile of items (LDS atomics);
//   2. scan:  per sequence, the class totals' exclusive scan gives the list
//             offsets, and a running sum over tiles each tile's base per class;
//   3. place: one wave per tile walks its items 64 at a time in order; a
//             lane's rank among the earlier lanes with its key comes from
//             ballots over the key's bits, so the order within a list is the
//             item order (the stable sort's).
// The class totals of a sequence sum to L, so sequence b's lists fill
// [b L, (b + 1) L) of the order.  Keys outside [0, ncls) are clamped into it
// (a caller error yields wrong lists, never an access outside the buffers).
#include "smat_host.hpp"

namespace smat {

namespace cs {
constexpr int kMinTile = 512;     // items per tile, while the tile counts stay small
constexpr int kMaxCls = 8192;     // classes per sequence (LDS table of ints)
constexpr int kThreads = 256;
constexpr int64_t kCountBudget = 1 << 22;   // tile counts per sequence (ints)
}  // namespace cs

// Items per tile: 512, doubled while a sequence's tile counts (tiles x
// classes) exceed 4 Mi ints.  Shorter tiles make more, shorter placement
// chains (one wave walks a tile 64 items at a time); the counts bound the
// workspace and the scan's walk over tiles.
static int csr_tile(int L, int ncls) {
  int tile = cs::kMinTile;
  while (tile < (1 << 20) && (int64_t)((L + tile - 1) / tile) * ncls > cs::kCountBudget)
    tile *= 2;
  return tile;
}

__device__ __forceinline__ int clamp_key(int64_t k, int ncls) {
  return k < 0 ? 0 : (k >= ncls ? ncls - 1 : (int)k);
}

// offs[0] = 0 for an empty batch (nb = 0: one offset, no lists).
__global__ __launch_bounds__(64) void csr_empty_kernel(int64_t* __restrict__ offs) {
  if (threadIdx.x == 0) offs[0] = 0;
}

// counts[(b * ntiles + t) * ncls + c] = items of tile t of sequence b with key c.
__global__ __launch_bounds__(cs::kThreads) void csr_count_kernel(const int64_t* __restrict__ keys,
                                                                 int* __restrict__ counts, int L,
                                                                 int ncls, int ntiles, int tile) {
  extern __shared__ int hist[];                      // ncls ints
  const int t = blockIdx.x, b = blockIdx.y;
  for (int c = threadIdx.x; c < ncls; c += cs::kThreads) hist[c] = 0;
  __syncthreads();
  const int64_t* kb = keys + (int64_t)b * L;
  const int i0 = t * tile, i1 = min(L, i0 + tile);
  for (int i = i0 + threadIdx.x; i < i1; i += cs::kThreads)
    atomicAdd(&hist[clamp_key(kb[i], ncls)], 1);
  __syncthreads();
  int* cb = counts + ((int64_t)b * ntiles + t) * ncls;
  for (int c = threadIdx.x; c < ncls; c += cs::kThreads) cb[c] = hist[c];
}

// Per sequence: offs[b * ncls + c] = b L + (items of classes < c), offs[nb * ncls] =
// nb L; counts become each tile's base: offs + items of the class in earlier tiles.
__global__ __launch_bounds__(cs::kThreads) void csr_scan_kernel(int* __restrict__ counts,
                                                                int64_t* __restrict__ offs, int nb,
                                                                int L, int ncls, int ntiles) {
  __shared__ int tot[cs::kMaxCls];
  __shared__ int wsum[cs::kThreads / 64];
  const int b = blockIdx.x;
  int* cb = counts + (int64_t)b * ntiles * ncls;
  for (int c = threadIdx.x; c < ncls; c += cs::kThreads) {
    int s = 0;
    for (int t = 0; t < ntiles; ++t) s += cb[(int64_t)t * ncls + c];
    tot[c] = s;
  }
  __syncthreads();
  // exclusive scan of tot over classes: each thread a contiguous run, then the
  // runs' sums scanned across the workgroup
  const int per = (ncls + cs::kThreads - 1) / cs::kThreads;
  const int c0 = threadIdx.x * per, c1 = min(ncls, c0 + per);
  int run = 0;
  for (int c = c0; c < c1; ++c) run += tot[c];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = run;
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int before = incl - run;
  for (int k = 0; k < w; ++k) before += wsum[k];
  __syncthreads();                                   // every tot[] read above is done
  const int64_t base = (int64_t)b * L;
  for (int c = c0; c < c1; ++c) {
    const int v = tot[c];
    tot[c] = before;
    before += v;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < ncls; c += cs::kThreads) {
    offs[(int64_t)b * ncls + c] = base + tot[c];
    int acc = tot[c];
    for (int t = 0; t < ntiles; ++t) {
      const int v = cb[(int64_t)t * ncls + c];
      cb[(int64_t)t * ncls + c] = acc;
      acc += v;
    }
  }
  if (b == nb - 1 && threadIdx.x == 0) offs[(int64_t)nb * ncls] = (int64_t)nb * L;
}

// One wave per tile: order[b L + base(c) + rank] = item (b seq_rows + row0 + i
// with glob, else i), items taken in order 64 at a time; bases are relative
// to b L.
__global__ __launch_bounds__(64) void csr_place_kernel(const int64_t* __restrict__ keys,
                                                       const int* __restrict__ bases,
                                                       int32_t* __restrict__ order, int L,
                                                       int ncls, int ntiles, int tile, int nbits,
                                                       int glob, int64_t seq_rows, int64_t row0) {
  extern __shared__ int next[];                      // ncls ints
  const int t = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int* bb = bases + ((int64_t)b * ntiles + t) * ncls;
  for (int c = lane; c < ncls; c += 64) next[c] = bb[c];
  __syncthreads();
  const int64_t* kb = keys + (int64_t)b * L;
  const int i0 = t * tile, i1 = min(L, i0 + tile);
  const uint64_t below = (1ull << lane) - 1ull;
  for (int g = i0; g < i1; g += 64) {
    const int i = g + lane;
    const bool valid = i < i1;
    const int key = valid ? clamp_key(kb[i], ncls) : 0;
    uint64_t match = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (key >> bit) & 1;
      const uint64_t bal = __ballot(on);
      match &= on ? bal : ~bal;
    }
    const int pos = valid ? next[key] + __popcll(match & below) : 0;
    __syncthreads();                                 // all reads of next[] before the update
    if (valid) {
      order[(int64_t)b * L + pos] = glob ? (int32_t)((int64_t)b * seq_rows + row0 + i) : (int32_t)i;
      // the highest lane of each key group advances that key's cursor
      if ((match >> lane) == 1ull) next[key] += __popcll(match);
    }
    __syncthreads();
  }
}

}  // namespace smat

extern "C" int64_t smat_csr_workspace_bytes(int nb, int L, int ncls) {
  if (nb <= 0 || L <= 0 || ncls <= 0) return 0;
  const int tile = smat::csr_tile(L, ncls);
  const int64_t ntiles = (L + tile - 1) / tile;
  return (int64_t)nb * ntiles * ncls * (int64_t)sizeof(int);
}

extern "C" int smat_csr_lists(const int64_t* keys, int32_t* order, int64_t* offs, void* workspace,
                              int nb, int L, int ncls, int global_index, int64_t seq_rows,
                              int64_t row0, void* stream) {
  using namespace smat;
  clear_error();
  SMAT_REQUIRE(offs && (nb == 0 || L == 0 || (keys && order && workspace)), SMAT_EINVAL,
               "smat_csr_lists: null pointer");
  SMAT_REQUIRE(!global_index || (seq_rows >= L && row0 >= 0 && row0 <= seq_rows - L &&
                                   (int64_t)nb * seq_rows < (1ll << 31)),
               SMAT_EINVAL,
               "smat_csr_lists: global items need L <= seq_rows, 0 <= row0 <= seq_rows - L and "
               "nb*seq_rows < 2^31 (L=%d seq_rows=%lld row0=%lld)", L, (long long)seq_rows,
               (long long)row0);
  SMAT_REQUIRE(nb >= 0 && L >= 0 && ncls >= 1 && ncls <= cs::kMaxCls &&
                   (int64_t)nb * L < (1ll << 31),
               SMAT_EUNSUPPORTED, "smat_csr_lists: need 1 <= ncls <= %d and nb*L < 2^31",
               cs::kMaxCls);
  hipStream_t st = (hipStream_t)stream;
  if (nb == 0) {
    // no lists: the single offset is 0 (a kernel, not a memset, so a captured
    // graph replays it as a kernel node)
    hipLaunchKernelGGL(csr_empty_kernel, dim3(1), dim3(64), 0, st, offs);
    return launch_status("smat_csr_lists");
  }
  // L = 0: no tiles; the scan alone writes the (all-zero) offsets
  const int tile = csr_tile(L, ncls);
  const int ntiles = (L + tile - 1) / tile;
  int nbits = 0;
  while ((1 << nbits) < ncls) ++nbits;
  int* counts = (int*)workspace;
  const size_t lds = (size_t)ncls * sizeof(int);
  if (ntiles)
    hipLaunchKernelGGL(csr_count_kernel, dim3(ntiles, nb), dim3(cs::kThreads), lds, st, keys,
                       counts, L, ncls, ntiles, tile);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(nb), dim3(cs::kThreads), 0, st, counts, offs, nb, L,
                     ncls, ntiles);
  if (ntiles)
    hipLaunchKernelGGL(csr_place_kernel, dim3(ntiles, nb), dim3(64), lds, st, keys, counts, order,
                       L, ncls, ntiles, tile, nbits, global_index, seq_rows, row0);
  return launch_status("smat_csr_lists");
}
