// Permutation kernels (building blocks in permute.h).
#include "permute.h"

namespace lmoe {

// Whole permutation in one block (n_pairs <= kChunk).
__global__ __launch_bounds__(1024) void permute_small_kernel(
    const int32_t* __restrict__ ids, int N, const int32_t* __restrict__ log2phy,
    int n_log2phy, int P, int skip, int block_m, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ row_idx, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta) {
  extern __shared__ int hist[];  // [P]
  __shared__ int scan_lds[33];
  __shared__ int err_lds;
  permute_block(ids, N, log2phy, n_log2phy, P, skip, block_m, counts, offsets, sorted_pairs,
                row_idx, active, tile_off, meta, hist, scan_lds, &err_lds);
}

// Whole permutation by one wave (n_pairs <= 64 * PPL, n_slots <= 1024).
template <int PPL>
__global__ __launch_bounds__(64) void permute_wave_kernel(
    const int32_t* __restrict__ ids, int N, const int32_t* __restrict__ log2phy,
    int n_log2phy, int P, int skip, int block_m, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ row_idx, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta) {
  extern __shared__ int lds[];  // [wave_perm_lds_ints(P)]
  permute_wave_any<PPL>(ids, N, log2phy, n_log2phy, P, skip, block_m, counts, offsets,
                        sorted_pairs, row_idx, active, tile_off, meta, lds);
}

// Two builds over the same pairs in one launch, one per block: block 0
// the bank table in skip mode 1, block 1 a later pass's table (the decode
// overflow stage buffer) in skip mode 2.  Block 0 leaves the row_idx of the
// pairs block 1 places (RowKeep), so the outputs are those of the two builds
// one after the other.
struct PermBuild {
  const int32_t* log2phy;
  int n_log2phy;
  int P;
  int32_t* counts;
  int32_t* offsets;
  int32_t* sorted_pairs;
  int32_t* active;
  int32_t* tile_off;
  int32_t* meta;
};

__device__ __forceinline__ RowKeep keep_of(bool second, const PermBuild& b) {
  RowKeep k;
  if (!second) {
    k.log2phy = b.log2phy;
    k.n_log2phy = b.n_log2phy;
    k.P = b.P;
  }
  return k;
}

__global__ __launch_bounds__(1024) void permute_small_two_kernel(
    const int32_t* __restrict__ ids, int N, int block_m, PermBuild a, PermBuild b,
    int32_t* __restrict__ row_idx) {
  extern __shared__ int hist[];  // [max(P_a, P_b)]
  __shared__ int scan_lds[33];
  __shared__ int err_lds;
  const bool second = blockIdx.x != 0;
  const PermBuild o = second ? b : a;
  permute_block(ids, N, o.log2phy, o.n_log2phy, o.P, second ? kSkipKeepRows : 1, block_m,
                o.counts, o.offsets, o.sorted_pairs, row_idx, o.active, o.tile_off, o.meta, hist,
                scan_lds, &err_lds, keep_of(second, b));
}

template <int PPL>
__global__ __launch_bounds__(64) void permute_wave_two_kernel(
    const int32_t* __restrict__ ids, int N, int block_m, PermBuild a, PermBuild b,
    int32_t* __restrict__ row_idx) {
  extern __shared__ int lds[];  // [max(wave_perm_lds_ints(P_a), wave_perm_lds_ints(P_b))]
  const bool second = blockIdx.x != 0;
  const PermBuild o = second ? b : a;
  permute_wave_any<PPL>(ids, N, o.log2phy, o.n_log2phy, o.P, second ? kSkipKeepRows : 1, block_m,
                        o.counts, o.offsets, o.sorted_pairs, row_idx, o.active, o.tile_off,
                        o.meta, lds, keep_of(second, b));
}

// Multi-block path, step 1: per-chunk histograms.
__global__ __launch_bounds__(1024) void permute_hist_kernel(
    const int32_t* __restrict__ ids, int N, const int32_t* __restrict__ log2phy,
    int n_log2phy, int P, int skip, int32_t* __restrict__ slot_of,
    int32_t* __restrict__ chunk_cnt, int32_t* __restrict__ chunk_err) {
  extern __shared__ int hist[];
  __shared__ int err_lds;
  for (int s = threadIdx.x; s < P; s += blockDim.x) hist[s] = 0;
  if (threadIdx.x == 0) err_lds = 0;
  __syncthreads();
  const int p = blockIdx.x * kChunk + threadIdx.x;
  if (p < N) {
    const int s = map_pair(ids, p, log2phy, n_log2phy, P, skip);
    slot_of[p] = s;
    if (s >= 0) atomicAdd(&hist[s], 1);
    if (s == -2) atomicAdd(&err_lds, 1);
  }
  __syncthreads();
  int32_t* dst = chunk_cnt + static_cast<size_t>(blockIdx.x) * P;
  for (int s = threadIdx.x; s < P; s += blockDim.x) dst[s] = hist[s];
  if (threadIdx.x == 0) chunk_err[blockIdx.x] = err_lds;
}

// Step 2: every chunk's block reads the count table (a few KB, in L2),
// forms the slot totals and its own chunk's per-slot bases (the counts of
// the chunks before it), turns the totals into offsets (scan_slots; block 0
// also writes counts / offsets / active / tile_off / meta) and scatters its
// pairs stably from those bases.  The redundant table reads cost less than a
// separate one-block scan launch between the histogram and the scatter (that
// launch: 7.2 us of a 15.4 us permutation of 32768 pairs).
// LDS: 2 P ints.
__global__ __launch_bounds__(1024) void permute_scan_scatter_kernel(
    int N, int P, int nchunks, int skip, int block_m, const int32_t* __restrict__ slot_of,
    const int32_t* __restrict__ chunk_cnt, const int32_t* __restrict__ chunk_err,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta,
    int32_t* __restrict__ sorted_pairs, int32_t* __restrict__ row_idx) {
  extern __shared__ int hist[];  // [P] totals -> offsets -> running bases
  int* before = hist + P;        // [P] this chunk's counts before it
  __shared__ int scan_lds[33];
  const int c0 = blockIdx.x;
  // this thread's pair first: its slot arrives while the table is summed
  const int p = c0 * kChunk + threadIdx.x;
  const int sp = p < N ? slot_of[p] : -1;
  for (int s = threadIdx.x; s < P; s += blockDim.x) {
    int tot = 0, pre = 0;
#pragma unroll 8
    for (int c = 0; c < nchunks; ++c) {
      const int v = chunk_cnt[static_cast<size_t>(c) * P + s];
      tot += v;
      pre += c < c0 ? v : 0;
    }
    hist[s] = tot;
    before[s] = pre;
  }
  __syncthreads();
  if (c0 == 0) {
    scan_slots<true>(hist, P, block_m, scan_lds, counts, offsets, active, tile_off, meta);
    if (threadIdx.x == 0) {
      int e = 0;
      for (int c = 0; c < nchunks; ++c) e += chunk_err[c];
      meta[LMOE_META_ERRORS] = e;
    }
  } else {
    scan_slots<false>(hist, P, block_m, scan_lds, counts, offsets, active, tile_off, meta);
  }
  __syncthreads();  // hist holds the offsets
  for (int s = threadIdx.x; s < P; s += blockDim.x) hist[s] += before[s];
  __syncthreads();
  const int pos = chunk_positions(sp >= 0 ? sp : -1, key_bits(P), hist);
  if (p < N) {
    if (pos >= 0 || skip != kSkipKeepRows) row_idx[p] = pos;
    if (pos >= 0) sorted_pairs[pos] = p;
  }
}

// expanded_x rows
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint16_t* __restrict__ x, int H, int k,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ meta,
    uint16_t* __restrict__ x_sorted) {
  const int pos = blockIdx.x;
  if (pos >= meta[LMOE_META_PAIRS]) return;
  const int t = sorted_pairs[pos] / k;
  const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(t) * H);
  uint4* dst = reinterpret_cast<uint4*>(x_sorted + static_cast<size_t>(pos) * H);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) dst[i] = src[i];
}

}  // namespace lmoe

using namespace lmoe;

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

extern "C" size_t lmoe_permute_workspace_bytes(int n_pairs, int n_slots) {
  if (n_pairs <= kChunk || n_slots <= 0) return 0;
  const size_t nchunks = (static_cast<size_t>(n_pairs) + kChunk - 1) / kChunk;
  return align_up(sizeof(int32_t) * n_pairs) +
         align_up(sizeof(int32_t) * nchunks * n_slots) +
         align_up(sizeof(int32_t) * nchunks);
}

extern "C" int lmoe_permute(const int32_t* ids, int n_pairs,
                            const int32_t* log2phy, int n_log2phy, int n_slots,
                            int skip_unmapped, int block_m, int32_t* counts,
                            int32_t* offsets, int32_t* sorted_pairs,
                            int32_t* row_idx, int32_t* active, int32_t* tile_off,
                            int32_t* meta, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  if (n_pairs < 0 || n_slots <= 0 || block_m <= 0) return LMOE_ERR_ARG;
  if ((n_pairs > 0 && ids == nullptr) || counts == nullptr || offsets == nullptr ||
      sorted_pairs == nullptr || row_idx == nullptr || active == nullptr ||
      tile_off == nullptr || meta == nullptr)
    return LMOE_ERR_ARG;
  if (log2phy != nullptr && n_log2phy <= 0) return LMOE_ERR_ARG;
  if (n_slots > kMaxSlots) return LMOE_ERR_SHAPE;
  if (skip_unmapped < 0 || skip_unmapped > kSkipKeepRows) return LMOE_ERR_ARG;
  const int skip = skip_unmapped;
  const size_t lds = sizeof(int) * static_cast<size_t>(n_slots);
  if (wave_perm_fits(n_pairs, n_slots)) {
    // decode sizes: one wave, no block barriers
    const size_t wlds = sizeof(int) * static_cast<size_t>(wave_perm_lds_ints(n_slots));
#define LMOE_PWK(Q)                                                                           \
  hipLaunchKernelGGL(permute_wave_kernel<Q>, dim3(1), dim3(kWave), wlds, stream, ids, n_pairs, \
                     log2phy, n_log2phy, n_slots, skip, block_m, counts, offsets, sorted_pairs,  \
                     row_idx, active, tile_off, meta)
    const int ppl = wave_perm_ppl(n_pairs);
    if (ppl == 1) LMOE_PWK(1);
    else if (ppl == 2) LMOE_PWK(2);
    else LMOE_PWK(4);
#undef LMOE_PWK
    LMOE_RETURN_LAUNCH();
  }
  if (n_pairs <= kChunk) {
    // one block; as few waves as the pairs and the slot scan need (block-wide
    // barriers are the cost of this kernel, and they grow with the waves)
    int threads = n_pairs > n_slots / 16 ? n_pairs : n_slots / 16;
    threads = ((threads + 63) / 64) * 64;
    threads = threads < 64 ? 64 : (threads > kChunk ? kChunk : threads);
    hipLaunchKernelGGL(permute_small_kernel, dim3(1), dim3(threads), lds, stream,
                       ids, n_pairs, log2phy, n_log2phy, n_slots, skip, block_m,
                       counts, offsets, sorted_pairs, row_idx, active, tile_off,
                       meta);
    LMOE_RETURN_LAUNCH();
  }
  if (workspace == nullptr ||
      workspace_bytes < lmoe_permute_workspace_bytes(n_pairs, n_slots))
    return LMOE_ERR_WORKSPACE;
  const int nchunks = (n_pairs + kChunk - 1) / kChunk;
  char* ws = static_cast<char*>(workspace);
  int32_t* slot_of = reinterpret_cast<int32_t*>(ws);
  ws += align_up(sizeof(int32_t) * n_pairs);
  int32_t* chunk_cnt = reinterpret_cast<int32_t*>(ws);
  ws += align_up(sizeof(int32_t) * static_cast<size_t>(nchunks) * n_slots);
  int32_t* chunk_err = reinterpret_cast<int32_t*>(ws);
  hipLaunchKernelGGL(permute_hist_kernel, dim3(nchunks), dim3(kChunk), lds,
                     stream, ids, n_pairs, log2phy, n_log2phy, n_slots, skip,
                     slot_of, chunk_cnt, chunk_err);
  hipLaunchKernelGGL(permute_scan_scatter_kernel, dim3(nchunks), dim3(kChunk), 2 * lds, stream,
                     n_pairs, n_slots, nchunks, skip, block_m, slot_of, chunk_cnt, chunk_err,
                     counts, offsets, active, tile_off, meta, sorted_pairs, row_idx);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_permute_two_tables(
    const int32_t* ids, int n_pairs, int block_m, int32_t* row_idx, const int32_t* log2phy_a,
    int n_log2phy_a, int n_slots_a, int32_t* counts_a, int32_t* offsets_a, int32_t* sorted_pairs_a,
    int32_t* active_a, int32_t* tile_off_a, int32_t* meta_a, const int32_t* log2phy_b,
    int n_log2phy_b, int n_slots_b, int32_t* counts_b, int32_t* offsets_b,
    int32_t* sorted_pairs_b, int32_t* active_b, int32_t* tile_off_b, int32_t* meta_b,
    hipStream_t stream) {
  if (n_pairs < 0 || n_slots_a <= 0 || n_slots_b <= 0 || block_m <= 0) return LMOE_ERR_ARG;
  if (n_log2phy_a <= 0 || n_log2phy_b <= 0) return LMOE_ERR_ARG;
  if ((n_pairs > 0 && ids == nullptr) || row_idx == nullptr || log2phy_a == nullptr ||
      log2phy_b == nullptr)
    return LMOE_ERR_ARG;
  if (counts_a == nullptr || offsets_a == nullptr || sorted_pairs_a == nullptr ||
      active_a == nullptr || tile_off_a == nullptr || meta_a == nullptr || counts_b == nullptr ||
      offsets_b == nullptr || sorted_pairs_b == nullptr || active_b == nullptr ||
      tile_off_b == nullptr || meta_b == nullptr)
    return LMOE_ERR_ARG;
  if (n_slots_a > kMaxSlots || n_slots_b > kMaxSlots) return LMOE_ERR_SHAPE;
  // one block per table: the multi-block builds are left to lmoe_permute
  if (n_pairs > kChunk) return LMOE_ERR_SHAPE;
  const PermBuild a{log2phy_a, n_log2phy_a, n_slots_a, counts_a, offsets_a, sorted_pairs_a,
                    active_a, tile_off_a, meta_a};
  const PermBuild b{log2phy_b, n_log2phy_b, n_slots_b, counts_b, offsets_b, sorted_pairs_b,
                    active_b, tile_off_b, meta_b};
  if (wave_perm_fits(n_pairs, n_slots_a) && wave_perm_fits(n_pairs, n_slots_b)) {
    const int ints_a = wave_perm_lds_ints(n_slots_a);
    const int ints_b = wave_perm_lds_ints(n_slots_b);
    const size_t wlds = sizeof(int) * static_cast<size_t>(ints_a > ints_b ? ints_a : ints_b);
#define LMOE_PW2(Q)                                                                             \
  hipLaunchKernelGGL(permute_wave_two_kernel<Q>, dim3(2), dim3(kWave), wlds, stream, ids,        \
                     n_pairs, block_m, a, b, row_idx)
    const int ppl = wave_perm_ppl(n_pairs);
    if (ppl == 1) LMOE_PW2(1);
    else if (ppl == 2) LMOE_PW2(2);
    else LMOE_PW2(4);
#undef LMOE_PW2
    LMOE_RETURN_LAUNCH();
  }
  // the larger table sets the block's threads and LDS (as lmoe_permute's
  // one-block path sizes them for one table)
  const int P = n_slots_a > n_slots_b ? n_slots_a : n_slots_b;
  int threads = n_pairs > P / 16 ? n_pairs : P / 16;
  threads = ((threads + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > kChunk ? kChunk : threads);
  hipLaunchKernelGGL(permute_small_two_kernel, dim3(2), dim3(threads),
                     sizeof(int) * static_cast<size_t>(P), stream, ids, n_pairs, block_m, a, b,
                     row_idx);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_gather_rows(const void* x, int H, int k,
                                const int32_t* sorted_pairs, const int32_t* meta,
                                int n_pairs, void* x_sorted, hipStream_t stream) {
  if (H <= 0 || k <= 0 || n_pairs < 0) return LMOE_ERR_ARG;
  if (H % 8 != 0) return LMOE_ERR_SHAPE;
  if (n_pairs == 0) return LMOE_OK;  // an empty batch: nothing read or written
  if (x == nullptr || sorted_pairs == nullptr || meta == nullptr || x_sorted == nullptr)
    return LMOE_ERR_ARG;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(n_pairs), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(x), H, k, sorted_pairs, meta,
                     static_cast<uint16_t*>(x_sorted));
  LMOE_RETURN_LAUNCH();
}
