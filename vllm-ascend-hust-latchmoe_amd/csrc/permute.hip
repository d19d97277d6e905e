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

// Step 2 (one block): column sums -> offsets, per-chunk bases.  With
// IN_LDS the nchunks x P count table is read into LDS with coalesced loads,
// each slot's column is scanned there, and the bases go back in parallel
// (the global walk costs one dependent round trip per chunk and slot).
// LDS: P ints (hist), plus nchunks * P with IN_LDS.
constexpr int kScanLdsInts = 16384;  // count table held in LDS up to 64 KiB

template <bool IN_LDS>
__global__ __launch_bounds__(1024) void permute_scan_kernel(
    int P, int nchunks, int block_m, int32_t* __restrict__ chunk_cnt,
    const int32_t* __restrict__ chunk_err, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta) {
  extern __shared__ int hist[];
  __shared__ int scan_lds[33];
  int* cc = hist + P;  // [nchunks][P] with IN_LDS
  const int n = nchunks * P;
  if (IN_LDS) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) cc[i] = chunk_cnt[i];
    __syncthreads();
  }
  for (int s = threadIdx.x; s < P; s += blockDim.x) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      int* q = IN_LDS ? cc + c * P + s : chunk_cnt + static_cast<size_t>(c) * P + s;
      const int v = *q;
      *q = run;
      run += v;
    }
    hist[s] = run;
  }
  __syncthreads();
  scan_slots(hist, P, block_m, scan_lds, counts, offsets, active, tile_off, meta);
  if (threadIdx.x == 0) {
    int e = 0;
    for (int c = 0; c < nchunks; ++c) e += chunk_err[c];
    meta[LMOE_META_ERRORS] = e;
  }
  __syncthreads();  // hist now holds offsets
  if (IN_LDS) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) chunk_cnt[i] = cc[i] + hist[i % P];
  } else {
    for (int s = threadIdx.x; s < P; s += blockDim.x) {
      const int base = hist[s];
      for (int c = 0; c < nchunks; ++c) chunk_cnt[static_cast<size_t>(c) * P + s] += base;
    }
  }
}

// Step 3: stable scatter of each chunk from its per-slot bases.
__global__ __launch_bounds__(1024) void permute_scatter_kernel(
    int N, int P, int skip, const int32_t* __restrict__ slot_of,
    const int32_t* __restrict__ chunk_cnt, int32_t* __restrict__ sorted_pairs,
    int32_t* __restrict__ row_idx) {
  extern __shared__ int run_base[];
  const int32_t* src = chunk_cnt + static_cast<size_t>(blockIdx.x) * P;
  for (int s = threadIdx.x; s < P; s += blockDim.x) run_base[s] = src[s];
  __syncthreads();
  const int p = blockIdx.x * kChunk + threadIdx.x;
  const int s = p < N ? slot_of[p] : -1;
  const int pos = chunk_positions(s >= 0 ? s : -1, key_bits(P), run_base);
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
  if (static_cast<long long>(nchunks) * n_slots <= kScanLdsInts) {
    const size_t scan_lds = sizeof(int) * (static_cast<size_t>(n_slots) +
                                           static_cast<size_t>(nchunks) * n_slots);
    hipLaunchKernelGGL(permute_scan_kernel<true>, dim3(1), dim3(kChunk), scan_lds, stream,
                       n_slots, nchunks, block_m, chunk_cnt, chunk_err, counts, offsets, active,
                       tile_off, meta);
  } else {
    hipLaunchKernelGGL(permute_scan_kernel<false>, dim3(1), dim3(kChunk), lds, stream,
                       n_slots, nchunks, block_m, chunk_cnt, chunk_err, counts, offsets, active,
                       tile_off, meta);
  }
  hipLaunchKernelGGL(permute_scatter_kernel, dim3(nchunks), dim3(kChunk), lds,
                     stream, n_pairs, n_slots, skip, slot_of, chunk_cnt, sorted_pairs,
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
