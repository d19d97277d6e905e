// Permutation kernels: token->slot remap through log2phy, count histogram per
// physical slot, stable counting sort of the flat (token, k) pairs by slot,
// active-slot list and the MFMA tile table.
//
// Reference behaviour: ExpertSlotMapping.remap_topk_ids
// (moe_offload/slot_mapping.py:116-140, phys = log2phy[ids], fail closed on
// -1) feeding npu_moe_init_routing_v2 (patches/patch_fused_moe.py:668-701:
// stable sort by expert, expanded_row_idx, count-type histogram).  The wave
// filter (skip_unmapped) plays the role of the per-wave expert table of
// phase_split.build_b2_device_wave_microbatch_plans (:1224-1384).
//
// Integer work only; every output is bit-exact and independent of launch
// shape.  Pairs of one chunk (1024 pairs) are ranked with wave64 ballots.
#include "lmoe_device.h"

namespace lmoe {

constexpr int kChunk = 1024;       // pairs per block
constexpr int kMaxSlots = 8192;    // LDS histogram bound

// slot of pair p: >= 0 placed, -1 skipped silently, -2 error
__device__ __forceinline__ int map_pair(const int32_t* __restrict__ ids, int p,
                                        const int32_t* __restrict__ log2phy,
                                        int n_log2phy, int P, int skip) {
  const int id = ids[p];
  int s;
  if (log2phy != nullptr) {
    // in wave mode an id the table does not cover belongs to another pass
    if (id < 0 || id >= n_log2phy) return skip ? -1 : -2;
    s = log2phy[id];
  } else {
    s = id;
  }
  if (s >= 0 && s < P) return s;
  if (skip && s == -1) return -1;
  return -2;
}

__device__ __forceinline__ uint64_t match_key(int key, int nbits) {
  uint64_t m = __ballot(1);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}

// Exclusive scan over a block of 1024 threads.  Returns the exclusive prefix
// of v; *total receives the block sum.  Uses scan_lds[32].
__device__ int block_exclusive_scan(int v, int* scan_lds, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += t;
  }
  if (lane == 63) scan_lds[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < nw; ++w) {
      const int c = scan_lds[w];
      scan_lds[w] = run;
      run += c;
    }
    scan_lds[nw] = run;
  }
  __syncthreads();
  const int excl = scan_lds[wave] + inc - v;
  *total = scan_lds[nw];
  __syncthreads();
  return excl;
}

// Scan counts[0..P) held in LDS (hist) into offsets/active/tile_off; writes
// counts, offsets, active, tile_off and meta[ACTIVE, PAIRS, TILES], and
// replaces hist[s] by offsets[s] in place (each s is owned by one thread).
__device__ void scan_slots(int* hist, int P, int block_m, int* scan_lds,
                           int32_t* counts, int32_t* offsets, int32_t* active,
                           int32_t* tile_off, int32_t* meta) {
  const int per = (P + blockDim.x - 1) / blockDim.x;
  const int s0 = threadIdx.x * per;
  int csum = 0, asum = 0, tsum = 0;
  for (int i = 0; i < per; ++i) {
    const int s = s0 + i;
    if (s < P) {
      const int c = hist[s];
      csum += c;
      asum += c > 0;
      tsum += (c + block_m - 1) / block_m;
    }
  }
  int ctot, atot, ttot;
  int cpre = block_exclusive_scan(csum, scan_lds, &ctot);
  int apre = block_exclusive_scan(asum, scan_lds, &atot);
  int tpre = block_exclusive_scan(tsum, scan_lds, &ttot);
  for (int i = 0; i < per; ++i) {
    const int s = s0 + i;
    if (s < P) {
      const int c = hist[s];
      counts[s] = c;
      offsets[s] = cpre;
      tile_off[s] = tpre;
      if (c > 0) active[apre++] = s;
      hist[s] = cpre;
      cpre += c;
      tpre += (c + block_m - 1) / block_m;
    }
  }
  if (threadIdx.x == 0) {
    offsets[P] = ctot;
    tile_off[P] = ttot;
    meta[LMOE_META_ACTIVE] = atot;
    meta[LMOE_META_PAIRS] = ctot;
    meta[LMOE_META_TILES] = ttot;
  }
}

// Stable ranks of one chunk.  slot[] is this thread's slot (>= 0 placed),
// run_base[s] holds the next free position of slot s and is advanced.
__device__ int chunk_positions(int s, int nbits, int* run_base) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const bool placed = s >= 0;
  const int key = placed ? s : (1 << nbits) - 1;
  const uint64_t m = match_key(key, nbits);
  const int rank = __popcll(m & lanemask_lt(lane));
  const int cnt = __popcll(m);
  const bool last = lane == 63 - __clzll(m);
  int pos = -1;
  for (int w = 0; w < nw; ++w) {
    if (wave == w && placed) {
      const int b = run_base[s];
      pos = b + rank;
      if (last) run_base[s] = b + cnt;
    }
    __syncthreads();
  }
  return pos;
}

__device__ __forceinline__ int key_bits(int P) {
  // keys 0..P (P = "not placed" sentinel fits when (1<<nbits)-1 >= P)
  int nbits = 1;
  while ((1 << nbits) - 1 < P) ++nbits;
  return nbits;
}

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
  for (int s = threadIdx.x; s < P; s += blockDim.x) hist[s] = 0;
  if (threadIdx.x == 0) err_lds = 0;
  __syncthreads();
  // each thread owns pairs threadIdx.x + c * blockDim.x, c < kSmallChunks
  constexpr int kSmallChunks = kChunk / 64;
  int sl[kSmallChunks];
#pragma unroll
  for (int c = 0; c < kSmallChunks; ++c) {
    const int p = threadIdx.x + c * blockDim.x;
    sl[c] = -1;
    if (p < N) {
      const int s = map_pair(ids, p, log2phy, n_log2phy, P, skip);
      sl[c] = s;
      if (s >= 0) atomicAdd(&hist[s], 1);
      if (s == -2) atomicAdd(&err_lds, 1);
    }
  }
  __syncthreads();
  scan_slots(hist, P, block_m, scan_lds, counts, offsets, active, tile_off, meta);
  if (threadIdx.x == 0) meta[LMOE_META_ERRORS] = err_lds;
  __syncthreads();  // hist now holds offsets: the running base of each slot
  const int nb = key_bits(P);
#pragma unroll
  for (int c = 0; c < kSmallChunks; ++c) {
    if (c * static_cast<int>(blockDim.x) < N) {  // uniform across the block
      const int p = threadIdx.x + c * blockDim.x;
      const int s = sl[c] >= 0 ? sl[c] : -1;
      const int pos = chunk_positions(s, nb, hist);  // chunks in pair order: stable
      if (p < N) {
        row_idx[p] = pos;
        if (pos >= 0) sorted_pairs[pos] = p;
      }
    }
  }
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

// Step 2 (one block): column sums -> offsets, per-chunk bases.
__global__ __launch_bounds__(1024) void permute_scan_kernel(
    int P, int nchunks, int block_m, int32_t* __restrict__ chunk_cnt,
    const int32_t* __restrict__ chunk_err, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ active,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ meta) {
  extern __shared__ int hist[];
  __shared__ int scan_lds[33];
  for (int s = threadIdx.x; s < P; s += blockDim.x) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      int32_t* q = chunk_cnt + static_cast<size_t>(c) * P + s;
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
  for (int s = threadIdx.x; s < P; s += blockDim.x) {
    const int base = hist[s];
    for (int c = 0; c < nchunks; ++c) chunk_cnt[static_cast<size_t>(c) * P + s] += base;
  }
}

// Step 3: stable scatter of each chunk from its per-slot bases.
__global__ __launch_bounds__(1024) void permute_scatter_kernel(
    int N, int P, const int32_t* __restrict__ slot_of,
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
    row_idx[p] = pos;
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
  const int skip = skip_unmapped ? 1 : 0;
  const size_t lds = sizeof(int) * static_cast<size_t>(n_slots);
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
  hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(kChunk), lds, stream,
                     n_slots, nchunks, block_m, chunk_cnt, chunk_err, counts,
                     offsets, active, tile_off, meta);
  hipLaunchKernelGGL(permute_scatter_kernel, dim3(nchunks), dim3(kChunk), lds,
                     stream, n_pairs, n_slots, slot_of, chunk_cnt, sorted_pairs,
                     row_idx);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_gather_rows(const void* x, int H, int k,
                                const int32_t* sorted_pairs, const int32_t* meta,
                                int n_pairs, void* x_sorted, hipStream_t stream) {
  if (x == nullptr || sorted_pairs == nullptr || meta == nullptr ||
      x_sorted == nullptr || H <= 0 || k <= 0 || n_pairs < 0)
    return LMOE_ERR_ARG;
  if (H % 8 != 0) return LMOE_ERR_SHAPE;
  if (n_pairs == 0) return LMOE_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(n_pairs), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(x), H, k, sorted_pairs, meta,
                     static_cast<uint16_t*>(x_sorted));
  LMOE_RETURN_LAUNCH();
}
