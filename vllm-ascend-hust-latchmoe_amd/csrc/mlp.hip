// Grouped SwiGLU expert MLP over the slot bank, and the weighted combine.
//
// Decode (few pairs per slot): weight-streaming GEMV kernels.  Every weight
// row is read from HBM exactly once with 16-byte (gate/up) or 8-byte (down)
// vector loads, several rows per lane in flight; token rows and act rows come
// from L1/L2.  The down projection can be fused with the weighted combine
// (one workgroup owns 4 output columns for every token), so the decode layer
// is permute + two kernels.
// Prefill (hundreds of pairs per slot): bf16 MFMA grouped GEMM, gemm_mfma.h.
//
// Reference behaviour: npu_grouped_matmul (GMM1) + npu_swiglu + GMM2 inside
// _apply_mlp (patches/patch_fused_moe.py:3772-3774, hooks :4249-4302) reading
// w1/w2 = slot bank (PreparedSlotWeights, slot_mapping.py:143-187), then
// npu_moe_token_unpermute (:3363-3366; out[t] = sum_j w[t,j] y[row(t,j)],
// phase_split.py:1649-1656).
#include "gemm_mfma.h"

namespace lmoe {

// ---------------------------------------------------------------------------
// gate_up GEMV + SiLU*mul.  grid (ceil(I/4), max_active), 4 waves; wave w of
// block (bx, a) owns i = 4*bx + w of the a-th active slot: its gate and up
// rows stay in registers while the slot's token rows stream past.
// ---------------------------------------------------------------------------
template <int NC>
__global__ __launch_bounds__(256) void gateup_gemv_kernel(
    const uint16_t* __restrict__ x, int H, int I, int topk,
    const uint16_t* __restrict__ w13, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, uint16_t* __restrict__ act) {
  const int a = blockIdx.y;
  if (a >= meta[LMOE_META_ACTIVE]) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int i = blockIdx.x * 4 + wave;
  if (i >= I) return;
  const int s = active[a];
  const int p0 = offsets[s];
  const int n = offsets[s + 1] - p0;
  const uint16_t* grow = w13 + (static_cast<size_t>(s) * 2 * I + i) * H;
  const uint16_t* urow = grow + static_cast<size_t>(I) * H;

  uint4 wg[NC], wu[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int h = c * 512 + lane * 8;
    if (h < H) {
      wg[c] = *reinterpret_cast<const uint4*>(grow + h);
      wu[c] = *reinterpret_cast<const uint4*>(urow + h);
    } else {
      wg[c] = make_uint4(0u, 0u, 0u, 0u);
      wu[c] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  for (int r0 = 0; r0 < n; r0 += 4) {
    float ag[4], au[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ag[q] = 0.0f;
      au[q] = 0.0f;
      if (r0 + q < n) {
        const int t = sorted_pairs[p0 + r0 + q] / topk;
        const uint16_t* xr = x + static_cast<size_t>(t) * H;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int h = c * 512 + lane * 8;
          if (h < H) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xr + h);
            ag[q] = dot8(xv, wg[c], ag[q]);
            au[q] = dot8(xv, wu[c], au[q]);
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ag[q] = wave_sum(ag[q]);
      au[q] = wave_sum(au[q]);
    }
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (r0 + q < n) {
          act[static_cast<size_t>(p0 + r0 + q) * I + i] = swiglu_bf16(ag[q], au[q]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// down GEMV fused with the weighted combine (n_pairs <= 1024).  grid
// ceil(H/4); wave w owns output column h = 4*bx + w for every pair: it walks
// the active slots G at a time (all G weight rows loaded before use), keeps
// y[pos][h] in LDS, then the block combines tokens in j order.
// ---------------------------------------------------------------------------
constexpr int kFusedMaxPairs = 1024;

template <int NU>
__global__ __launch_bounds__(256) void down_combine_gemv_kernel(
    const uint16_t* __restrict__ act, int I, int H, int T, int topk,
    const uint16_t* __restrict__ w2, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, const int32_t* __restrict__ meta,
    const int32_t* __restrict__ row_idx, const uint16_t* __restrict__ wts,
    const uint16_t* __restrict__ add, uint16_t* __restrict__ out) {
  __shared__ float ybuf[kFusedMaxPairs * 4];
  constexpr int G = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = blockIdx.x * 4 + wave;
  const int na = meta[LMOE_META_ACTIVE];
  if (h < H) {
    for (int a0 = 0; a0 < na; a0 += G) {
      uint2 wv[G][NU];
      int sl[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        sl[g] = (a0 + g < na) ? active[a0 + g] : -1;
        const uint16_t* row =
            w2 + (static_cast<size_t>(sl[g] >= 0 ? sl[g] : 0) * H + h) * I;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const int e = (u * 64 + lane) * 4;
          wv[g][u] = (sl[g] >= 0 && e < I) ? *reinterpret_cast<const uint2*>(row + e)
                                            : make_uint2(0u, 0u);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (sl[g] < 0) continue;
        const int p0 = offsets[sl[g]];
        const int n = offsets[sl[g] + 1] - p0;
        for (int r = 0; r < n; ++r) {
          const int pos = p0 + r;
          const uint16_t* arow = act + static_cast<size_t>(pos) * I;
          float acc = 0.0f;
#pragma unroll
          for (int u = 0; u < NU; ++u) {
            const int e = (u * 64 + lane) * 4;
            if (e < I) acc = dot4(*reinterpret_cast<const uint2*>(arow + e), wv[g][u], acc);
          }
          acc = wave_sum(acc);
          if (lane == 0) ybuf[pos * 4 + wave] = round_bf16(acc);  // GMM2 output is bf16
        }
      }
    }
  }
  __syncthreads();
  for (int q = threadIdx.x; q < T * 4; q += blockDim.x) {
    const int t = q >> 2;
    const int c = q & 3;
    const int hh = blockIdx.x * 4 + c;
    if (hh >= H) continue;
    float acc = 0.0f;
    for (int j = 0; j < topk; ++j) {
      const int p = t * topk + j;
      const int r = row_idx[p];
      if (r >= 0) acc += bf16_to_f32(wts[p]) * ybuf[r * 4 + c];
    }
    if (add != nullptr) acc += bf16_to_f32(add[static_cast<size_t>(t) * H + hh]);
    out[static_cast<size_t>(t) * H + hh] = static_cast<uint16_t>(f32_to_bf16_bits(acc));
  }
}

// ---------------------------------------------------------------------------
// down GEMV per slot, writes y[pair][h] (bf16).  grid (ceil(H/16),
// max_active); wave w owns rows h0 + 4w .. h0 + 4w + 3 of the a-th slot.
// ---------------------------------------------------------------------------
template <int NU>
__global__ __launch_bounds__(256) void down_gemv_kernel(
    const uint16_t* __restrict__ act, int I, int H,
    const uint16_t* __restrict__ w2, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, const int32_t* __restrict__ active,
    const int32_t* __restrict__ meta, uint16_t* __restrict__ y) {
  const int a = blockIdx.y;
  if (a >= meta[LMOE_META_ACTIVE]) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h0 = blockIdx.x * 16 + wave * 4;
  if (h0 >= H) return;
  const int s = active[a];
  const int p0 = offsets[s];
  const int n = offsets[s + 1] - p0;
  uint2 wv[4][NU];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int h = h0 + rr;
    const uint16_t* row = w2 + (static_cast<size_t>(s) * H + (h < H ? h : 0)) * I;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int e = (u * 64 + lane) * 4;
      wv[rr][u] = (h < H && e < I) ? *reinterpret_cast<const uint2*>(row + e)
                                   : make_uint2(0u, 0u);
    }
  }
  for (int r = 0; r < n; ++r) {
    const int pos = p0 + r;
    const uint16_t* arow = act + static_cast<size_t>(pos) * I;
    uint2 av[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int e = (u * 64 + lane) * 4;
      av[u] = (e < I) ? *reinterpret_cast<const uint2*>(arow + e) : make_uint2(0u, 0u);
    }
    float acc[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      acc[rr] = 0.0f;
#pragma unroll
      for (int u = 0; u < NU; ++u) acc[rr] = dot4(av[u], wv[rr][u], acc[rr]);
      acc[rr] = wave_sum(acc[rr]);
    }
    if (lane == 0) {
      const int pair = sorted_pairs[pos];
      uint16_t* yr = y + static_cast<size_t>(pair) * H;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (h0 + rr < H) yr[h0 + rr] = static_cast<uint16_t>(f32_to_bf16_bits(acc[rr]));
    }
  }
}

// ---------------------------------------------------------------------------
// weighted combine, y indexed by flat pair.  grid (T, ceil(H/2048)); each
// thread owns 8 consecutive columns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ w, int T, int topk, int H,
    const uint16_t* __restrict__ add, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (t >= T || h >= H) return;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  for (int j = 0; j < topk; ++j) {
    const int p = t * topk + j;
    if (row_idx != nullptr && row_idx[p] < 0) continue;
    const float wj = bf16_to_f32(w[p]);
    const uint4 v = *reinterpret_cast<const uint4*>(y + static_cast<size_t>(p) * H + h);
    acc[0] += wj * bf16lo(v.x);
    acc[1] += wj * bf16hi(v.x);
    acc[2] += wj * bf16lo(v.y);
    acc[3] += wj * bf16hi(v.y);
    acc[4] += wj * bf16lo(v.z);
    acc[5] += wj * bf16hi(v.z);
    acc[6] += wj * bf16lo(v.w);
    acc[7] += wj * bf16hi(v.w);
  }
  if (add != nullptr) {
    const uint4 v = *reinterpret_cast<const uint4*>(add + static_cast<size_t>(t) * H + h);
    acc[0] += bf16lo(v.x);
    acc[1] += bf16hi(v.x);
    acc[2] += bf16lo(v.y);
    acc[3] += bf16hi(v.y);
    acc[4] += bf16lo(v.z);
    acc[5] += bf16hi(v.z);
    acc[6] += bf16lo(v.w);
    acc[7] += bf16hi(v.w);
  }
  uint4 o;
  o.x = pack_bf16x2(acc[0], acc[1]);
  o.y = pack_bf16x2(acc[2], acc[3]);
  o.z = pack_bf16x2(acc[4], acc[5]);
  o.w = pack_bf16x2(acc[6], acc[7]);
  *reinterpret_cast<uint4*>(out + static_cast<size_t>(t) * H + h) = o;
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
static int launch_gateup_gemv(const uint16_t* x, int H, int I, int topk,
                              const uint16_t* w13, const int32_t* offsets,
                              const int32_t* sorted_pairs, const int32_t* active,
                              const int32_t* meta, int max_active, uint16_t* act,
                              hipStream_t stream) {
  dim3 grid((I + 3) / 4, max_active);
  const int nc = (H + 511) / 512;
#define LMOE_GU(NC)                                                            \
  hipLaunchKernelGGL(gateup_gemv_kernel<NC>, grid, dim3(256), 0, stream, x, H, \
                     I, topk, w13, offsets, sorted_pairs, active, meta, act)
  if (nc <= 4) LMOE_GU(4);
  else if (nc <= 8) LMOE_GU(8);
  else if (nc <= 14) LMOE_GU(14);
  else if (nc <= 16) LMOE_GU(16);
  else return LMOE_ERR_SHAPE;
#undef LMOE_GU
  return LMOE_OK;
}

static int nu_for(int I) { return (I + 255) / 256; }

}  // namespace lmoe

using namespace lmoe;

static long long slot_elems_w13(int H, int I) { return 2LL * I * H; }
static long long slot_elems_w2(int H, int I) { return 1LL * H * I; }

static int check_mlp_args(int T, int H, int I, int k, int n_slots, int n_pairs) {
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0 || n_pairs < 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 8192 || H > 8192) return LMOE_ERR_SHAPE;
  return LMOE_OK;
}

static int resolve_path(int path, int n_pairs) {
  return path == LMOE_PATH_AUTO ? (n_pairs <= 256 ? LMOE_PATH_GEMV : LMOE_PATH_MFMA) : path;
}

extern "C" int lmoe_gateup_silu(const void* x, int T, int H, int I, int k,
                                const void* w13_slots, int n_slots,
                                const int32_t* offsets, const int32_t* sorted_pairs,
                                const int32_t* active, const int32_t* tile_off,
                                const int32_t* meta, int n_pairs, int block_m,
                                int path, void* act, hipStream_t stream) {
  if (x == nullptr || w13_slots == nullptr || offsets == nullptr || sorted_pairs == nullptr ||
      active == nullptr || meta == nullptr || act == nullptr)
    return LMOE_ERR_ARG;
  int st = check_mlp_args(T, H, I, k, n_slots, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_pairs == 0) return LMOE_OK;
  path = resolve_path(path, n_pairs);
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  if (path == LMOE_PATH_GEMV) {
    st = launch_gateup_gemv(static_cast<const uint16_t*>(x), H, I, k,
                            static_cast<const uint16_t*>(w13_slots), offsets, sorted_pairs,
                            active, meta, max_active, static_cast<uint16_t*>(act), stream);
    if (st != LMOE_OK) return st;
    LMOE_RETURN_LAUNCH();
  }
  if (path != LMOE_PATH_MFMA) return LMOE_ERR_UNSUPPORTED;
  if (tile_off == nullptr) return LMOE_ERR_ARG;
  if (block_m != kBM) return LMOE_ERR_UNSUPPORTED;
  GemmArgs g{};
  g.topk = k;
  g.offsets = offsets;
  g.sorted_pairs = sorted_pairs;
  g.tile_off = tile_off;
  g.meta = meta;
  g.P = n_slots;
  g.a = static_cast<const uint16_t*>(x);
  g.w = static_cast<const uint16_t*>(w13_slots);
  g.w_slot_stride = slot_elems_w13(H, I);
  g.N = I;
  g.K = H;
  g.I = I;
  g.out = act;
  const int ub_tiles = n_pairs / kBM + max_active + 1;
  hipLaunchKernelGGL(grouped_gemm_kernel<kGateUp>, dim3(ub_tiles, (I + 63) / 64), dim3(256), 0,
                     stream, g);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_down(const void* act, int H, int I, const void* w2_slots, int n_slots,
                         const int32_t* offsets, const int32_t* sorted_pairs,
                         const int32_t* active, const int32_t* tile_off,
                         const int32_t* meta, int n_pairs, int block_m, int path,
                         void* y, hipStream_t stream) {
  if (act == nullptr || w2_slots == nullptr || offsets == nullptr || sorted_pairs == nullptr ||
      active == nullptr || meta == nullptr || y == nullptr)
    return LMOE_ERR_ARG;
  int st = check_mlp_args(1, H, I, 1, n_slots, n_pairs);
  if (st != LMOE_OK) return st;
  if (n_pairs == 0) return LMOE_OK;
  path = resolve_path(path, n_pairs);
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  const uint16_t* actb = static_cast<const uint16_t*>(act);
  const uint16_t* w2 = static_cast<const uint16_t*>(w2_slots);
  uint16_t* yb = static_cast<uint16_t*>(y);
  if (path == LMOE_PATH_GEMV) {
    dim3 grid((H + 15) / 16, max_active);
    const int nu = nu_for(I);
#define LMOE_DN(NU)                                                            \
  hipLaunchKernelGGL(down_gemv_kernel<NU>, grid, dim3(256), 0, stream, actb, I, H, \
                     w2, offsets, sorted_pairs, active, meta, yb)
    if (nu <= 3) LMOE_DN(3);
    else if (nu <= 4) LMOE_DN(4);
    else if (nu <= 8) LMOE_DN(8);
    else if (nu <= 16) LMOE_DN(16);
    else return LMOE_ERR_SHAPE;
#undef LMOE_DN
    LMOE_RETURN_LAUNCH();
  }
  if (path != LMOE_PATH_MFMA) return LMOE_ERR_UNSUPPORTED;
  if (tile_off == nullptr) return LMOE_ERR_ARG;
  if (block_m != kBM) return LMOE_ERR_UNSUPPORTED;
  GemmArgs g{};
  g.topk = 1;
  g.offsets = offsets;
  g.sorted_pairs = sorted_pairs;
  g.tile_off = tile_off;
  g.meta = meta;
  g.P = n_slots;
  g.a = actb;
  g.w = w2;
  g.w_slot_stride = slot_elems_w2(H, I);
  g.N = H;
  g.K = I;
  g.out = yb;
  const int ub_tiles = n_pairs / kBM + max_active + 1;
  hipLaunchKernelGGL(grouped_gemm_kernel<kDown>, dim3(ub_tiles, (H + 127) / 128), dim3(256), 0,
                     stream, g);
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_grouped_mlp(const void* x, int T, int H, int I, int k,
                                const void* w13_slots, const void* w2_slots,
                                int n_slots, const int32_t* offsets,
                                const int32_t* sorted_pairs,
                                const int32_t* active, const int32_t* tile_off,
                                const int32_t* meta, int n_pairs, int block_m,
                                int path, void* act, void* y,
                                hipStream_t stream) {
  if (w2_slots == nullptr || y == nullptr) return LMOE_ERR_ARG;
  int st = lmoe_gateup_silu(x, T, H, I, k, w13_slots, n_slots, offsets, sorted_pairs, active,
                            tile_off, meta, n_pairs, block_m, path, act, stream);
  if (st != LMOE_OK) return st;
  return lmoe_down(act, H, I, w2_slots, n_slots, offsets, sorted_pairs, active, tile_off, meta,
                   n_pairs, block_m, path, y, stream);
}

extern "C" int lmoe_fused_moe_decode(const void* x, int T, int H, int I, int k,
                                     const void* w13_slots, const void* w2_slots,
                                     int n_slots, const uint16_t* w,
                                     const int32_t* offsets,
                                     const int32_t* sorted_pairs,
                                     const int32_t* row_idx,
                                     const int32_t* active, const int32_t* meta,
                                     const void* add, void* act, void* out,
                                     hipStream_t stream) {
  if (x == nullptr || w13_slots == nullptr || w2_slots == nullptr || w == nullptr ||
      offsets == nullptr || sorted_pairs == nullptr || row_idx == nullptr ||
      active == nullptr || meta == nullptr || act == nullptr || out == nullptr)
    return LMOE_ERR_ARG;
  if (T < 0 || H <= 0 || I <= 0 || k <= 0 || n_slots <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0 || I % 64 != 0 || I > 4096 || H > 8192) return LMOE_ERR_SHAPE;
  const int n_pairs = T * k;
  if (n_pairs > kFusedMaxPairs) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;
  const int max_active = n_pairs < n_slots ? n_pairs : n_slots;
  int st = launch_gateup_gemv(static_cast<const uint16_t*>(x), H, I, k,
                              static_cast<const uint16_t*>(w13_slots), offsets,
                              sorted_pairs, active, meta, max_active,
                              static_cast<uint16_t*>(act), stream);
  if (st != LMOE_OK) return st;
  dim3 grid((H + 3) / 4);
  const int nu = nu_for(I);
#define LMOE_DC(NU)                                                             \
  hipLaunchKernelGGL(down_combine_gemv_kernel<NU>, grid, dim3(256), 0, stream,  \
                     static_cast<const uint16_t*>(act), I, H, T, k,              \
                     static_cast<const uint16_t*>(w2_slots), offsets, active, meta, \
                     row_idx, w, static_cast<const uint16_t*>(add),              \
                     static_cast<uint16_t*>(out))
  if (nu <= 3) LMOE_DC(3);
  else if (nu <= 4) LMOE_DC(4);
  else if (nu <= 8) LMOE_DC(8);
  else if (nu <= 16) LMOE_DC(16);
  else return LMOE_ERR_SHAPE;
#undef LMOE_DC
  LMOE_RETURN_LAUNCH();
}

extern "C" int lmoe_combine(const void* y, const int32_t* row_idx,
                            const uint16_t* w, int T, int k, int H,
                            const void* add, void* out, hipStream_t stream) {
  if (y == nullptr || w == nullptr || out == nullptr) return LMOE_ERR_ARG;
  if (T < 0 || k <= 0 || H <= 0) return LMOE_ERR_ARG;
  if (H % 8 != 0) return LMOE_ERR_SHAPE;
  if (T == 0) return LMOE_OK;
  dim3 grid(T, (H + 2047) / 2048);
  hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, stream,
                     static_cast<const uint16_t*>(y), row_idx, w, T, k, H,
                     static_cast<const uint16_t*>(add), static_cast<uint16_t*>(out));
  LMOE_RETURN_LAUNCH();
}
