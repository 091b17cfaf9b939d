// Routing on the GPU: the router's top-k softmax, the counting sort of the (token, slot) pairs by
// expert, the per-expert offsets and the tile map.  All selection and ordering here is integer
// work and is exact: the same inputs give the same indices, offsets and permutation every run.
//
// Reference behaviour (paths into thinkube/meepsquared; TF: = transformers):
//   router       TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266 — softmax(fp32) -> topk -> renorm
//   sort/offsets src/meepsquared/_moe.py:77-87 — sort(expert_ids), histc, cumsum(int32), sentinels
//   tile map     src/meepsquared/_grouped.py:83-103
#include "common.hpp"

namespace mlora {

// ------------------------------------------------------------------------------------------------
// top-k softmax: one wave per token, each lane holding the logits e = lane + 64*i
// ------------------------------------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<bf16>(const bf16* p) { return (float)*p; }
template <>
__device__ __forceinline__ float load_logit<_Float16>(const _Float16* p) { return (float)*p; }

// A key whose unsigned order is (value descending, then index ascending) under max.
__device__ __forceinline__ uint64_t rank_key(float v, int idx) {
  uint32_t b = __float_as_uint(v + 0.0f);  // -0 and +0 are one value
  uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ float key_value(uint64_t key) {
  uint32_t ord = (uint32_t)(key >> 32);
  uint32_t b = (ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord;
  return __uint_as_float(b);
}

constexpr int kTopkMaxPerLane = 16;  // E <= 1024

template <typename TL, typename TW, int PL>  // PL: logits per lane, ceil(E / 64)
__global__ __launch_bounds__(256) void topk_softmax_kernel(const TL* __restrict__ logits, int64_t ld, int64_t T,
                                                           int E, int k, int renorm, int64_t* __restrict__ out_idx,
                                                           TW* __restrict__ out_w) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const TL* row = logits + t * ld;
  float v[PL];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = lane + 64 * i;
    v[i] = (e < E) ? load_logit(row + e) : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  m = wave_max(m);
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = lane + 64 * i;
    if (e < E) z += expf(v[i] - m);
  }
  z = wave_sum(z);

  uint32_t taken = 0;
  float sel_sum = 0.f, my_p = 0.f;
  int my_idx = 0;
  for (int j = 0; j < k; ++j) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((taken >> i) & 1u)) {
        uint64_t key = rank_key(v[i], e);
        best = key > best ? key : best;
      }
    }
    best = wave_max_u64(best);
    const int idx = (int)(0xFFFFFFFFu - (uint32_t)best);
    if ((idx & 63) == lane) taken |= 1u << (idx >> 6);
    const float p = expf(key_value(best) - m) / z;
    sel_sum += p;
    if (lane == j) {
      my_p = p;
      my_idx = idx;
    }
  }
  if (lane < k) {
    const float w = renorm ? my_p / sel_sum : my_p;
    out_idx[t * k + lane] = my_idx;
    out_w[t * k + lane] = (TW)w;
  }
}

// ------------------------------------------------------------------------------------------------
// block-wide exclusive scan of an int array in LDS (blockDim.x a multiple of 64); returns the total
// ------------------------------------------------------------------------------------------------
__device__ int block_exclusive_scan(int* arr, int n, int* tmp /* blockDim/64 + 1 ints */) {
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, w = tid >> 6;
  const int per = (n + nt - 1) / nt;
  const int beg = min(tid * per, n), end = min(beg + per, n);
  int s = 0;
  for (int i = beg; i < end; ++i) s += arr[i];
  int v = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  if (lane == 63) tmp[w] = v;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < nt / 64; ++i) {
      int c = tmp[i];
      tmp[i] = run;
      run += c;
    }
    tmp[nt / 64] = run;
  }
  __syncthreads();
  int excl = v - s + tmp[w];
  for (int i = beg; i < end; ++i) {
    int c = arr[i];
    arr[i] = excl;
    excl += c;
  }
  const int total = tmp[nt / 64];
  __syncthreads();
  return total;
}

// The tile map from the experts' row starts start[0..E] (start[E] = the end of the last expert):
// the reference's formula (src/meepsquared/_grouped.py:97-102) for every entry, the spares included.
__device__ void write_tile_map(const int* start, int* tstart /* E+1 */, int* tmp, int E, int bm,
                               int32_t* tile_expert, int32_t* tile_row, int32_t* tiles, int64_t max_tiles) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) tstart[e] = (start[e + 1] - start[e] + bm - 1) / bm;
  __syncthreads();
  const int total = block_exclusive_scan(tstart, E, tmp);
  if (threadIdx.x == 0) {
    tstart[E] = total;
    tiles[0] = total;
  }
  __syncthreads();
  for (int64_t t = threadIdx.x; t < max_tiles; t += blockDim.x) {
    // searchsorted(tile_ends, t, right=True): the first expert whose tiles end after t
    int lo = 0, hi = E;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((int64_t)tstart[mid + 1] <= t) lo = mid + 1; else hi = mid;
    }
    const int e = lo < E ? lo : E - 1;
    tile_expert[t] = e;
    tile_row[t] = (int32_t)((int64_t)start[e] + (t - (int64_t)tstart[e]) * bm);
  }
}

__global__ __launch_bounds__(1024) void tile_map_kernel(const int32_t* __restrict__ offsets, int E, int bm,
                                                        int32_t* tile_expert, int32_t* tile_row, int32_t* tiles,
                                                        int64_t max_tiles) {
  extern __shared__ int sh[];
  int* start = sh;               // E + 1
  int* tstart = sh + (E + 1);    // E + 1
  int* tmp = tstart + (E + 1);   // 17
  for (int e = threadIdx.x; e <= E; e += blockDim.x) start[e] = e == 0 ? 0 : offsets[e - 1];
  __syncthreads();
  write_tile_map(start, tstart, tmp, E, bm, tile_expert, tile_row, tiles, max_tiles);
}

// ------------------------------------------------------------------------------------------------
// counting sort: histogram per block, a scan over (bin, block), a stable scatter
// ------------------------------------------------------------------------------------------------
constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortSub = 16;                                 // sub-chunks of 64 per wave
constexpr int kSortChunk = kSortThreads * kSortSub;           // ids per block

__device__ __forceinline__ int bin_of(int64_t id, int E) { return (id >= 0 && id < E) ? (int)id : E; }

// The lanes of this wave whose bin equals this lane's (all 64 lanes take part).
__device__ __forceinline__ uint64_t same_bin(int bin, int nbits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    const int bit = (bin >> b) & 1;
    const uint64_t set = __ballot(bit);
    m &= bit ? set : ~set;
  }
  return m;
}

// The bins of this lane's ids in the wave's 1024 (all loaded before any is used: one memory round
// trip, not one per sub-chunk); bin E+1 marks lanes past the end of the ids.
__device__ __forceinline__ void load_bins(const int64_t* ids, int64_t S, int E, int64_t base, int (&bins)[kSortSub]) {
  const int lane = threadIdx.x & 63;
  int64_t v[kSortSub];
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) {
    const int64_t i = base + sc * 64 + lane;
    v[sc] = i < S ? ids[i] : -2;
  }
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) bins[sc] = v[sc] == -2 && base + sc * 64 + lane >= S ? E + 1 : bin_of(v[sc], E);
}

// Per-wave histogram of the wave's 1024 ids into cnt[0..E] (bin E = sentinels); bin E+1 is not counted.
__device__ void wave_histogram(const int64_t* ids, int64_t S, int E, int nbits, int64_t base, int* cnt) {
  const int lane = threadIdx.x & 63;
  int bins[kSortSub];
  load_bins(ids, S, E, base, bins);
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) {
    const int bin = bins[sc];
    const uint64_t mask = same_bin(bin, nbits);
    const int leader = 63 - __builtin_clzll(mask);
    if (lane == leader && bin <= E) cnt[bin] += __builtin_popcountll(mask);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(const int64_t* __restrict__ ids, int64_t S, int E,
                                                                 int nbits, int32_t* __restrict__ ws) {
  extern __shared__ int sh[];  // kSortWaves x (E+1)
  const int w = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kSortWaves * (E + 1); i += kSortThreads) sh[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortChunk + (int64_t)w * (kSortChunk / kSortWaves);
  wave_histogram(ids, S, E, nbits, base, sh + w * (E + 1));
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kSortThreads) {
    int s = 0;
    for (int ww = 0; ww < kSortWaves; ++ww) s += sh[ww * (E + 1) + e];
    ws[(int64_t)blockIdx.x * (E + 1) + e] = s;
  }
}

// One block: per bin, the exclusive sum over blocks (in place in ws), then the bins' starts added;
// offsets and, when asked, the tile map.
__global__ __launch_bounds__(1024) void sort_scan_kernel(int32_t* __restrict__ ws, int nblk, int E,
                                                         int32_t* __restrict__ offsets, int bm, int32_t* tile_expert,
                                                         int32_t* tile_row, int32_t* tiles, int64_t max_tiles) {
  extern __shared__ int sh[];
  int* start = sh;              // E + 2: per-bin totals, scanned into starts
  int* tstart = sh + (E + 2);   // E + 1
  int* tmp = tstart + (E + 1);  // 17
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    int s = 0;
    for (int b = 0; b < nblk; ++b) {
      const int c = ws[(int64_t)b * (E + 1) + e];
      ws[(int64_t)b * (E + 1) + e] = s;
      s += c;
    }
    start[e] = s;
  }
  __syncthreads();
  block_exclusive_scan(start, E + 1, tmp);  // start[e] = first row of bin e; start[E] = offsets[E-1]
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    const int st = start[e];
    for (int b = 0; b < nblk; ++b) ws[(int64_t)b * (E + 1) + e] += st;
    if (e > 0) offsets[e - 1] = st;
  }
  __syncthreads();
  if (tile_expert != nullptr) write_tile_map(start, tstart, tmp, E, bm, tile_expert, tile_row, tiles, max_tiles);
}

__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(const int64_t* __restrict__ ids, int64_t S, int E,
                                                                    int nbits, const int32_t* __restrict__ ws,
                                                                    int64_t* __restrict__ perm,
                                                                    int64_t* __restrict__ inv) {
  extern __shared__ int sh[];  // kSortWaves x (E+1)
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < kSortWaves * (E + 1); i += kSortThreads) sh[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortChunk + (int64_t)w * (kSortChunk / kSortWaves);
  int* cnt = sh + w * (E + 1);
  wave_histogram(ids, S, E, nbits, base, cnt);
  __syncthreads();
  // each wave's first position per bin: the block's base, then the earlier waves' counts
  for (int e = threadIdx.x; e <= E; e += kSortThreads) {
    int run = ws[(int64_t)blockIdx.x * (E + 1) + e];
    for (int ww = 0; ww < kSortWaves; ++ww) {
      const int c = sh[ww * (E + 1) + e];
      sh[ww * (E + 1) + e] = run;
      run += c;
    }
  }
  __syncthreads();
  int bins[kSortSub];
  load_bins(ids, S, E, base, bins);
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) {
    const int64_t i = base + sc * 64 + lane;
    const int bin = bins[sc];
    const uint64_t mask = same_bin(bin, nbits);
    const int leader = 63 - __builtin_clzll(mask);
    const int rank = __builtin_popcountll(mask & ((1ull << lane) - 1ull));
    if (bin <= E) {
      const int64_t pos = (int64_t)cnt[bin] + rank;
      perm[pos] = i;
      if (inv != nullptr) inv[i] = pos;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == leader && bin <= E) cnt[bin] += __builtin_popcountll(mask);
    __builtin_amdgcn_wave_barrier();
  }
}

static int nbits_for(int E) { return 32 - __builtin_clz((unsigned)(E + 1)); }

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_route_topk(const void* logits, int logits_dtype, int64_t ld_logits, int64_t T, int E, int k,
                                int renorm, int64_t* out_idx, void* out_w, int w_dtype, void* stream) {
  clear_error();
  if (T < 0) return fail("route_topk: T=%lld is negative", (long long)T);
  if (E < 1 || E > 64 * kTopkMaxPerLane) return fail("route_topk: E=%d outside [1, %d]", E, 64 * kTopkMaxPerLane);
  if (k < 1 || k > E || k > 64) return fail("route_topk: k=%d outside [1, min(E=%d, 64)]", k, E);
  if (ld_logits < E) return fail("route_topk: ld_logits=%lld < E=%d", (long long)ld_logits, E);
  if (T == 0) return 0;
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  hipStream_t s = as_stream(stream);
#define MLORA_TOPK_PL(TL, TW, PL)                                                                        \
  hipLaunchKernelGGL((topk_softmax_kernel<TL, TW, PL>), grid, block, 0, s, (const TL*)logits, ld_logits, T, E, \
                     k, renorm, out_idx, (TW*)out_w)
#define MLORA_TOPK(TL, TW)                                                                                     \
  do {                                                                                                         \
    if (E <= 64) MLORA_TOPK_PL(TL, TW, 1);                                                                     \
    else if (E <= 128) MLORA_TOPK_PL(TL, TW, 2);                                                               \
    else if (E <= 256) MLORA_TOPK_PL(TL, TW, 4);                                                               \
    else if (E <= 512) MLORA_TOPK_PL(TL, TW, 8);                                                               \
    else MLORA_TOPK_PL(TL, TW, kTopkMaxPerLane);                                                               \
  } while (0)
  if (w_dtype != MLORA_DT_BF16 && w_dtype != MLORA_DT_F32) return fail("route_topk: w_dtype %d is not bf16/f32", w_dtype);
  const bool wf = w_dtype == MLORA_DT_F32;
  switch (logits_dtype) {
    case MLORA_DT_F32: if (wf) MLORA_TOPK(float, float); else MLORA_TOPK(float, bf16); break;
    case MLORA_DT_BF16: if (wf) MLORA_TOPK(bf16, float); else MLORA_TOPK(bf16, bf16); break;
    case MLORA_DT_F16: if (wf) MLORA_TOPK(_Float16, float); else MLORA_TOPK(_Float16, bf16); break;
    default: return fail("route_topk: logits dtype %d is not bf16/f16/f32", logits_dtype);
  }
#undef MLORA_TOPK
#undef MLORA_TOPK_PL
  return launch_status("route_topk");
}

extern "C" size_t mlora_route_sort_workspace_bytes(int64_t S, int E) {
  const int64_t nblk = S > 0 ? (S + kSortChunk - 1) / kSortChunk : 1;
  return (size_t)nblk * (size_t)(E + 1) * sizeof(int32_t);
}

extern "C" int mlora_route_sort(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv, int32_t* offsets,
                                int block_m, int32_t* tile_expert, int32_t* tile_row, int32_t* tiles,
                                int64_t max_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (S < 0 || S >= ((int64_t)1 << 31)) return fail("route_sort: S=%lld outside [0, 2^31)", (long long)S);
  if (E < 1 || E > 2048) return fail("route_sort: E=%d outside [1, 2048]", E);
  if (tile_expert != nullptr && (block_m < 1 || tile_row == nullptr || tiles == nullptr || max_tiles < 0))
    return fail("route_sort: the tile map needs block_m >= 1, tile_row, tiles and max_tiles >= 0");
  const size_t need = mlora_route_sort_workspace_bytes(S, E);
  if (workspace == nullptr || workspace_bytes < need)
    return fail("route_sort: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  const int nblk = (int)(S > 0 ? (S + kSortChunk - 1) / kSortChunk : 0);
  int32_t* ws = (int32_t*)workspace;
  const int nbits = nbits_for(E);
  const size_t sh_waves = (size_t)kSortWaves * (E + 1) * sizeof(int);
  if (nblk > 0) {
    hipLaunchKernelGGL(sort_hist_kernel, dim3(nblk), dim3(kSortThreads), sh_waves, s, ids, S, E, nbits, ws);
    if (int rc = launch_status("route_sort/hist")) return rc;
  }
  const size_t sh_scan = (size_t)((E + 2) + (E + 1) + 17) * sizeof(int);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), sh_scan, s, ws, nblk, E, offsets, block_m, tile_expert,
                     tile_row, tiles, max_tiles);
  if (int rc = launch_status("route_sort/scan")) return rc;
  if (nblk > 0) {
    hipLaunchKernelGGL(sort_scatter_kernel, dim3(nblk), dim3(kSortThreads), sh_waves, s, ids, S, E, nbits, ws, perm,
                       inv);
    if (int rc = launch_status("route_sort/scatter")) return rc;
  }
  return 0;
}

extern "C" int mlora_tile_map(const int32_t* offsets, int E, int64_t rows, int block_m, int32_t* tile_expert,
                              int32_t* tile_row, int32_t* tiles, int64_t max_tiles, void* stream) {
  clear_error();
  if (E < 1 || E > 4096) return fail("tile_map: E=%d outside [1, 4096]", E);
  if (block_m < 1) return fail("tile_map: block_m=%d < 1", block_m);
  if (rows < 0 || max_tiles < 0) return fail("tile_map: negative rows or max_tiles");
  const size_t sh = (size_t)(2 * (E + 1) + 17) * sizeof(int);
  hipLaunchKernelGGL(tile_map_kernel, dim3(1), dim3(1024), sh, as_stream(stream), offsets, E, block_m, tile_expert,
                     tile_row, tiles, max_tiles);
  return launch_status("tile_map");
}
