// Routing on the GPU: the router's top-k softmax, the counting sort of the (token, slot) pairs by
// expert, the per-expert offsets and the tile map.  All selection and ordering here is integer
// work and is exact: the same inputs give the same indices, offsets and permutation every run.
//
// Reference behaviour (paths into thinkube/meepsquared; TF: = transformers):
//   router       TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266 — softmax(fp32) -> topk -> renorm
//   sort/offsets src/meepsquared/_moe.py:77-87 — sort(expert_ids), histc, cumsum(int32), sentinels
//   tile map     src/meepsquared/_grouped.py:83-103
#include <mutex>

#include "common.hpp"

namespace mlora {

// ------------------------------------------------------------------------------------------------
// top-k softmax: L lanes per token (64 / L tokens per wave), lane g of a token holding the logits
// e = g + L*i, i < PL.  Every reduction over a token's lanes is a butterfly of DPP moves (quad
// permutations, then the half-row and row mirrors), so the k selection rounds never touch LDS.
// ------------------------------------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<bf16>(const bf16* p) { return (float)*p; }
template <>
__device__ __forceinline__ float load_logit<_Float16>(const _Float16* p) { return (float)*p; }

// A key whose unsigned order is (value descending, then index ascending) under max; never 0.
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

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
// The value of this lane's partner at step S of a butterfly over aligned groups of 2^(S+1) lanes:
// lane ^ 1, lane ^ 2 (quad permutations), then the mirror image within 8 and within 16 lanes (each
// pairs the two halves of the group reduced so far), then lane ^ 16 and lane ^ 32.
template <int S>
__device__ __forceinline__ uint32_t bfly(uint32_t v) {
  if constexpr (S == 0) return dpp_u32<0xB1>(v);        // quad_perm [1, 0, 3, 2]
  else if constexpr (S == 1) return dpp_u32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  else if constexpr (S == 2) return dpp_u32<0x141>(v);  // row_half_mirror
  else if constexpr (S == 3) return dpp_u32<0x140>(v);  // row_mirror
  else return (uint32_t)__shfl_xor((int)v, S == 4 ? 16 : 32, kWave);
}
// Reductions over a token's L lanes; every lane of the group ends with the same value (each step
// combines two equal-shaped partial results with a commutative operation).
template <int L, int S = 0>
__device__ __forceinline__ float group_max(float v) {
  if constexpr ((1 << S) >= L) return v;
  else return group_max<L, S + 1>(fmaxf(v, __uint_as_float(bfly<S>(__float_as_uint(v)))));
}
template <int L, int S = 0>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr ((1 << S) >= L) return v;
  else return group_sum<L, S + 1>(v + __uint_as_float(bfly<S>(__float_as_uint(v))));
}
template <int L, int S = 0>
__device__ __forceinline__ uint64_t group_max_key(uint64_t v) {
  if constexpr ((1 << S) >= L) {
    return v;
  } else {
    const uint64_t w = ((uint64_t)bfly<S>((uint32_t)(v >> 32)) << 32) | bfly<S>((uint32_t)v);
    return group_max_key<L, S + 1>(w > v ? w : v);
  }
}

constexpr int kTopkMaxE = 1024;

// torch.topk on the GPU returns the k selected values sorted by a bitonic network over 32 positions
// when k <= 32 (the k values in expert order — those above the k-th value first, then those equal to
// it — then empty positions); its comparator swaps a pair when "a above b and a present, or b empty"
// equals the comparator's direction flag, so equal values change places whenever a comparator with
// flag false meets them.  Reproduced here so the indices are those torch gives, ties included.
// Entries are codes rank << 8 | list position (rank: the first selection round that took this value,
// so a smaller rank is a larger value); an empty position has rank 0xFF.
constexpr int kTieNet = 32;

// The network run by a token's L lanes on the 32 positions, position i = lane + L·q held in c[q]: at each
// compare-exchange stage (merge size `size`, distance `stride`) position i meets i ^ stride — in this lane's
// other slot when stride >= L, else in lane ^ stride — and both keep the same one of the pair.  The pair's
// direction flag is bit `size` of its positions (false in the final merge).
template <int L>
__device__ __forceinline__ void tie_network(uint32_t (&c)[L >= kTieNet ? 1 : kTieNet / L], int gl) {
  constexpr int NQ = L >= kTieNet ? 1 : kTieNet / L;
  auto stage = [&](int size, int stride) {
    uint32_t other[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      other[q] = stride >= L ? c[q ^ (stride / L)] : (uint32_t)__shfl_xor((int)c[q], stride, kWave);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int i = gl + L * q;
      const bool lower = (i & stride) == 0;
      const uint32_t a = lower ? c[q] : other[q], b = lower ? other[q] : c[q];
      const bool swap = (a >> 8) < (b >> 8) || (b >> 8) == 0xFFu;  // a above b (so present), or b empty
      const bool flag = size < kTieNet && (i & size) != 0;
      if (swap == flag) c[q] = other[q];
    }
  };
#pragma unroll
  for (int size = 2; size < kTieNet; size *= 2)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride /= 2) stage(size, stride);
#pragma unroll
  for (int stride = kTieNet / 2; stride > 0; stride /= 2) stage(kTieNet, stride);
}

template <typename TL, typename TW, int L, int PL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const TL* __restrict__ logits, int64_t ld, int64_t T,
                                                           int E, int k, int renorm, int64_t* __restrict__ out_idx,
                                                           TW* __restrict__ out_w) {
  constexpr int G = kWave / L;  // tokens per wave
  constexpr int TB = 4 * G;     // tokens per block
  // the k selected experts per token for the reordering (k <= 32): index, probability, rank, then the
  // list positions in torch's order
  __shared__ int s_idx[TB][kTieNet];
  __shared__ float s_p[TB][kTieNet];
  __shared__ uint32_t s_code[TB][kTieNet];
  const int lane = threadIdx.x & 63, gl = lane & (L - 1);
  const int tok = (threadIdx.x >> 6) * G + lane / L;  // this lane's token within the block
  const int64_t t0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * G;
  // waves past T take no part in the work but reach every barrier
  const bool wave_live = t0 < T;
  const int64_t t = t0 + lane / L;
  const bool live = t < T;
  const bool reorder = k >= 2 && k <= kTieNet;
  float sel_sum = 0.f, sp[PL];
  int si[PL], sr[PL];
#pragma unroll
  for (int s = 0; s < PL; ++s) {
    sp[s] = 0.f;
    si[s] = 0;
    sr[s] = 0;
  }
  if (wave_live) {
    const TL* row = logits + (live ? t : 0) * ld;
    float v[PL];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = gl + L * i;
      v[i] = (live && e < E) ? load_logit(row + e) : -INFINITY;
      m = fmaxf(m, v[i]);
    }
    m = group_max<L>(m);
    float z = 0.f;
    uint64_t key[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = gl + L * i;
      // keyed on x - max in fp32, the softmax's exponent: equal keys are exactly equal probabilities
      const float d = v[i] - m;
      if (e < E) z += expf(d);
      key[i] = e < E ? rank_key(d, e) : 0;  // 0: absent or already taken
    }
    z = group_sum<L>(z);

    // round j: the largest key left over the token's lanes; lane j % L keeps it in its slot j / L,
    // with its rank (the first round that took an equal value)
    uint32_t prev = 0;
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < PL; ++i) best = key[i] > best ? key[i] : best;
      best = group_max_key<L>(best);
#pragma unroll
      for (int i = 0; i < PL; ++i) key[i] = key[i] == best ? 0 : key[i];
      const uint32_t ord = (uint32_t)(best >> 32);
      if (j == 0 || ord != prev) rank = j;
      prev = ord;
      const int idx = (int)(0xFFFFFFFFu - (uint32_t)best);
      const float p = expf(key_value(best)) / z;
      sel_sum += p;
      if (gl == (j & (L - 1))) {
#pragma unroll
        for (int s = 0; s < PL; ++s)
          if (s == j / L) {
            sp[s] = p;
            si[s] = idx;
            sr[s] = rank;
          }
      }
    }
    if (reorder) {
#pragma unroll
      for (int s = 0; s < PL; ++s) {
        const int j = s * L + gl;
        if (j < k) {
          s_idx[tok][j] = si[s];
          s_p[tok][j] = sp[s];
          s_code[tok][j] = (uint32_t)sr[s];
        }
      }
    }
  }
  if (reorder) {
    __syncthreads();
    // each selection's place in expert order: those above the k-th value by expert index, then those
    // equal to it (already in expert order, at the end of the list)
    int gpos[PL];
    if (wave_live) {
      const int rk = (int)s_code[tok][k - 1];
#pragma unroll
      for (int s = 0; s < PL; ++s) {
        const int j = s * L + gl;
        gpos[s] = j;
        if (j < k && sr[s] != rk) {
          int below = 0;
          for (int i = 0; i < rk; ++i) below += s_idx[tok][i] < si[s];
          gpos[s] = below;
        }
      }
    }
    __syncthreads();
    if (wave_live) {
#pragma unroll
      for (int s = 0; s < PL; ++s) {
        const int j = s * L + gl;
        if (j < k) s_code[tok][gpos[s]] = ((uint32_t)sr[s] << 8) | (uint32_t)j;
      }
    }
    __syncthreads();
    constexpr int NQ = L >= kTieNet ? 1 : kTieNet / L;
    uint32_t c[NQ];
    if (wave_live) {  // every lane of a live wave: the network exchanges values between lanes
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int i = gl + L * q;
        c[q] = i < k ? s_code[tok][i] : 0xFFFFu;  // (k <= 32: positions past 31 are always empty)
      }
      tie_network<L>(c, gl);
    }
    __syncthreads();  // every read of the gather order is done before it is overwritten
    if (wave_live) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int i = gl + L * q;
        if (i < k) s_code[tok][i] = c[q] & 0xFFu;  // output i takes list position c[q] & 0xFF
      }
    }
    __syncthreads();
  }
  if (live) {
#pragma unroll
    for (int s = 0; s < PL; ++s) {
      const int j = s * L + gl;
      if (j < k) {
        int ix = si[s];
        float p = sp[s];
        if (reorder) {
          const int from = (int)s_code[tok][j];
          ix = s_idx[tok][from];
          p = s_p[tok][from];
        }
        out_idx[t * k + j] = ix;
        out_w[t * k + j] = (TW)(renorm ? p / sel_sum : p);
      }
    }
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
// counting sort: one wave per chunk of 256 ids.  A histogram per chunk, one block that turns the
// (chunk, bin) counts into each chunk's first position per bin, then a stable scatter per chunk.
// ------------------------------------------------------------------------------------------------
constexpr int kSortSub = 4;                  // sub-chunks of 64 ids per chunk
constexpr int kSortChunk = kWave * kSortSub;  // ids per chunk (one wave, one workgroup)
constexpr int kScanThreads = 1024;

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

// The bins of this lane's ids in chunk `c` (all loaded before any is used); bin E+1 marks lanes past
// the end of the ids.
__device__ __forceinline__ void load_bins(const int64_t* ids, int64_t S, int E, int64_t c, int (&bins)[kSortSub]) {
  const int lane = threadIdx.x & 63;
  const int64_t base = c * kSortChunk;
  int64_t v[kSortSub];
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) {
    const int64_t i = base + sc * 64 + lane;
    v[sc] = i < S ? ids[i] : 0;
  }
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc) bins[sc] = base + sc * 64 + lane >= S ? E + 1 : bin_of(v[sc], E);
}

// ws[c][e] = how many ids of chunk c fall in bin e (bin E: the sentinels)
__global__ __launch_bounds__(kWave) void sort_hist_kernel(const int64_t* __restrict__ ids, int64_t S, int E,
                                                          int32_t* __restrict__ ws) {
  extern __shared__ int cnt[];  // E + 1
  const int lane = threadIdx.x;
  for (int e = lane; e <= E; e += kWave) cnt[e] = 0;
  __syncthreads();
  int bins[kSortSub];
  load_bins(ids, S, E, blockIdx.x, bins);
#pragma unroll
  for (int sc = 0; sc < kSortSub; ++sc)
    if (bins[sc] <= E) atomicAdd(&cnt[bins[sc]], 1);
  __syncthreads();
  for (int e = lane; e <= E; e += kWave) ws[(int64_t)blockIdx.x * (E + 1) + e] = cnt[e];
}

constexpr int kScanBatch = 16;  // chunks per load batch
constexpr int kScanGroups = 4;  // 64-bin groups loaded together

// The NP ranges of chunks the scan splits each bin's column into: as many as fit 48 KB of LDS.
__host__ __device__ inline int scan_ranges(int E) {
  const int G = (E + 1 + 63) / 64;
  int np = 16;
  while (np > 1 && np * G * 64 * (int)sizeof(int) > 48 * 1024) np >>= 1;
  return np;
}

// The counts ws[c][g*64 + l] of chunks cb .. cb + kScanBatch - 1 (those below c1) for the groups
// g0 .. g0 + kScanGroups - 1 (those up to bin E): kScanGroups x kScanBatch loads in flight at once.
__device__ __forceinline__ void scan_load(const int32_t* ws, int E, int l, int g0, int cb, int c1,
                                          int (&val)[kScanGroups][kScanBatch]) {
#pragma unroll
  for (int gi = 0; gi < kScanGroups; ++gi)
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const int e = (g0 + gi) * 64 + l, c = cb + u;
      val[gi][u] = c < c1 && e <= E ? ws[(int64_t)c * (E + 1) + e] : 0;
    }
}

// One block: start[e] = the first row of bin e (an exclusive scan of the bins' totals), offsets, then
// every ws[c][e] replaced by the first row of chunk c's ids of bin e.  Thread (w, l), w < NP, handles
// bin g*64 + l of every 64-bin group g over the w-th of NP ranges of chunks (pass 1: its sums; pass 2:
// the running first rows written back); the ranges' sums are scanned down each bin's column in LDS.
__global__ __launch_bounds__(kScanThreads) void sort_scan_kernel(int32_t* __restrict__ ws, int nch, int E,
                                                                 int32_t* __restrict__ offsets, int bm,
                                                                 int32_t* tile_expert, int32_t* tile_row,
                                                                 int32_t* tiles, int64_t max_tiles) {
  extern __shared__ int sh[];
  int* start = sh;              // E + 2: per-bin totals, scanned into starts
  int* tstart = sh + (E + 2);   // E + 1
  int* tmp = tstart + (E + 1);  // 17
  int* part = tmp + 17;         // [G][NP][64]: each range's count of each bin, then its first row
  const int NP = scan_ranges(E), G = (E + 1 + 63) / 64;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int per = (nch + NP - 1) / NP;
  const int c0 = w < NP ? min(w * per, nch) : nch, c1 = w < NP ? min(c0 + per, nch) : nch;
  for (int g0 = 0; g0 < G; g0 += kScanGroups) {
    int sum[kScanGroups] = {};
    for (int cb = c0; cb < c1; cb += kScanBatch) {
      int val[kScanGroups][kScanBatch];
      scan_load(ws, E, l, g0, cb, c1, val);
#pragma unroll
      for (int gi = 0; gi < kScanGroups; ++gi)
#pragma unroll
        for (int u = 0; u < kScanBatch; ++u) sum[gi] += val[gi][u];
    }
    if (w < NP) {
#pragma unroll
      for (int gi = 0; gi < kScanGroups; ++gi)
        if (g0 + gi < G) part[((g0 + gi) * NP + w) * 64 + l] = sum[gi];
    }
  }
  __syncthreads();
  for (int e = tid; e <= E; e += kScanThreads) {
    const int g = e >> 6, ll = e & 63;
    int tot = 0;
    for (int q = 0; q < NP; ++q) tot += part[(g * NP + q) * 64 + ll];
    start[e] = tot;
  }
  __syncthreads();
  block_exclusive_scan(start, E + 1, tmp);  // start[e] = first row of bin e; start[E] = offsets[E-1]
  for (int e = tid + 1; e <= E; e += kScanThreads) offsets[e - 1] = start[e];
  for (int e = tid; e <= E; e += kScanThreads) {  // each bin's column: the first row of each range
    const int g = e >> 6, ll = e & 63;
    int run = start[e];
    for (int q = 0; q < NP; ++q) {
      const int c = part[(g * NP + q) * 64 + ll];
      part[(g * NP + q) * 64 + ll] = run;
      run += c;
    }
  }
  __syncthreads();
  for (int g0 = 0; g0 < G; g0 += kScanGroups) {
    int run[kScanGroups];
#pragma unroll
    for (int gi = 0; gi < kScanGroups; ++gi) run[gi] = w < NP && g0 + gi < G ? part[((g0 + gi) * NP + w) * 64 + l] : 0;
    for (int cb = c0; cb < c1; cb += kScanBatch) {
      int val[kScanGroups][kScanBatch];
      scan_load(ws, E, l, g0, cb, c1, val);
#pragma unroll
      for (int gi = 0; gi < kScanGroups; ++gi)
#pragma unroll
        for (int u = 0; u < kScanBatch; ++u) {
          const int e = (g0 + gi) * 64 + l, c = cb + u;
          if (c < c1 && e <= E) ws[(int64_t)c * (E + 1) + e] = run[gi];
          run[gi] += val[gi][u];
        }
    }
  }
  __syncthreads();
  if (tile_expert != nullptr) write_tile_map(start, tstart, tmp, E, bm, tile_expert, tile_row, tiles, max_tiles);
}

// Chunk c's ids in order: each id's position is its bin's next free row, taken a sub-chunk of 64 at
// a time (lanes of one bin in lane order), so equal ids keep their input order.
__global__ __launch_bounds__(kWave) void sort_scatter_kernel(const int64_t* __restrict__ ids, int64_t S, int E,
                                                             int nbits, const int32_t* __restrict__ ws,
                                                             int64_t* __restrict__ perm, int64_t* __restrict__ inv) {
  extern __shared__ int cnt[];  // E + 1: the next row of each bin
  const int lane = threadIdx.x;
  int bins[kSortSub];
  load_bins(ids, S, E, blockIdx.x, bins);
  for (int e = lane; e <= E; e += kWave) cnt[e] = ws[(int64_t)blockIdx.x * (E + 1) + e];
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortChunk;
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
  if (E < 1 || E > kTopkMaxE) return fail("route_topk: E=%d outside [1, %d]", E, kTopkMaxE);
  if (k < 1 || k > E || k > 64) return fail("route_topk: k=%d outside [1, min(E=%d, 64)]", k, E);
  if (ld_logits < E) return fail("route_topk: ld_logits=%lld < E=%d", (long long)ld_logits, E);
  if (T == 0) return 0;
  hipStream_t s = as_stream(stream);
  // lanes per token L and logits per lane PL: 8 logits per lane up to E = 512
  const int L = E <= 32 ? 4 : E <= 64 ? 8 : E <= 128 ? 16 : E <= 256 ? 32 : 64;
  const int64_t waves = (T + kWave / L - 1) / (kWave / L);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
#define MLORA_TOPK_LP(TL, TW, L_, PL)                                                                      \
  hipLaunchKernelGGL((topk_softmax_kernel<TL, TW, L_, PL>), grid, block, 0, s, (const TL*)logits, ld_logits, T, \
                     E, k, renorm, out_idx, (TW*)out_w)
#define MLORA_TOPK(TL, TW)                                                                                     \
  do {                                                                                                         \
    if (E <= 8) MLORA_TOPK_LP(TL, TW, 4, 2);                                                                   \
    else if (E <= 32) MLORA_TOPK_LP(TL, TW, 4, 8);                                                             \
    else if (E <= 64) MLORA_TOPK_LP(TL, TW, 8, 8);                                                             \
    else if (E <= 128) MLORA_TOPK_LP(TL, TW, 16, 8);                                                           \
    else if (E <= 256) MLORA_TOPK_LP(TL, TW, 32, 8);                                                           \
    else if (E <= 512) MLORA_TOPK_LP(TL, TW, 64, 8);                                                           \
    else MLORA_TOPK_LP(TL, TW, 64, 16);                                                                        \
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
#undef MLORA_TOPK_LP
  return launch_status("route_topk");
}

extern "C" size_t mlora_route_sort_workspace_bytes(int64_t S, int E) {
  const int64_t nch = S > 0 ? (S + kSortChunk - 1) / kSortChunk : 1;
  return (size_t)nch * (size_t)(E + 1) * sizeof(int32_t);
}

// The sort proper, on the caller's workspace ws (need bytes, checked by the entry points).
static int route_sort(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv, int32_t* offsets,
                      int block_m, int32_t* tile_expert, int32_t* tile_row, int32_t* tiles, int64_t max_tiles,
                      int32_t* ws, hipStream_t s) {
  const int nch = (int)(S > 0 ? (S + kSortChunk - 1) / kSortChunk : 0);
  const int nbits = nbits_for(E);
  const size_t sh_bins = (size_t)(E + 1) * sizeof(int);
  if (nch > 0) {
    hipLaunchKernelGGL(sort_hist_kernel, dim3(nch), dim3(kWave), sh_bins, s, ids, S, E, ws);
    if (int rc = launch_status("route_sort/hist")) return rc;
  }
  const size_t sh_scan = (size_t)((E + 2) + (E + 1) + 17 + ((E + 1 + 63) / 64) * scan_ranges(E) * 64) * sizeof(int);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(kScanThreads), sh_scan, s, ws, nch, E, offsets, block_m,
                     tile_expert, tile_row, tiles, max_tiles);
  if (int rc = launch_status("route_sort/scan")) return rc;
  if (nch > 0) {
    hipLaunchKernelGGL(sort_scatter_kernel, dim3(nch), dim3(kWave), sh_bins, s, ids, S, E, nbits, ws, perm, inv);
    if (int rc = launch_status("route_sort/scatter")) return rc;
  }
  return 0;
}

static int route_sort_check(int64_t S, int E, int block_m, const int32_t* tile_expert, const int32_t* tile_row,
                            const int32_t* tiles, int64_t max_tiles) {
  if (S < 0 || S >= ((int64_t)1 << 31)) return fail("route_sort: S=%lld outside [0, 2^31)", (long long)S);
  if (E < 1 || E > 2048) return fail("route_sort: E=%d outside [1, 2048]", E);
  if (tile_expert != nullptr && (block_m < 1 || tile_row == nullptr || tiles == nullptr || max_tiles < 0))
    return fail("route_sort: the tile map needs block_m >= 1, tile_row, tiles and max_tiles >= 0");
  return 0;
}

extern "C" int mlora_route_sort(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv, int32_t* offsets,
                                int block_m, int32_t* tile_expert, int32_t* tile_row, int32_t* tiles,
                                int64_t max_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = route_sort_check(S, E, block_m, tile_expert, tile_row, tiles, max_tiles)) return rc;
  const size_t need = mlora_route_sort_workspace_bytes(S, E);
  if (workspace == nullptr || workspace_bytes < need)
    return fail("route_sort: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  return route_sort(ids, S, E, perm, inv, offsets, block_m, tile_expert, tile_row, tiles, max_tiles,
                    (int32_t*)workspace, as_stream(stream));
}

// ------------------------------------------------------------------------------------------------
// The sort for callers that cannot allocate (HIP graph capture, serving loops): the per-chunk
// histograms live in this array, one per GPU, held until the process ends.  Host code never uses the
// array's name as an address (on the host it is a stand-in, not device memory): the device address is
// taken with hipGetSymbolAddress once per device, with that device current, and kept.  The sort writes
// every entry it later reads, so nothing needs clearing between calls; calls that overlap on one GPU
// (two streams at once) share the array and race.
// ------------------------------------------------------------------------------------------------
constexpr size_t kSortScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[kSortScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// the scratch array's device address on the current device, or nullptr (the error recorded)
static int32_t* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail("route_sort_noalloc: no current device (or device index %d past %d)", dev, kMaxDevices - 1);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      fail("route_sort_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
           hipGetErrorString(err));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return (int32_t*)g_scratch_ptr[dev];
}

extern "C" int mlora_route_sort_noalloc(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv,
                                        int32_t* offsets, int block_m, int32_t* tile_expert, int32_t* tile_row,
                                        int32_t* tiles, int64_t max_tiles, void* stream) {
  clear_error();
  if (int rc = route_sort_check(S, E, block_m, tile_expert, tile_row, tiles, max_tiles)) return rc;
  const size_t need = mlora_route_sort_workspace_bytes(S, E);
  if (need > kSortScratchBytes)
    return fail("route_sort_noalloc: S=%lld ids over E=%d experts need %zu bytes of scratch, past its %zu "
                "(use mlora_route_sort with a workspace)", (long long)S, E, need, kSortScratchBytes);
  int32_t* ws = scratch_on_current_device();
  if (ws == nullptr) return 1;
  return route_sort(ids, S, E, perm, inv, offsets, block_m, tile_expert, tile_row, tiles, max_tiles, ws,
                    as_stream(stream));
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
