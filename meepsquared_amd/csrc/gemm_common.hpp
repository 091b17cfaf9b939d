// Definitions shared by the grouped-product kernels (grouped_gemm.hip, grouped_gemm_bf16.hip):
// the argument block, buffer-resource loads, and the tile map each persistent workgroup derives
// from the experts' row offsets.
#pragma once

#include "common.hpp"

namespace mlora {

constexpr int kMaxRank = 64;
constexpr int kXcds = 8;
constexpr uint32_t kOob = 0x80000000u;  // an offset past every resource's end: the load returns zero

enum { W_BF16 = 0, W_FP8 = 1, W_NF4 = 2 };

struct GemmArgs {
  const bf16* x;
  int64_t ldx;
  const int64_t* gather;  // NULL, or row r of the product is row gather[r] / gk of x (x has xrows rows)
  int gk;
  int64_t xrows;
  const void* row_scale;  // NULL, or (with gather) output row r is multiplied by row_scale[gather[r]]
  int row_scale_dt;       // MLORA_DT_BF16 or MLORA_DT_F32
  const uint8_t* w;      // bytes
  int64_t w_se, w_sk, w_sn;  // elements
  const float* scale;
  int64_t scale_se;
  int scale_kind;
  const uint8_t* nf4_q;
  const float* nf4_absmax2;
  const float* nf4_code2;
  const float* nf4_offset;
  const float* nf4_code;
  const bf16* at;        // A_e^T: [e][r][k], k contiguous
  int64_t at_se, at_sr;
  const bf16* bt;        // B_e^T: [e][n][r], r contiguous
  int64_t bt_se, bt_sn;
  int rank;              // a multiple of 16
  float scaling;
  const bf16* bias;
  int64_t bias_se;
  bf16* out;
  int64_t ldo;
  bf16* low;
  int64_t ldl;
  const int32_t* offsets;
  int64_t rows;
  int E, K, N;
  // The adapter gradient sum over each expert's rows of l[row] (x) x[row] (rank 16), fused into the
  // product (bf16 stacks): NULL dbl, or rows x 16 values of l, and the fp32 workspace of per-tile
  // partial sums, [slot][16][K].
  const bf16* dbl;
  int64_t dbl_ld;
  float* dbw;
  bf16* dbo;                 // the gradient (experts, K, 16) by its strides, written by the finishing launch
  int64_t dbo_se, dbo_sk, dbo_sr;
  // SwiGLU of the product fused into its epilogue (the DMA-fed product): NULL act, or N = 2 swi columns
  // (gate, then up) and act[row][c] = bf16(silu(out[row][c]) · out[row][swi + c]) of the stored bf16 values,
  // row stride lda.  Each 256-column tile then holds 128 gate columns and the 128 up columns that pair with
  // them.
  bf16* act;
  int64_t lda;
  int swi;
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int64_t cap = 0x7FFFFFF0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(bytes < cap ? bytes : cap), 0x00020000);
}
__device__ __forceinline__ u32x4 ld128(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ u32x2 ld64(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld32(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }

// The tile map in LDS: starts[e] = expert e's first row (clamped into [0, rows]; starts[E] = the end
// of the last expert) and tstart[e] = its first tile of bm rows (tstart[E] = the tile count).
// Called by every thread of the workgroup; ends with the map complete and visible.
template <int NT>
__device__ __forceinline__ void build_tile_map(const GemmArgs& p, int bm, int* starts, int* tstart, int tid) {
  const int E = p.E;
  for (int e = tid; e <= E; e += NT) {
    const int64_t o = e == 0 ? 0 : (int64_t)p.offsets[e - 1];
    starts[e] = (int)(o < 0 ? 0 : (o > p.rows ? p.rows : o));
  }
  __syncthreads();
  for (int e = tid; e < E; e += NT) {
    const int c = max(starts[e + 1] - starts[e], 0);
    tstart[e] = (c + bm - 1) / bm;
  }
  __syncthreads();
  if (tid < 64) {  // exclusive scan of tstart[0..E) by one wave, 64 at a time
    const int lane = tid;
    int run = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      const int v = e < E ? tstart[e] : 0;
      int incl = v;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
      }
      if (e < E) tstart[e] = run + incl - v;
      run += __shfl(incl, 63, 64);
    }
    if (lane == 0) tstart[E] = run;
  }
  __syncthreads();
}

// One work item (tile t, column block nblk) decoded from the map, as wave-uniform scalars.
struct Item {
  int e, nblk, n0, mrows;
  int64_t row0;
};

__device__ __forceinline__ Item decode_item(int64_t item, int nb, int E, int bm, int bn, const int* starts,
                                            const int* tstart) {
  const int t = (int)(item / nb);
  Item it;
  it.nblk = (int)(item - (int64_t)t * nb);
  int lo = 0, hi = E - 1;  // the expert e with tstart[e] <= t < tstart[e+1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tstart[mid] <= t) lo = mid; else hi = mid - 1;
  }
  // values read from LDS are per-lane to the compiler: make them wave-uniform (SGPRs)
  it.e = __builtin_amdgcn_readfirstlane(lo);
  const int e_start = __builtin_amdgcn_readfirstlane(starts[it.e]);
  const int e_end = __builtin_amdgcn_readfirstlane(starts[it.e + 1]);
  const int e_t0 = __builtin_amdgcn_readfirstlane(tstart[it.e]);
  it.row0 = (int64_t)e_start + (int64_t)(t - e_t0) * bm;
  it.mrows = (int)min((int64_t)bm, (int64_t)e_end - it.row0);
  it.n0 = it.nblk * bn;
  return it;
}

// The bf16-stack product (grouped_gemm_bf16.hip): LDS-DMA fed, multi-stage.
int launch_grouped_gemm_bf16(const GemmArgs& a, bool k_contiguous, hipStream_t s);
// the fused adapter gradient's workspace rows of 16 x K fp32 (one per tile), and its expert limit
int64_t grouped_gemm_db_slots(int64_t rows, int E);
int grouped_gemm_db_max_experts();
// whether the DMA-fed product's tile shape pairs gate and up columns for the fused SwiGLU (GemmArgs::act)
bool grouped_gemm_swiglu_fits();
// the DMA-fed product for a quantised stack read with k contiguous (decoded in registers)
bool grouped_gemm_dma_takes(const GemmArgs& a, int w_dtype, bool k_contiguous, bool scale_on_k);
int launch_grouped_gemm_dma_q(const GemmArgs& a, int w_dtype, bool scale_on_k, hipStream_t s);

}  // namespace mlora
