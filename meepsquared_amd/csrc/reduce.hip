// The adapters' gradients: for every expert e,
//
//   out[e, n, r] = bf16(scaling · sum over expert e's rows of g[row, n] · l[row, r])
//
// a product whose depth is the expert's row count.  One workgroup per (expert, 64 columns of g)
// walks the expert's rows 64 at a time: a 64-row slice of g is transposed into LDS as [n][row]
// (k = rows contiguous, the MFMA's layout) and the matching slice of l as [r][row]; each wave
// accumulates a 16 x R block with v_mfma_f32_16x16x32_bf16 in fp32.  The next slice is loaded into
// registers while the current one is multiplied.  Every output element has exactly one writer
// and a fixed summation order: no atomics, the same bits every run.
//
// Rows of g may be gathered (row r read from g[gather[r] / gk]) and weighted by a per-row scale,
// applied to the narrow operand: row r of l taken as bf16(row_scale[scale_index[r]] · l[r]).
//
// Reference behaviour: src/meepsquared/_grouped.py:232-256 (_grouped_reduce_kernel), :362-370 (_reduce).
#include "common.hpp"

namespace mlora {

constexpr int RB_N = 64;  // columns of g per workgroup
constexpr int RPT = 2;                 // rows of g each thread loads per slice
constexpr int RB_ROWS = 32 * RPT;      // rows per slice
constexpr int RP_ = RB_ROWS + 8;

__device__ __forceinline__ uint32_t lo2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int NRB>
__global__ __launch_bounds__(256) void grouped_reduce_kernel(const bf16* __restrict__ g, int64_t ldg,
                                                             const int64_t* __restrict__ gather, int gk,
                                                             const void* __restrict__ row_scale, int rs_dt,
                                                             const int64_t* __restrict__ rs_idx,
                                                             const bf16* __restrict__ l, int64_t ldl, int64_t rows,
                                                             int N, float scaling, const int32_t* __restrict__ offsets,
                                                             bf16* __restrict__ out, int64_t o_se, int64_t o_sn,
                                                             int64_t o_sr) {
  constexpr int R = NRB * 16;
  __shared__ __attribute__((aligned(16))) bf16 Gs[RB_N * RP_];  // [n][row]
  __shared__ __attribute__((aligned(16))) bf16 Ls[R * RP_];     // [r][row]
  // gathered rows: consecutive workgroups take consecutive column blocks of one expert, so the rows
  // they read at once are whole rows of the source (4 % faster at config 1); the expert's own rows:
  // consecutive workgroups take consecutive experts (5 % faster)
  const int e = gather != nullptr ? blockIdx.y : blockIdx.x;
  const int n0 = (gather != nullptr ? blockIdx.x : blockIdx.y) * RB_N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the expert's rows, clamped into [0, rows]
  const int64_t start = e == 0 ? 0 : min(max((int64_t)offsets[e - 1], (int64_t)0), rows);
  const int64_t end = min(max((int64_t)offsets[e], (int64_t)0), rows);

  // this thread's RPT rows x 8 columns of g; the 4R threads that copy l (RPT rows x 8 ranks each)
  // are spread over the waves where 256 divides evenly
  constexpr int LSTRIDE = 256 % (4 * R) == 0 ? 256 / (4 * R) : 1;
  const int gr = (tid >> 3) * RPT, gc = (tid & 7) * 8;
  const int lo = tid / LSTRIDE;
  const int lr = (lo / (R / 8)) * RPT, lc = (lo % (R / 8)) * 8;
  const bool l_owner = tid % LSTRIDE == 0 && lo < 4 * R;
  const bool g_cols = n0 + gc < N;

  u32x4 gv[RPT], lv[RPT];
  float ws[RPT];
  // the rows a slice reads, fetched one slice ahead so that no load waits on an index load: g's
  // source row of each of this thread's RPT rows, and the row-scale index of each of its l rows
  int64_t gsrc[RPT], sidx[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) ws[q] = 1.f;
  auto fetch_rows = [&](int64_t row0) {
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int64_t row = row0 + gr + q;
      gsrc[q] = gather == nullptr || row >= end ? row : (int64_t)((uint32_t)gather[row] / (uint32_t)gk);
      const int64_t lrow = row0 + lr + q;
      sidx[q] = row_scale != nullptr && l_owner && lrow < end ? rs_idx[lrow] : 0;
    }
  };
  auto load = [&](int64_t row0) {
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int64_t row = row0 + gr + q;
      gv[q] = (row < end && g_cols) ? *(const u32x4*)(g + gsrc[q] * ldg + n0 + gc) : u32x4{0u, 0u, 0u, 0u};
      const int64_t lrow = row0 + lr + q;
      if (l_owner) {
        lv[q] = lrow < end ? *(const u32x4*)(l + lrow * ldl + lc) : u32x4{0u, 0u, 0u, 0u};
        if (row_scale != nullptr && lrow < end)
          ws[q] = rs_dt == MLORA_DT_F32 ? ((const float*)row_scale)[sidx[q]] : (float)((const bf16*)row_scale)[sidx[q]];
      }
    }
    fetch_rows(row0 + RB_ROWS);
  };
  auto store = [&]() {
    if (row_scale != nullptr && l_owner) {  // l's rows weighted here, after the loads have had the MFMAs to land
#pragma unroll
      for (int q = 0; q < RPT; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m)
          lv[q][m] = pack_bf16x2(bf16_bits_to_f32(lv[q][m] & 0xFFFFu) * ws[q], bf16_bits_to_f32(lv[q][m] >> 16) * ws[q]);
    }
    // transpose RPT rows x 8 columns into 8 columns x RPT rows, two rows per 32-bit store
#pragma unroll
    for (int pr = 0; pr < RPT; pr += 2)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        *(uint32_t*)(Gs + (gc + 2 * m) * RP_ + gr + pr) = lo2(gv[pr][m], gv[pr + 1][m]);
        *(uint32_t*)(Gs + (gc + 2 * m + 1) * RP_ + gr + pr) = hi2(gv[pr][m], gv[pr + 1][m]);
        if (l_owner) {
          *(uint32_t*)(Ls + (lc + 2 * m) * RP_ + lr + pr) = lo2(lv[pr][m], lv[pr + 1][m]);
          *(uint32_t*)(Ls + (lc + 2 * m + 1) * RP_ + lr + pr) = hi2(lv[pr][m], lv[pr + 1][m]);
        }
      }
  };

  f32x4 acc[NRB];
#pragma unroll
  for (int j = 0; j < NRB; ++j) acc[j] = f32x4{};
  if (start < end) {
    fetch_rows(start);
    load(start);
  }
  for (int64_t row0 = start; row0 < end; row0 += RB_ROWS) {
    store();
    __syncthreads();
    if (row0 + RB_ROWS < end) load(row0 + RB_ROWS);
#pragma unroll
    for (int kk = 0; kk < RB_ROWS / 32; ++kk) {
      const bf16x8 a = *(const bf16x8*)(Gs + (wave * 16 + (lane & 15)) * RP_ + kk * 32 + (lane >> 4) * 8);
#pragma unroll
      for (int j = 0; j < NRB; ++j) {
        const bf16x8 b = *(const bf16x8*)(Ls + (j * 16 + (lane & 15)) * RP_ + kk * 32 + (lane >> 4) * 8);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // acc[j][v]: n = n0 + wave*16 + 4*(lane/16) + v, r = j*16 + lane%16
#pragma unroll
  for (int j = 0; j < NRB; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int n = n0 + wave * 16 + 4 * (lane >> 4) + v;
      const int r = j * 16 + (lane & 15);
      if (n < N) out[(int64_t)e * o_se + (int64_t)n * o_sn + (int64_t)r * o_sr] = (bf16)(acc[j][v] * scaling);
    }
}

}  // namespace mlora

using namespace mlora;

static int grouped_reduce_impl(const void* g, int64_t ldg, const int64_t* gather, int gk, const void* row_scale,
                               int rs_dt, const int64_t* rs_idx, const void* l, int64_t ldl, int64_t rows, int N, int R,
                               float scaling, const int32_t* offsets, int E, void* out, int64_t o_se, int64_t o_sn,
                               int64_t o_sr, void* stream) {
  clear_error();
  if (gather != nullptr && gk < 1) return fail("grouped_reduce_gather: k=%d must be >= 1", gk);
  if (row_scale != nullptr && (rs_idx == nullptr || (rs_dt != MLORA_DT_BF16 && rs_dt != MLORA_DT_F32)))
    return fail("grouped_reduce_gather: a row scale needs its index and a bf16/f32 dtype (got %d)", rs_dt);
  if (E < 1 || E > 65535) return fail("grouped_reduce: E=%d outside [1, 65535]", E);
  if (N < 8 || N % 8 || ldg < N || ldg % 8 || ((uintptr_t)g & 15u))
    return fail("grouped_reduce: g needs N (%d) and its row stride (%lld) multiples of 8, 16-byte aligned", N, (long long)ldg);
  if (R < 16 || R > 64 || R % 16) return fail("grouped_reduce: R=%d must be 16, 32, 48 or 64", R);
  if (ldl < R || ldl % 8 || ((uintptr_t)l & 15u)) return fail("grouped_reduce: l needs 16-byte aligned rows of >= R values");
  const unsigned nblk = (unsigned)((N + RB_N - 1) / RB_N);
  const dim3 grid(gather != nullptr ? nblk : (unsigned)E, gather != nullptr ? (unsigned)E : nblk), block(256);
  hipStream_t s = as_stream(stream);
#define MLORA_RED(NRB)                                                                                               \
  hipLaunchKernelGGL(grouped_reduce_kernel<NRB>, grid, block, 0, s, (const bf16*)g, ldg, gather, gk, row_scale, rs_dt,   \
                     rs_idx, (const bf16*)l, ldl, rows, N, scaling, offsets, (bf16*)out, o_se, o_sn, o_sr)
  switch (R / 16) {
    case 1: MLORA_RED(1); break;
    case 2: MLORA_RED(2); break;
    case 3: MLORA_RED(3); break;
    default: MLORA_RED(4); break;
  }
#undef MLORA_RED
  return launch_status("grouped_reduce");
}

extern "C" int mlora_grouped_reduce(const void* g, int64_t ldg, const void* l, int64_t ldl, int64_t rows, int N, int R,
                                    float scaling, const int32_t* offsets, int E, void* out, int64_t o_se,
                                    int64_t o_sn, int64_t o_sr, void* stream) {
  return grouped_reduce_impl(g, ldg, nullptr, 1, nullptr, 0, nullptr, l, ldl, rows, N, R, scaling, offsets, E, out,
                             o_se, o_sn, o_sr, stream);
}

extern "C" int mlora_grouped_reduce_gather(const void* g, int64_t ldg, const int64_t* gather, int k,
                                           const void* row_scale, int row_scale_dtype, const int64_t* scale_index,
                                           const void* l, int64_t ldl, int64_t rows, int N, int R, float scaling,
                                           const int32_t* offsets, int E, void* out, int64_t o_se, int64_t o_sn,
                                           int64_t o_sr, void* stream) {
  if (gather == nullptr && row_scale == nullptr) {
    clear_error();
    return fail("grouped_reduce_gather: neither gather nor a row scale");
  }
  return grouped_reduce_impl(g, ldg, gather, k, row_scale, row_scale_dtype, scale_index, l, ldl, rows, N, R, scaling,
                             offsets, E, out, o_se, o_sn, o_sr, stream);
}
