// The adapters' gradients: for every expert e,
//
//   out[e, n, r] = bf16(scaling · sum over expert e's rows of g[row, n] · l[row, r])
//
// a product whose depth is the expert's row count, bound by reading g once.  One workgroup per
// (expert, 64 columns of g); each of its four waves walks its own 32-row chunks of the expert
// (chunks wave, wave + 4, ...) on its own: the chunk's 32 x 64 slice of g and 32 x R slice of l are
// loaded into registers two chunks ahead of use, transposed into the wave's own LDS area as [n][row]
// and [r][row] (rows contiguous: the MFMA's k), and multiplied with v_mfma_f32_16x16x32_bf16 into
// fp32.  Gathered row indices and row-scale indices are staged in LDS for 1024 rows at a time, so a
// data load never waits behind an index load.  No barrier inside the chunk loop: a wave's LDS writes
// and reads are ordered among themselves.  At the end the four waves' partial sums are added in a
// fixed order (wave 0, 1, 2, 3): no atomics, the same bits every run.
//
// Rows of g may be gathered (row r read from g[gather[r] / gk]) and weighted by a per-row scale,
// applied to the narrow operand: row r of l taken as bf16(row_scale[scale_index[r]] · l[r]).
//
// With few experts (E <= 32), an expert's rows are cut into parts of at most P rows (P = part_rows(rows,
// E): at least 4096, and at least the mean rows per expert), one workgroup per (part, 64 columns), so that
// an expert holding a large share of the rows (Zipf routing) is spread over many workgroups instead of
// bounding the launch; with more experts each holds a small share and P covers every expert.  Part p of
// expert e is grid row e + floor(start_e / P) + p (an injective map, so no scan of the experts is needed;
// grid rows that map to no part exit at once).  A single-part expert's workgroup writes its result; a
// split expert's parts write fp32 partial sums to the workspace and reduce_finish_kernel, the next launch,
// adds them in part order: deterministic.
//
// Reference behaviour: src/meepsquared/_grouped.py:232-256 (_grouped_reduce_kernel), :362-370 (_reduce).
#include "common.hpp"

namespace mlora {

constexpr int RB_N = 64;      // columns of g per workgroup
constexpr int RB_CH = 32;     // rows per chunk, a wave's unit of work
constexpr int RB_WAVES = 4;   // waves per workgroup
constexpr int RB_IB = 1024;  // rows whose indices are staged in LDS at a time
constexpr int RB_P = RB_CH + 8;  // LDS pitch of the transposed tiles in bf16 (80 bytes: the MFMA
                                 // operand reads of 16 lanes cover the 64 banks once)
constexpr int RB_MIN_PART = 4096;  // rows per part at least
constexpr int RB_SPLIT_E = 32;     // experts up to which an expert's rows are split into parts

// rows per part: with up to RB_SPLIT_E experts a power of two, at least RB_MIN_PART and the mean rows per
// expert (balanced routing splits nothing; a skewed expert splits into a few parts); else all the rows
__host__ __device__ inline int64_t part_rows(int64_t rows, int E) {
  if (E > RB_SPLIT_E) return rows > 0 ? rows : 1;
  const int64_t mean = (rows + E - 1) / E;
  int64_t p = RB_MIN_PART;
  while (p < mean) p <<= 1;
  return p;
}
// grid rows: expert e's parts at e + floor(start_e / P) + p, all below E + rows / P + 1
__host__ __device__ inline int64_t part_slots(int64_t rows, int E) { return rows / part_rows(rows, E) + E + 1; }

__device__ __forceinline__ int64_t expert_start(const int32_t* offsets, int64_t rows, int e) {
  return e == 0 ? 0 : min(max((int64_t)offsets[e - 1], (int64_t)0), rows);
}

__device__ __forceinline__ uint32_t lo2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// one chunk in registers: rows 4 (lane / 8) + q, columns 8 (lane % 8) .. +7 of g; NRB pieces of l
// (piece lane + 64 q: row piece / (2 NRB), ranks 8 (piece % (2 NRB)) .. +7) with their row scales
template <int NRB>
struct RedChunk {
  u32x4 g[4];
  u32x4 l[NRB];
  uint32_t ws[NRB];  // the dword holding each piece's row scale
  uint32_t si[NRB];  // and that scale's index
};
// GATHER: rows of g read through gather; SCALED: l weighted by row_scale (compile-time, so that the
// chunk loop has no branch: a load in a branch is copied at the join, and the copy waits for it)
template <int NRB, bool GATHER, bool SCALED>
__global__ __launch_bounds__(256) void grouped_reduce_kernel(const bf16* __restrict__ g, int64_t ldg,
                                                             const int64_t* __restrict__ gather, int gk,
                                                             const void* __restrict__ row_scale, int rs_dt,
                                                             const int64_t* __restrict__ rs_idx,
                                                             const bf16* __restrict__ l, int64_t ldl, int64_t rows,
                                                             int N, float scaling, const int32_t* __restrict__ offsets,
                                                             int E, int64_t P, float* __restrict__ partial,
                                                             bf16* __restrict__ out, int64_t o_se, int64_t o_sn,
                                                             int64_t o_sr) {
  constexpr int R = NRB * 16;
  __shared__ __attribute__((aligned(16))) bf16 Gs[RB_WAVES][RB_N * RB_P];  // [n][row], one area per wave
  __shared__ __attribute__((aligned(16))) bf16 Ls[RB_WAVES][R * RB_P];     // [r][row]
  // a block of rows' indices, staged once for all waves: g's source rows and the row-scale indices
  // (read from LDS, an index never shares the vector-memory counter with the data loads)
  __shared__ uint32_t Is[GATHER ? RB_IB : 1];
  __shared__ uint32_t Ss[SCALED ? RB_IB : 1];
  static_assert(RB_WAVES * RB_N * RB_P * 2 >= RB_WAVES * RB_N * 16 * 4, "the partial sums fit in Gs");
  // Split experts, or gathered rows: consecutive workgroups take consecutive column blocks of one part,
  // so the rows they read at once are whole rows of the source, and parts run in expert order (a split
  // expert starts early).  Otherwise one part per expert and consecutive workgroups take consecutive
  // experts (grid x: the expert).
  const bool whole = P >= rows;  // every expert is one part: grid row = expert
  const bool by_expert = whole && !GATHER;
  const int slot = by_expert ? blockIdx.x : blockIdx.y;
  const int nbk = by_expert ? blockIdx.y : blockIdx.x;
  const int nblk = (N + RB_N - 1) / RB_N;
  const int n0 = nbk * RB_N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the chunk loop is a scalar loop
  auto base = [&](int x) { return (int64_t)x + expert_start(offsets, rows, x) / P; };
  int e;
  if (whole) {
    if (slot >= E) return;
    e = slot;
  } else {
    int lo = 0, hi = E - 1;  // the last expert whose first part's row is at or before this one
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (base(mid) <= slot) lo = mid; else hi = mid - 1;
    }
    e = __builtin_amdgcn_readfirstlane(lo);
  }
  const int64_t estart = expert_start(offsets, rows, e), eend = expert_start(offsets, rows, e + 1);
  const int np = eend > estart ? (int)((eend - estart + P - 1) / P) : 1;  // an empty expert: one part of zeros
  const int part = whole ? 0 : slot - (int)base(e);
  if (part >= np) return;  // a grid row between two experts' parts
  const int64_t start = min(eend, estart + (int64_t)part * P);
  const int64_t end = min(eend, start + P);

  const int gq = (lane >> 3) * 4, gc = (lane & 7) * 8;
  const bool g_cols = n0 + gc < N;
  const int gcc = g_cols ? n0 + gc : 0;  // a column that is always in g
  int lr[NRB], lc[NRB];
#pragma unroll
  for (int q = 0; q < NRB; ++q) {
    const int pc = lane + 64 * q;
    lr[q] = pc / (2 * NRB);
    lc[q] = (pc % (2 * NRB)) * 8;
  }

  f32x4 acc[4][NRB];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int j = 0; j < NRB; ++j) acc[cb][j] = f32x4{};
  bf16* gs = Gs[wave];
  bf16* ls = Ls[wave];

  for (int64_t b0 = start; b0 < end; b0 += RB_IB) {
    const int64_t b1 = min(end, b0 + (int64_t)RB_IB);
    const int nb = (int)(b1 - b0);
    if constexpr (GATHER || SCALED) {
      __syncthreads();  // every wave is done with the previous block's indices
      for (int i = tid; i < nb; i += 256) {
        if constexpr (GATHER) Is[i] = (uint32_t)gather[b0 + i] / (uint32_t)gk;
        if constexpr (SCALED) Ss[i] = (uint32_t)rs_idx[b0 + i];
      }
      __syncthreads();
    }
    const int chunks = (nb + RB_CH - 1) / RB_CH;
    const int nc = chunks > wave ? (chunks - wave + RB_WAVES - 1) / RB_WAVES : 0;  // this wave's chunks
    // Every load is unconditional: rows past the block's end read its last row (the values are dropped
    // in consume), so no load sits in a branch, where the compiler would wait for it on the spot.
    auto rel0 = [&](int c) { return (wave + RB_WAVES * c) * RB_CH; };  // the chunk's first row in the block
    auto clamp = [&](int r) { return r < nb ? r : nb - 1; };
    auto load = [&](RedChunk<NRB>& ch, int c) {
      const int r0 = rel0(c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = clamp(r0 + gq + q);
        const int64_t src = GATHER ? (int64_t)Is[r] : b0 + r;
        ch.g[q] = *(const u32x4*)(g + src * ldg + gcc);
      }
#pragma unroll
      for (int q = 0; q < NRB; ++q) {
        const int r = clamp(r0 + lr[q]);
        ch.l[q] = *(const u32x4*)(l + (b0 + r) * ldl + lc[q]);
        if constexpr (SCALED) {
          // the dword holding the row's scale (a bf16 scale is one half of it, picked in consume): one
          // load for either dtype
          ch.si[q] = Ss[r];
          ch.ws[q] = *(const uint32_t*)((const char*)row_scale +
                                        (((uint64_t)ch.si[q] << (rs_dt == MLORA_DT_F32 ? 2 : 1)) & ~(uint64_t)3));
        }
      }
    };
    auto consume = [&](RedChunk<NRB>& ch, int c) {
      const int r0 = rel0(c);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (!(r0 + gq + q < nb && g_cols)) ch.g[q] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int q = 0; q < NRB; ++q) {
        if (!(r0 + lr[q] < nb)) ch.l[q] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (SCALED) {
          const float w = rs_dt == MLORA_DT_F32 ? __uint_as_float(ch.ws[q])
                                                : bf16_bits_to_f32((ch.si[q] & 1u) ? ch.ws[q] >> 16 : ch.ws[q] & 0xFFFFu);
#pragma unroll
          for (int m = 0; m < 4; ++m)
            ch.l[q][m] = pack_bf16x2(bf16_bits_to_f32(ch.l[q][m] & 0xFFFFu) * w, bf16_bits_to_f32(ch.l[q][m] >> 16) * w);
        }
      }
      // 4 rows x 8 columns of g -> 8 columns x 4 rows (8 bytes per column)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        *(u32x2*)(gs + (gc + 2 * m) * RB_P + gq) = u32x2{lo2(ch.g[0][m], ch.g[1][m]), lo2(ch.g[2][m], ch.g[3][m])};
        *(u32x2*)(gs + (gc + 2 * m + 1) * RB_P + gq) = u32x2{hi2(ch.g[0][m], ch.g[1][m]), hi2(ch.g[2][m], ch.g[3][m])};
      }
#pragma unroll
      for (int q = 0; q < NRB; ++q)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          *(uint16_t*)(ls + (lc[q] + 2 * m) * RB_P + lr[q]) = (uint16_t)(ch.l[q][m] & 0xFFFFu);
          *(uint16_t*)(ls + (lc[q] + 2 * m + 1) * RB_P + lr[q]) = (uint16_t)(ch.l[q][m] >> 16);
        }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes have landed
      asm volatile("" ::: "memory");
      bf16x8 b[NRB];
#pragma unroll
      for (int j = 0; j < NRB; ++j) b[j] = *(const bf16x8*)(ls + (j * 16 + (lane & 15)) * RB_P + (lane >> 4) * 8);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const bf16x8 a = *(const bf16x8*)(gs + (cb * 16 + (lane & 15)) * RB_P + (lane >> 4) * 8);
#pragma unroll
        for (int j = 0; j < NRB; ++j) acc[cb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[j], acc[cb][j], 0, 0, 0);
      }
      asm volatile("" ::: "memory");
    };

    // loads run two chunks ahead of use.  Both halves of the loop body run every iteration (a chunk
    // past the wave's last holds only masked rows, which add zeros): a conditional half would make the
    // compiler copy the loaded registers at the loop's back edge, and a copy waits for its load.
    // sched_barrier keeps the phases in program order, so each wait leaves the later chunk in flight.
    RedChunk<NRB> ca, cb_;
    load(ca, 0);
    __builtin_amdgcn_sched_barrier(0);
    load(cb_, 1);
    __builtin_amdgcn_sched_barrier(0);
    for (int c = 0; c < nc; c += 2) {
      consume(ca, c);
      __builtin_amdgcn_sched_barrier(0);
      load(ca, c + 2);
      __builtin_amdgcn_sched_barrier(0);
      consume(cb_, c + 1);
      __builtin_amdgcn_sched_barrier(0);
      load(cb_, c + 3);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // the waves' partial sums, added in wave order; acc[cb][j][v] is column cb*16 + 4*(lane/16) + v,
  // rank j*16 + lane%16
  float* red = (float*)&Gs[0][0];
#pragma unroll
  for (int j = 0; j < NRB; ++j) {
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(wave * RB_N + cb * 16 + 4 * (lane >> 4) + v) * 16 + (lane & 15)] = acc[cb][j][v];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < RB_N * 16 / 256; ++u) {
      const int idx = tid + 256 * u, col = idx >> 4, r = idx & 15;
      float s = red[idx];
#pragma unroll
      for (int w = 1; w < RB_WAVES; ++w) s += red[w * RB_N * 16 + idx];
      const int n = n0 + col;
      if (np == 1) {
        if (n < N) out[(int64_t)e * o_se + (int64_t)n * o_sn + (int64_t)(j * 16 + r) * o_sr] = (bf16)(s * scaling);
      } else {  // a split expert: this part's sums, [grid row][column block][64][R]
        partial[(((int64_t)slot * nblk + nbk) * RB_N + col) * R + j * 16 + r] = s;
      }
    }
  }
}

// The parts of each split expert added in part order, scaled and rounded: one workgroup per (64 columns,
// expert); a single-part expert's result is written already.
__global__ __launch_bounds__(256) void reduce_finish_kernel(const float* __restrict__ partial,
                                                            const int32_t* __restrict__ offsets, int64_t rows, int E,
                                                            int64_t P, int N, int R, float scaling,
                                                            bf16* __restrict__ out, int64_t o_se, int64_t o_sn,
                                                            int64_t o_sr) {
  const int e = blockIdx.y, nb = blockIdx.x, nblk = gridDim.x;
  const int64_t estart = expert_start(offsets, rows, e), eend = expert_start(offsets, rows, e + 1);
  const int np = eend > estart ? (int)((eend - estart + P - 1) / P) : 1;
  if (np <= 1) return;
  const int64_t s0 = (int64_t)e + estart / P;
  for (int idx = threadIdx.x; idx < RB_N * R; idx += 256) {
    const int col = idx / R, r = idx - col * R, n = nb * RB_N + col;
    float sum = 0.f;
    for (int q = 0; q < np; ++q) sum += partial[((s0 + q) * nblk + nb) * RB_N * R + idx];
    if (n < N) out[(int64_t)e * o_se + (int64_t)n * o_sn + (int64_t)r * o_sr] = (bf16)(sum * scaling);
  }
}

// ---- SwiGLU's backward with the two adapter reductions that read its operands ----
//
// The layer's backward between its two products (src/meepsquared/_moe.py:118-126, SwiGLU as TF
// integrations/moe.py:509-520) in one pass over each expert's rows:
//   dgu  = SwiGLU'(gu) applied to dact = w_r · g[r]                  (the gate_up product's input gradient)
//   dwp  = per 64 columns of act, sum g[r] · act[r]                 (the combine weights' gradient, in parts)
//   dA   = s2 · sum_r act[r]^T ⊗ bf16(w_r · l2[r])                   (the down adapter's A gradient, rank 16)
//   dB   = su · sum_r dgu[r]^T ⊗ lu[r]                               (the gate_up adapter's B gradient, rank 16)
// act = bf16(silu(gate) · up) as the forward rounds it; w_r = w[perm[r]].  One workgroup per (part of an
// expert's rows, 64 columns of act), which reads the 64 gate and 64 up columns of gu and the 64 columns of
// g of its rows and writes the 128 columns of dgu: the reductions are fed from the registers the SwiGLU
// backward already holds, so neither act nor dgu is read back.  The reductions run as grouped_reduce_kernel
// does (the same chunk-to-wave assignment, MFMA order and wave-order sum), so dA and dB carry the same bits
// as grouped_reduce_gather(act, l2, row_scale = w) and grouped_reduce(dgu, lu) would.  Rows past
// offsets[E-1] (sentinels) are not visited: swiglu_reduce_rows_kernel zeroes their dgu and dw.
// Reference behaviour: src/meepsquared/_grouped.py:362-370 (_reduce) for dA and dB.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// the sum over each aligned group of eight lanes, the same bits in every lane of the group
__device__ __forceinline__ float sum8(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x141>(v);  // row_half_mirror: lane i and lane 7 - i of each eight
  return v;
}

template <typename TW>
__global__ __launch_bounds__(256) void swiglu_backward_reduce_kernel(
    const bf16* __restrict__ gu, const bf16* __restrict__ g, int64_t rows, int I, const TW* __restrict__ w,
    const int64_t* __restrict__ perm, const bf16* __restrict__ l2, int64_t ld2, float s2, const bf16* __restrict__ lu,
    int64_t ldu, float su, const int32_t* __restrict__ offsets, int E, int64_t P, bf16* __restrict__ dgu,
    float* __restrict__ dwp, float* __restrict__ partial, bf16* __restrict__ da, int64_t a_se, int64_t a_sn,
    int64_t a_sr, bf16* __restrict__ db, int64_t b_se, int64_t b_sn, int64_t b_sr) {
  __shared__ __attribute__((aligned(16))) bf16 Ts[RB_WAVES][RB_N * RB_P];  // [n][row]: act, then dgate, then dup
  __shared__ __attribute__((aligned(16))) bf16 L2s[RB_WAVES][16 * RB_P];   // [r][row]: bf16(w · l2)
  __shared__ __attribute__((aligned(16))) bf16 Lus[RB_WAVES][16 * RB_P];   // [r][row]: lu
  __shared__ float Ws[RB_IB];                                              // the block's row weights
  static_assert(RB_WAVES * RB_N * RB_P * 2 >= RB_WAVES * RB_N * 16 * 4, "the partial sums fit in Ts");
  const int nbk = blockIdx.x, slot = blockIdx.y;
  const int nblk = gridDim.x;
  const int n0 = nbk * RB_N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  auto base = [&](int x) { return (int64_t)x + expert_start(offsets, rows, x) / P; };
  int e;
  {
    int lo = 0, hi = E - 1;  // the last expert whose first part's grid row is at or before this one
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (base(mid) <= slot) lo = mid; else hi = mid - 1;
    }
    e = __builtin_amdgcn_readfirstlane(lo);
  }
  const int64_t estart = expert_start(offsets, rows, e), eend = expert_start(offsets, rows, e + 1);
  const int np = eend > estart ? (int)((eend - estart + P - 1) / P) : 1;  // an empty expert: one part of zeros
  const int part = slot - (int)base(e);
  if (part >= np) return;  // a grid row between two experts' parts
  const int64_t start = min(eend, estart + (int64_t)part * P);
  const int64_t end = min(eend, start + P);

  const int gq = (lane >> 3) * 4, gc = (lane & 7) * 8;
  const bool g_cols = n0 + gc < I;
  const int gcc = g_cols ? n0 + gc : 0;  // a column that is always in g
  const int lr = lane >> 1, lc = (lane & 1) * 8;  // this lane's piece of the l rows: row lr, ranks lc .. lc+7
  const int64_t I2 = 2 * (int64_t)I;

  f32x4 acc_a[4], acc_g[4], acc_u[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) acc_a[cb] = acc_g[cb] = acc_u[cb] = f32x4{};
  bf16* ts = Ts[wave];
  bf16* l2s = L2s[wave];
  bf16* lus = Lus[wave];

  struct Chunk {
    u32x4 gt[4], up[4], gr[4];  // rows gq + q, columns gc .. gc+7: gate, up, g
    u32x4 a, b;                 // row lr, ranks lc .. lc+7: l2, lu
  };

  for (int64_t b0 = start; b0 < end; b0 += RB_IB) {
    const int64_t b1 = min(end, b0 + (int64_t)RB_IB);
    const int nb = (int)(b1 - b0);
    __syncthreads();  // every wave is done with the previous block's weights
    for (int i = tid; i < nb; i += 256) Ws[i] = load_w(w, perm[b0 + i]);
    __syncthreads();
    const int chunks = (nb + RB_CH - 1) / RB_CH;
    const int nc = chunks > wave ? (chunks - wave + RB_WAVES - 1) / RB_WAVES : 0;
    auto rel0 = [&](int c) { return (wave + RB_WAVES * c) * RB_CH; };
    auto clamp = [&](int r) { return r < nb ? r : nb - 1; };
    auto load = [&](Chunk& ch, int c) {  // unconditional: rows past the block's end read its last row
      const int r0 = rel0(c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r = b0 + clamp(r0 + gq + q);
        ch.gt[q] = *(const u32x4*)(gu + r * I2 + gcc);
        ch.up[q] = *(const u32x4*)(gu + r * I2 + I + gcc);
        ch.gr[q] = *(const u32x4*)(g + r * I + gcc);
      }
      const int64_t r = b0 + clamp(r0 + lr);
      ch.a = *(const u32x4*)(l2 + r * ld2 + lc);
      ch.b = *(const u32x4*)(lu + r * ldu + lc);
    };
    auto consume = [&](Chunk& ch, int c, auto&& next) {
      const int r0 = rel0(c);
      u32x4 act[4], dgv[4], duv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = r0 + gq + q;
        const bool live = rr < nb && g_cols;
        float gg[8], u[8], d[8], dg[8], du[8], av[8];
        unpack8(ch.gt[q], gg);
        unpack8(ch.up[q], u);
        unpack8(ch.gr[q], d);
        float dot = swiglu_grad8(gg, u, d, Ws[clamp(rr)], live, dg, du, av);
        act[q] = live ? pack8(av) : u32x4{0u, 0u, 0u, 0u};
        dgv[q] = pack8(dg);
        duv[q] = pack8(du);
        if (live) {
          const int64_t r = b0 + rr;
          *(u32x4*)(dgu + r * I2 + n0 + gc) = dgv[q];
          *(u32x4*)(dgu + r * I2 + I + n0 + gc) = duv[q];
        }
        // the row's 64 columns: the eight lanes that hold it, summed in a fixed order
        dot = sum8(live ? dot : 0.f);
        if ((lane & 7) == 0 && rr < nb) dwp[nbk * rows + b0 + rr] = dot;  // [strip][row]: a chunk's 32 rows contiguous
      }
      const bool lrow = r0 + lr < nb;
      u32x4 la = ch.a, lb = ch.b;
      {
        const float wt = Ws[clamp(r0 + lr)];
#pragma unroll
        for (int m = 0; m < 4; ++m)
          la[m] = pack_bf16x2(bf16_bits_to_f32(la[m] & 0xFFFFu) * wt, bf16_bits_to_f32(la[m] >> 16) * wt);
      }
      if (!lrow) la = lb = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        *(uint16_t*)(l2s + (lc + 2 * m) * RB_P + lr) = (uint16_t)(la[m] & 0xFFFFu);
        *(uint16_t*)(l2s + (lc + 2 * m + 1) * RB_P + lr) = (uint16_t)(la[m] >> 16);
        *(uint16_t*)(lus + (lc + 2 * m) * RB_P + lr) = (uint16_t)(lb[m] & 0xFFFFu);
        *(uint16_t*)(lus + (lc + 2 * m + 1) * RB_P + lr) = (uint16_t)(lb[m] >> 16);
      }
      // one operand tile at a time through the wave's [n][row] area (a wave's LDS accesses run in order,
      // so each tile's writes follow the previous tile's reads)
      auto product = [&](const u32x4 (&v)[4], const bf16* ls, f32x4 (&acc)[4]) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          *(u32x2*)(ts + (gc + 2 * m) * RB_P + gq) = u32x2{lo2(v[0][m], v[1][m]), lo2(v[2][m], v[3][m])};
          *(u32x2*)(ts + (gc + 2 * m + 1) * RB_P + gq) = u32x2{hi2(v[0][m], v[1][m]), hi2(v[2][m], v[3][m])};
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's writes have landed
        asm volatile("" ::: "memory");
        const bf16x8 b = *(const bf16x8*)(ls + (lane & 15) * RB_P + (lane >> 4) * 8);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          const bf16x8 a = *(const bf16x8*)(ts + (cb * 16 + (lane & 15)) * RB_P + (lane >> 4) * 8);
          acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[cb], 0, 0, 0);
        }
        asm volatile("" ::: "memory");
      };
      next();  // the next chunk's loads, into the registers this chunk no longer needs
      product(act, l2s, acc_a);
      product(dgv, lus, acc_g);
      product(duv, lus, acc_u);
    };

    // one chunk in registers: the next chunk's loads go out once this one's SwiGLU math is done, and run
    // under its transposes and reduction MFMAs (139 VGPRs, so three waves per SIMD; two chunks in flight
    // held 203 and ran 7-10 % slower)
    Chunk ca;
    load(ca, 0);
    for (int c = 0; c < nc; ++c) consume(ca, c, [&]() { load(ca, c + 1); });
  }

  // the waves' partial sums, added in wave order; acc[cb][v] is column cb*16 + 4*(lane/16) + v, rank lane%16
  float* red = (float*)&Ts[0][0];
#pragma unroll
  for (int which = 0; which < 3; ++which) {
    const f32x4(&acc)[4] = which == 0 ? acc_a : which == 1 ? acc_g : acc_u;
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(wave * RB_N + cb * 16 + 4 * (lane >> 4) + v) * 16 + (lane & 15)] = acc[cb][v];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < RB_N * 16 / 256; ++u) {
      const int idx = tid + 256 * u, col = idx >> 4, r = idx & 15;
      float sum = red[idx];
#pragma unroll
      for (int wv = 1; wv < RB_WAVES; ++wv) sum += red[wv * RB_N * 16 + idx];
      const int n = n0 + col;
      if (np == 1) {
        if (n < I) {
          if (which == 0) da[(int64_t)e * a_se + (int64_t)n * a_sn + (int64_t)r * a_sr] = (bf16)(sum * s2);
          else db[(int64_t)e * b_se + (int64_t)(n + (which == 2 ? I : 0)) * b_sn + (int64_t)r * b_sr] = (bf16)(sum * su);
        }
      } else {  // a split expert: this part's sums, [grid row][column block][which][64][16]
        partial[(((int64_t)slot * nblk + nbk) * 3 + which) * RB_N * 16 + idx] = sum;
      }
    }
  }
}

// The combine weights' gradient: dw[perm[r]] = the row's per-64-column parts added in column order; rows
// past offsets[E-1] (sentinels) get zero there and in dgu.
template <typename TW>
__global__ __launch_bounds__(256) void swiglu_reduce_rows_kernel(const float* __restrict__ dwp, int nblk, int64_t rows,
                                                                 int64_t I2, const int64_t* __restrict__ perm,
                                                                 const int32_t* __restrict__ offsets, int E,
                                                                 bf16* __restrict__ dgu, TW* __restrict__ dw) {
  const int64_t valid = expert_start(offsets, rows, E);
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    if (r < valid) {  // four parts' loads in flight at a time (the strips lie rows apart), added in order
      int c = 0;
      for (; c + 4 <= nblk; c += 4) {
        const float v0 = dwp[c * rows + r], v1 = dwp[(c + 1) * rows + r], v2 = dwp[(c + 2) * rows + r],
                    v3 = dwp[(c + 3) * rows + r];
        s += v0;
        s += v1;
        s += v2;
        s += v3;
      }
      for (; c < nblk; ++c) s += dwp[c * rows + r];
    } else {
      for (int64_t c = 0; c < I2; c += 8) *(u32x4*)(dgu + r * I2 + c) = u32x4{0u, 0u, 0u, 0u};
    }
    dw[perm[r]] = (TW)s;
  }
}

// The parts of each split expert added in part order for dA and both halves of dB, scaled and rounded.
__global__ __launch_bounds__(256) void swiglu_reduce_finish_kernel(const float* __restrict__ partial,
                                                                   const int32_t* __restrict__ offsets, int64_t rows,
                                                                   int E, int64_t P, int I, float s2, float su,
                                                                   bf16* __restrict__ da, int64_t a_se, int64_t a_sn,
                                                                   int64_t a_sr, bf16* __restrict__ db, int64_t b_se,
                                                                   int64_t b_sn, int64_t b_sr) {
  const int e = blockIdx.y, nb = blockIdx.x, nblk = gridDim.x;
  const int64_t estart = expert_start(offsets, rows, e), eend = expert_start(offsets, rows, e + 1);
  const int np = eend > estart ? (int)((eend - estart + P - 1) / P) : 1;
  if (np <= 1) return;
  const int64_t s0 = (int64_t)e + estart / P;
  for (int idx = threadIdx.x; idx < 3 * RB_N * 16; idx += 256) {
    const int which = idx / (RB_N * 16), rem = idx - which * RB_N * 16, col = rem >> 4, r = rem & 15;
    const int n = nb * RB_N + col;
    float sum = 0.f;
    for (int q = 0; q < np; ++q) sum += partial[((s0 + q) * nblk + nb) * 3 * RB_N * 16 + idx];
    if (n >= I) continue;
    if (which == 0) da[(int64_t)e * a_se + (int64_t)n * a_sn + (int64_t)r * a_sr] = (bf16)(sum * s2);
    else db[(int64_t)e * b_se + (int64_t)(n + (which == 2 ? I : 0)) * b_sn + (int64_t)r * b_sr] = (bf16)(sum * su);
  }
}

}  // namespace mlora

using namespace mlora;

extern "C" size_t mlora_grouped_reduce_workspace_bytes(int64_t rows, int N, int R, int E) {
  if (rows < 0 || E < 1 || N < 1 || R < 1 || rows <= part_rows(rows, E)) return 0;  // no expert can be split
  const int64_t nblk = (N + RB_N - 1) / RB_N;
  return (size_t)part_slots(rows, E) * (size_t)nblk * RB_N * (size_t)R * sizeof(float);
}

static int grouped_reduce_impl(const void* g, int64_t ldg, const int64_t* gather, int gk, const void* row_scale,
                               int rs_dt, const int64_t* rs_idx, const void* l, int64_t ldl, int64_t rows, int N, int R,
                               float scaling, const int32_t* offsets, int E, void* out, int64_t o_se, int64_t o_sn,
                               int64_t o_sr, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (gather != nullptr && gk < 1) return fail("grouped_reduce_gather: k=%d must be >= 1", gk);
  if (row_scale != nullptr && (rs_idx == nullptr || (rs_dt != MLORA_DT_BF16 && rs_dt != MLORA_DT_F32)))
    return fail("grouped_reduce_gather: a row scale needs its index and a bf16/f32 dtype (got %d)", rs_dt);
  if (E < 1 || E > 65535) return fail("grouped_reduce: E=%d outside [1, 65535]", E);
  if (rows < 0 || rows > (int64_t)0xFFFFFFFFu) return fail("grouped_reduce: rows=%lld outside [0, 2^32)", (long long)rows);
  if (N < 8 || N % 8 || ldg < N || ldg % 8 || ((uintptr_t)g & 15u))
    return fail("grouped_reduce: g needs N (%d) and its row stride (%lld) multiples of 8, 16-byte aligned", N, (long long)ldg);
  if (R < 16 || R > 64 || R % 16) return fail("grouped_reduce: R=%d must be 16, 32, 48 or 64", R);
  if (ldl < R || ldl % 8 || ((uintptr_t)l & 15u)) return fail("grouped_reduce: l needs 16-byte aligned rows of >= R values");
  const size_t need = mlora_grouped_reduce_workspace_bytes(rows, N, R, E);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 15u)))
    return fail("grouped_reduce: workspace of %zu bytes, %zu needed (16-byte aligned)", workspace_bytes, need);
  const unsigned nblk = (unsigned)((N + RB_N - 1) / RB_N);
  const int64_t P = part_rows(rows, E), slots = part_slots(rows, E);
  if (slots > 65535) return fail("grouped_reduce: %lld grid rows past the grid's 65535", (long long)slots);
  // one part per expert and rows not gathered: the expert is grid x (consecutive workgroups, consecutive experts)
  const bool by_expert = P >= rows && gather == nullptr;
  const dim3 grid(by_expert ? (unsigned)slots : nblk, by_expert ? nblk : (unsigned)slots), block(256);
  hipStream_t s = as_stream(stream);
#define MLORA_RED(NRB, GA, SC)                                                                                       \
  hipLaunchKernelGGL((grouped_reduce_kernel<NRB, GA, SC>), grid, block, 0, s, (const bf16*)g, ldg, gather, gk, row_scale, \
                     rs_dt, rs_idx, (const bf16*)l, ldl, rows, N, scaling, offsets, E, P, (float*)workspace,         \
                     (bf16*)out, o_se, o_sn, o_sr)
#define MLORA_RED_R(GA, SC)            \
  switch (R / 16) {                    \
    case 1: MLORA_RED(1, GA, SC); break; \
    case 2: MLORA_RED(2, GA, SC); break; \
    case 3: MLORA_RED(3, GA, SC); break; \
    default: MLORA_RED(4, GA, SC); break; \
  }
  if (gather != nullptr && row_scale != nullptr) MLORA_RED_R(true, true)
  else if (gather != nullptr) MLORA_RED_R(true, false)
  else if (row_scale != nullptr) MLORA_RED_R(false, true)
  else MLORA_RED_R(false, false)
#undef MLORA_RED_R
#undef MLORA_RED
  if (int rc = launch_status("grouped_reduce")) return rc;
  if (need > 0) {  // some expert may have been split
    hipLaunchKernelGGL(reduce_finish_kernel, dim3(nblk, (unsigned)E), dim3(256), 0, s, (const float*)workspace, offsets,
                       rows, E, P, N, R, scaling, (bf16*)out, o_se, o_sn, o_sr);
    return launch_status("grouped_reduce/finish");
  }
  return 0;
}

extern "C" int mlora_grouped_reduce(const void* g, int64_t ldg, const void* l, int64_t ldl, int64_t rows, int N, int R,
                                    float scaling, const int32_t* offsets, int E, void* out, int64_t o_se,
                                    int64_t o_sn, int64_t o_sr, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  return grouped_reduce_impl(g, ldg, nullptr, 1, nullptr, 0, nullptr, l, ldl, rows, N, R, scaling, offsets, E, out,
                             o_se, o_sn, o_sr, workspace, workspace_bytes, stream);
}

extern "C" int mlora_grouped_reduce_gather(const void* g, int64_t ldg, const int64_t* gather, int k,
                                           const void* row_scale, int row_scale_dtype, const int64_t* scale_index,
                                           const void* l, int64_t ldl, int64_t rows, int N, int R, float scaling,
                                           const int32_t* offsets, int E, void* out, int64_t o_se, int64_t o_sn,
                                           int64_t o_sr, void* workspace, size_t workspace_bytes, void* stream) {
  if (gather == nullptr && row_scale == nullptr) {
    clear_error();
    return fail("grouped_reduce_gather: neither gather nor a row scale");
  }
  return grouped_reduce_impl(g, ldg, gather, k, row_scale, row_scale_dtype, scale_index, l, ldl, rows, N, R, scaling,
                             offsets, E, out, o_se, o_sn, o_sr, workspace, workspace_bytes, stream);
}

// dw parts [I / 64][rows] fp32 (256-byte aligned), then, when an expert can be split, the parts' sums
static size_t swiglu_reduce_dw_bytes(int64_t S, int64_t I) {
  const int64_t nblk = (I + RB_N - 1) / RB_N;
  return (size_t)((S * nblk * (int64_t)sizeof(float) + 255) & ~(int64_t)255);
}

extern "C" size_t mlora_swiglu_backward_reduce_workspace_bytes(int64_t S, int64_t I, int E) {
  if (S < 0 || I < 8 || E < 1) return 0;
  const int64_t nblk = (I + RB_N - 1) / RB_N;
  const size_t split = S > part_rows(S, E) ? (size_t)part_slots(S, E) * nblk * 3 * RB_N * 16 * sizeof(float) : 0;
  return swiglu_reduce_dw_bytes(S, I) + split;
}

extern "C" int mlora_swiglu_backward_reduce(const void* gu, const void* g, int64_t S, int64_t I, const void* w,
                                            int w_dtype, const int64_t* perm, const int32_t* offsets, int E,
                                            const void* low2, int64_t ld2, float scaling2, void* dA, int64_t a_se,
                                            int64_t a_sn, int64_t a_sr, const void* lowgu, int64_t ldu,
                                            float scaling_gu, void* dB, int64_t b_se, int64_t b_sn, int64_t b_sr,
                                            void* dgu, void* dw, void* workspace, size_t workspace_bytes,
                                            void* stream) {
  clear_error();
  if (S < 1 || S > (int64_t)0xFFFFFFFFu) return fail("swiglu_backward_reduce: S=%lld outside [1, 2^32)", (long long)S);
  if (I < 8 || I % 8 || I > (1 << 24)) return fail("swiglu_backward_reduce: I=%lld must be a multiple of 8", (long long)I);
  if (E < 1 || E > 65535) return fail("swiglu_backward_reduce: E=%d outside [1, 65535]", E);
  if (w_dtype != MLORA_DT_BF16 && w_dtype != MLORA_DT_F32)
    return fail("swiglu_backward_reduce: weight dtype %d is not bf16/f32", w_dtype);
  if (((uintptr_t)gu | (uintptr_t)g | (uintptr_t)dgu | (uintptr_t)low2 | (uintptr_t)lowgu) & 15u)
    return fail("swiglu_backward_reduce: gu, g, dgu and the low tensors must be 16-byte aligned");
  if (ld2 < 16 || ld2 % 8 || ldu < 16 || ldu % 8)
    return fail("swiglu_backward_reduce: the low tensors need rows of >= 16 values, strides multiples of 8");
  const size_t need = mlora_swiglu_backward_reduce_workspace_bytes(S, I, E);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail("swiglu_backward_reduce: workspace of %zu bytes, %zu needed (256-byte aligned)", workspace_bytes, need);
  const unsigned nblk = (unsigned)((I + RB_N - 1) / RB_N);
  const int64_t P = part_rows(S, E), slots = part_slots(S, E);
  if (slots > 65535) return fail("swiglu_backward_reduce: %lld grid rows past the grid's 65535", (long long)slots);
  float* dwp = (float*)workspace;
  float* partial = (float*)((char*)workspace + swiglu_reduce_dw_bytes(S, I));
  hipStream_t s = as_stream(stream);
  const dim3 grid(nblk, (unsigned)slots), block(256);
  const unsigned rgrid = (unsigned)((S + 255) / 256 < 4096 ? (S + 255) / 256 : 4096);
#define MLORA_SWR(TW)                                                                                               \
  hipLaunchKernelGGL(swiglu_backward_reduce_kernel<TW>, grid, block, 0, s, (const bf16*)gu, (const bf16*)g, S, (int)I, \
                     (const TW*)w, perm, (const bf16*)low2, ld2, scaling2, (const bf16*)lowgu, ldu, scaling_gu,      \
                     offsets, E, P, (bf16*)dgu, dwp, partial, (bf16*)dA, a_se, a_sn, a_sr, (bf16*)dB, b_se, b_sn,  \
                     b_sr);                                                                                          \
  if (int rc = launch_status("swiglu_backward_reduce")) return rc;                                                  \
  hipLaunchKernelGGL(swiglu_reduce_rows_kernel<TW>, dim3(rgrid), block, 0, s, (const float*)dwp, (int)nblk, S,       \
                     2 * I, perm, offsets, E, (bf16*)dgu, (TW*)dw)
  if (w_dtype == MLORA_DT_F32) {
    MLORA_SWR(float);
  } else {
    MLORA_SWR(bf16);
  }
#undef MLORA_SWR
  if (int rc = launch_status("swiglu_backward_reduce/rows")) return rc;
  if (S > P) {  // some expert may have been split
    hipLaunchKernelGGL(swiglu_reduce_finish_kernel, dim3(nblk, (unsigned)E), block, 0, s, (const float*)partial,
                       offsets, S, E, P, (int)I, scaling2, scaling_gu, (bf16*)dA, a_se, a_sn, a_sr, (bf16*)dB, b_se,
                       b_sn, b_sr);
    return launch_status("swiglu_backward_reduce/finish");
  }
  return 0;
}
