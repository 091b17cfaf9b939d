// fp8 products: the grouped product of an fp8 e4m3 stack with activations quantised to e4m3, on
// gfx950's block-scaled fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
//
// Two kernels, one pass each:
//   * fp8_prep: for every row and every 64 columns of x, a power-of-two scale 2^e with
//     amax·2^-e <= 448 (stored as its E8M0 byte, 127 + e) and the 64 values e4m3(x·2^-e) (round to
//     nearest even); in the same pass over x, the LoRA product low = bf16(x · A_e) in fp32 on the
//     bf16 values (the adapters never see the quantised x).  Rows are cut into 64-row tiles that
//     never straddle two experts, so each tile multiplies one A_e on the MFMA.
//   * fp8_gemm: the bf16 kernel's decomposition (persistent grid, XCD ranges, 256 x 256 tiles,
//     8 waves, a 4-slot LDS ring fed by DMA) with 64-deep fp8 stages: per stage the x8 tile, the
//     W8 tile and the 256 rows' scale words reach LDS by buffer_load ... lds; each 32 x 32 x 64
//     MFMA takes the x rows' scale bytes as its B-operand scales (the same for both 32-deep halves
//     of the stage), so the accumulator holds the product of the unquantised-scale values directly.
//     The epilogue applies the stack's own scale (per expert or per output row), adds
//     scaling · low · B_e and the bias, and rounds once to bf16.
// The reference quantises x per row and per BLOCK_K tile with scale amax/448 inside its Triton
// kernel (src/meepsquared/_grouped.py:191-194, X_FP8); here the tile is 64 columns and the scale is
// amax/448 rounded up to a power of two, the form the MFMA applies in hardware.
//
// Reference behaviour: src/meepsquared/_grouped.py:70-80 (fp8_products), :120-221 (_grouped_gemm_kernel
// with X_FP8), :313-345 (_launch).
#include <mutex>
#include <unordered_map>

#include "gemm_common.hpp"

namespace mlora {
namespace f8 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

// ------------------------------------------------------------------------------------------------
// prep
// ------------------------------------------------------------------------------------------------
constexpr int PR = 64;   // rows per prep tile, columns per scale block
constexpr int PT = 256;  // threads per prep workgroup
constexpr int XP = 72;   // LDS row pitch (elements) of the x and A^T chunks

struct PrepArgs {
  const bf16* x;
  int64_t ldx, rows;
  int K;
  const float* colscale;  // NULL, or per-column multipliers of the quantised values: colscale[e*cs_se + k]
  int64_t cs_se;
  uint8_t* x8;
  int64_t ld8;            // >= TERMS * (K rounded up to 64); the 64-block's columns past K are written as zero
  int32_t* xs;            // E8M0 scale of row r, block b at xs[b * ldxs + r] (two terms: byte 1 the lo term's)
  int64_t ldxs;
  const bf16* at;         // A_e^T (E, R, K) k contiguous, or NULL
  int64_t at_se, at_sr;
  bf16* low;
  int64_t ldl;
  const int32_t* offsets;
  int E;
};

__device__ __forceinline__ int64_t start_of(const int32_t* offsets, int64_t rows, int e) {
  if (e == 0) return 0;
  const int64_t o = offsets[e - 1];
  return o < 0 ? 0 : (o > rows ? rows : o);
}

// tend[e] = tiles of `bm` rows of experts 0..e (inclusive scan); called by all NT threads
template <int NT>
__device__ __forceinline__ void tile_ends(const int32_t* offsets, int64_t rows, int E, int bm, int* tend, int tid) {
  for (int e = tid; e < E; e += NT) {
    const int64_t c = start_of(offsets, rows, e + 1) - start_of(offsets, rows, e);
    tend[e] = c > 0 ? (int)((c + bm - 1) / bm) : 0;
  }
  __syncthreads();
  if (tid < 64) {
    int run = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + tid;
      int incl = e < E ? tend[e] : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (tid >= o) incl += u;
      }
      if (e < E) tend[e] = run + incl;
      run += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
}

// tile t -> (expert, first row, rows), wave-uniform
__device__ __forceinline__ void decode_tile(const int32_t* offsets, int64_t rows, int E, int bm, const int* tend, int t,
                                            int& e, int64_t& row0, int& mrows) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (tend[mid] > t) hi = mid; else lo = mid + 1;
  }
  e = __builtin_amdgcn_readfirstlane(lo);
  const int t0 = e == 0 ? 0 : __builtin_amdgcn_readfirstlane(tend[e - 1]);
  row0 = start_of(offsets, rows, e) + (int64_t)(t - t0) * bm;
  mrows = (int)min((int64_t)bm, start_of(offsets, rows, e + 1) - row0);
}

// E8M0 byte of the smallest power of two 2^e with amax * 2^-e <= 448 (127 + e; 127 for amax = 0)
__device__ __forceinline__ uint32_t e8m0_for(float amax) {
  const uint32_t b = __float_as_uint(amax);
  if (b == 0u) return 127u;
  const int E = (int)(b >> 23);             // biased exponent of amax (amax >= 0)
  const uint32_t m = b & 0x7FFFFFu;
  const int byte = E - 8 + (m > 0x600000u ? 1 : 0);  // 448 = 1.75 * 2^8
  return (uint32_t)(byte < 0 ? 0 : (byte > 254 ? 254 : byte));
}

// TERMS = 2: each 64-column block also gets the residual x - hi·2^e1 (exact in fp32) quantised the same
// way with its own scale 2^e2; row r's bytes of block b are hi at 128b .. 128b+63, lo at 128b+64 ..
template <int NRB, int TERMS>
__global__ __launch_bounds__(PT) void fp8_prep_kernel(PrepArgs p) {
  constexpr int R = NRB * 16;
  __shared__ __attribute__((aligned(16))) bf16 xt[PR * XP];               // the 64 x 64 chunk of x
  __shared__ __attribute__((aligned(16))) bf16 att[(R > 0 ? R : 1) * XP];  // the R x 64 chunk of A_e^T
  extern __shared__ __attribute__((aligned(16))) int tend[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  tile_ends<PT>(p.offsets, p.rows, p.E, PR, tend, tid);
  const int t = blockIdx.x;
  if (t >= tend[p.E - 1]) return;  // uniform over the workgroup
  int e, mrows;
  int64_t row0;
  decode_tile(p.offsets, p.rows, p.E, PR, tend, t, e, row0, mrows);

  f32x4 lacc[NRB > 0 ? NRB : 1];
#pragma unroll
  for (int rb = 0; rb < (NRB > 0 ? NRB : 1); ++rb) lacc[rb] = f32x4{};
  const int nkb = (p.K + PR - 1) / PR;
  // this thread's two 8-column pieces of the 64 x 64 chunk, the next chunk's loaded while the
  // current one is quantised (and A_e^T's chunk with them)
  auto load_x = [&](int kb, int h) -> u32x4 {
    const int c = tid + h * PT, row = c >> 3, cc = c & 7, col = kb * PR + cc * 8;
    return (kb < nkb && row < mrows && col < p.K) ? *(const u32x4*)(p.x + (row0 + row) * p.ldx + col)
                                                  : u32x4{0u, 0u, 0u, 0u};
  };
  u32x4 nx0 = load_x(0, 0), nx1 = load_x(0, 1);
  for (int kb = 0; kb < nkb; ++kb) {
    const u32x4 cur[2] = {nx0, nx1};
    nx0 = load_x(kb + 1, 0);
    nx1 = load_x(kb + 1, 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = tid + h * PT, row = c >> 3, cc = c & 7;
      const int col = kb * PR + cc * 8;
      const bool ok = row < mrows && col < p.K;
      const u32x4 v = cur[h];
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_bits_to_f32(v[j] & 0xFFFFu);
        f[2 * j + 1] = bf16_bits_to_f32(v[j] >> 16);
      }
      if (p.colscale != nullptr && ok) {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= p.colscale[(int64_t)e * p.cs_se + col + j];
      }
      float amax = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
      amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
      const uint32_t eb = e8m0_for(amax);
      const float inv = __uint_as_float((254u - eb) << 23);  // 2^-(eb - 127), exact
      u32x2 q = {0u, 0u};
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j >> 2] |= f32_to_e4m3(f[j] * inv) << (8 * (j & 3));
      uint32_t word = eb;
      u32x2 q2 = {0u, 0u};
      if constexpr (TERMS == 2) {
        // the residual of each value after its hi term (exact: the hi term is within a factor two of
        // the value, or zero), then its block's scale and bytes
        const float sc = __uint_as_float(eb << 23);  // 2^(eb - 127)
        float amax2 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          f[j] -= fp8_e4m3_to_f32((q[j >> 2] >> (8 * (j & 3))) & 0xFFu) * sc;
          amax2 = fmaxf(amax2, fabsf(f[j]));
        }
        amax2 = fmaxf(amax2, __shfl_xor(amax2, 1, 64));
        amax2 = fmaxf(amax2, __shfl_xor(amax2, 2, 64));
        amax2 = fmaxf(amax2, __shfl_xor(amax2, 4, 64));
        const uint32_t eb2 = e8m0_for(amax2);
        const float inv2 = __uint_as_float((254u - eb2) << 23);
#pragma unroll
        for (int j = 0; j < 8; ++j) q2[j >> 2] |= f32_to_e4m3(f[j] * inv2) << (8 * (j & 3));
        word |= eb2 << 8;
      }
      if (row < mrows) {
        uint8_t* dst = p.x8 + (row0 + row) * p.ld8 + (int64_t)kb * PR * TERMS + cc * 8;
        *(u32x2*)dst = q;
        if constexpr (TERMS == 2) *(u32x2*)(dst + PR) = q2;
        if (cc == 0) p.xs[(int64_t)kb * p.ldxs + row0 + row] = (int32_t)word;
      }
      if constexpr (NRB > 0) *(u32x4*)(xt + row * XP + cc * 8) = v;
    }
    if constexpr (NRB > 0) {
      if (p.at != nullptr) {
        for (int c = tid; c < R * 8; c += PT) {
          const int r = c >> 3, cc = c & 7, col = kb * PR + cc * 8;
          *(u32x4*)(att + r * XP + cc * 8) =
              col < p.K ? *(const u32x4*)(p.at + (int64_t)e * p.at_se + (int64_t)r * p.at_sr + col) : u32x4{0u, 0u, 0u, 0u};
        }
        __syncthreads();
        // wave w: rows 16w .. 16w+15 of the tile times the R columns of A_e, 32 deep per MFMA
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 a = *(const bf16x8*)(xt + (16 * wave + (lane & 15)) * XP + s * 32 + 8 * (lane >> 4));
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb) {
            const bf16x8 b = *(const bf16x8*)(att + (rb * 16 + (lane & 15)) * XP + s * 32 + 8 * (lane >> 4));
            lacc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, lacc[rb], 0, 0, 0);
          }
        }
        __syncthreads();
      }
    }
  }
  if constexpr (NRB > 0) {
    if (p.at != nullptr) {
      // lacc[rb][v]: row 16w + 4*(lane/16) + v, rank rb*16 + lane%16
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * wave + 4 * (lane >> 4) + v;
          if (row < mrows) p.low[(row0 + row) * p.ldl + rb * 16 + (lane & 15)] = (bf16)lacc[rb][v];
        }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// the fp8 grouped product
// ------------------------------------------------------------------------------------------------
constexpr int BM = 256, BN = 256, BK = 64;  // BK in fp8 elements (bytes) per term
constexpr int WAVES_M = 2, WAVES_N = 4, NW = 8, kThreads = 512;
constexpr int FM = BM / WAVES_M / 32, FN = BN / WAVES_N / 32;
constexpr int WI = BN * BK / 16 / (64 * NW);  // 16-byte DMA copies of the stack tile per wave
// TERMS activation terms (1: e4m3 values; 2: hi and lo): a stage holds 64 k of each, the x rows
// 64 * TERMS bytes long; four ring slots for one term, three for two (LDS)
template <int TERMS>
struct Cfg {
  static constexpr int XB = BK * TERMS;                 // bytes of one x row per stage
  static constexpr int CH = XB / 16;                    // its 16-byte chunks
  static constexpr int XI = BM * XB / 16 / (64 * NW);   // x copies per wave per stage
  static constexpr int PS = XI + WI + 1;                // and one 4-byte copy of 64 rows' scale words
  static constexpr int STAGES = TERMS == 2 ? 3 : 4;
  static constexpr int RING = BM * XB + BN * BK + BM * 4;  // bytes of a slot: x, W8, scale words
};
// a slot also holds one of the epilogue's [256][RP + 8] bf16 tiles
template <int NRB, int TERMS>
struct Slot {
  static constexpr int kEpi = BM * (NRB * 16 + 8) * 2;
  static constexpr int kBytes = Cfg<TERMS>::RING > kEpi ? Cfg<TERMS>::RING : kEpi;
};
static_assert(4 * Slot<4, 1>::kBytes + 4096 * 4 <= 163840, "four one-term slots and the largest tile map fit in LDS");
constexpr int kMaxE2 = (163840 - 3 * Slot<4, 2>::kBytes) / 4;  // experts whose tile map fits beside three two-term slots
static_assert(kMaxE2 >= 1024, "three two-term slots leave room for the tile map");
static_assert(Cfg<1>::XI == 2 && Cfg<2>::XI == 4 && WI == 2, "tile split");

struct Args {
  GemmArgs g;          // x unused; w = the fp8 stack with k contiguous (w_sk == 1); low unused
  const uint8_t* x8;
  int64_t ld8;
  const int32_t* xs;
  int64_t ldxs;
  const bf16* lowin;   // bf16(x · A_e) from fp8_prep, or NULL without adapters
  int64_t ldli;
};

// rows of 64 bytes, 16-byte chunk c of row r in slot c ^ ((r >> 2) & 3)
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 2) & 3)) << 4); }
// x rows of 64 * TERMS bytes: four chunks as above; eight: chunk c of row r in slot c ^ ((r >> 1) & 7),
// so the eight rows eight consecutive lanes read (two per 256-byte bank span) hit eight bank groups
template <int TERMS>
__device__ __forceinline__ int swzx(int row, int chunk) {
  if constexpr (TERMS == 1) return swz(row, chunk);
  else return row * Cfg<TERMS>::XB + ((chunk ^ ((row >> 1) & 7)) << 4);
}
template <int TERMS>
__device__ __forceinline__ int swzx_f(int row) { return TERMS == 1 ? (row >> 2) & 3 : (row >> 1) & 7; }

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int TERMS>
struct Feed {
  static constexpr int XI = Cfg<TERMS>::XI, CH = Cfg<TERMS>::CH, XB = Cfg<TERMS>::XB;
  rsrc_t rx, rw, rs;
  uint32_t xo[XI], wo[WI], so;
  int xk[XI], wk[WI];
  int xd[XI], wd[WI], sd;
  int K, ld8;

  __device__ __forceinline__ void init(const Args& a, int64_t row0, int mrows, int e, int n0, int wave, int lane) {
    const GemmArgs& p = a.g;
    rx = make_rsrc(a.x8 + row0 * a.ld8, (int64_t)mrows * a.ld8);
    rw = make_rsrc(p.w + (int64_t)e * p.w_se, p.w_se);
    rs = make_rsrc(a.xs + row0, (a.ldxs * ((p.K + BK - 1) / BK) - row0) * 4);
    K = p.K;
    ld8 = (int)a.ld8;
#pragma unroll
    for (int q = 0; q < XI; ++q) {
      const int instr = wave * XI + q, ci = instr * 64 + lane;
      const int row = ci / CH, c = (ci % CH) ^ swzx_f<TERMS>(row);
      xo[q] = (uint32_t)(row * a.ld8 + c * 16);
      xk[q] = (c % 4) * 16;  // the chunk's first k within its term
      xd[q] = instr * 1024;
    }
#pragma unroll
    for (int q = 0; q < WI; ++q) {
      const int instr = wave * WI + q, ci = instr * 64 + lane;
      const int row = ci >> 2, c = (ci & 3) ^ ((row >> 2) & 3);
      const int n = n0 + row;
      wo[q] = n < p.N ? (uint32_t)((int64_t)n * p.w_sn + c * 16) : 0u;
      wk[q] = n < p.N ? c * 16 : (1 << 30);
      wd[q] = BM * XB + instr * 1024;
    }
    // wave w copies the scale words of rows 64 (w % 4) .. +63 (waves w and w + 4 the same ones)
    so = (uint32_t)((64 * (wave & 3) + lane) * 4);
    sd = BM * XB + BN * BK + 256 * (wave & 3);
  }

  __device__ __forceinline__ void issue(const Args& a, uint8_t* slot, int kt) const {
    const int k0 = kt * BK;
#pragma unroll
    for (int q = 0; q < XI; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(slot + xd[q]), 16,
                                               xk[q] + k0 < K ? xo[q] + (uint32_t)(k0 * TERMS) : kOob, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < WI; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)(slot + wd[q]), 16,
                                               wk[q] + k0 < K ? wo[q] + (uint32_t)k0 : kOob, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(slot + sd), 4,
                                             k0 < K ? so + (uint32_t)(kt * a.ldxs * 4) : kOob, 0, 0, 0);
  }
};

// 32 fp8 values of MFMA operand row r: this lane's half (32 k) of term t's 64, from a row of 64*TERMS bytes
template <int TERMS>
__device__ __forceinline__ v8i x_frag(const uint8_t* xs8, int r, int term, int lane) {
  const int c0 = 4 * term + 2 * (lane >> 5);
  const u32x4 lo = *(const u32x4*)(xs8 + swzx<TERMS>(r, c0));
  const u32x4 hi = *(const u32x4*)(xs8 + swzx<TERMS>(r, c0 + 1));
  return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

template <int AM, int TERMS>
__device__ __forceinline__ void compute(const uint8_t* slot, int lane, int wm, int wn, f32x16 (&acc)[FM][FN]) {
  if constexpr (AM > 0) {
    constexpr int XB = Cfg<TERMS>::XB;
    const uint8_t* xs8 = slot;
    const uint8_t* ws8 = slot + BM * XB;
    const int32_t* sw = (const int32_t*)(slot + BM * XB + BN * BK);
    v8i xf[AM][TERMS], wf[FN];
    int sx[AM];
#pragma unroll
    for (int i = 0; i < AM; ++i) {
      const int r = (i * WAVES_M + wm) * 32 + (lane & 31);
#pragma unroll
      for (int t = 0; t < TERMS; ++t) xf[i][t] = x_frag<TERMS>(xs8, r, t, lane);
      sx[i] = sw[r];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = (wn * FN + j) * 32 + (lane & 31);
      const u32x4 lo = *(const u32x4*)(ws8 + swz(n, 2 * (lane >> 5)));
      const u32x4 hi = *(const u32x4*)(ws8 + swz(n, 2 * (lane >> 5) + 1));
      wf[j] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
    // term t's scale is byte t of the row's scale word (the MFMA's scale operand selects the byte)
#pragma unroll
    for (int i = 0; i < AM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[j], xf[i][0], acc[i][j], 0, 0, 0, 127, 0, sx[i]);
        if constexpr (TERMS == 2)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[j], xf[i][1], acc[i][j], 0, 0, 0, 127, 1, sx[i]);
      }
  }
}

template <int S, int AM, int TERMS>
__device__ __forceinline__ void stage(const Args& a, const Feed<TERMS>& f, uint8_t* const (&slots)[4],
                                      int kt, int lane, int wm, int wn, f32x16 (&acc)[FM][FN]) {
  constexpr int ST = Cfg<TERMS>::STAGES;
  wait_vm<Cfg<TERMS>::PS * (ST - 2)>();
  stage_barrier();
  f.issue(a, slots[(S + ST - 1) % ST], kt + ST - 1);
  compute<AM, TERMS>(slots[S], lane, wm, wn, acc);
}

template <int AM, int TERMS>
__device__ __forceinline__ void kloop(const Args& a, const Feed<TERMS>& f, uint8_t* const (&slots)[4],
                                      int nk, int lane, int wm, int wn, f32x16 (&acc)[FM][FN]) {
  constexpr int ST = Cfg<TERMS>::STAGES;
  int kt = 0;
  if constexpr (ST == 4) {
    for (; kt + 4 <= nk; kt += 4) {
      stage<0, AM, TERMS>(a, f, slots, kt, lane, wm, wn, acc);
      stage<1, AM, TERMS>(a, f, slots, kt + 1, lane, wm, wn, acc);
      stage<2, AM, TERMS>(a, f, slots, kt + 2, lane, wm, wn, acc);
      stage<3, AM, TERMS>(a, f, slots, kt + 3, lane, wm, wn, acc);
    }
    const int rem = nk - kt;
    if (rem > 0) stage<0, AM, TERMS>(a, f, slots, kt, lane, wm, wn, acc);
    if (rem > 1) stage<1, AM, TERMS>(a, f, slots, kt + 1, lane, wm, wn, acc);
    if (rem > 2) stage<2, AM, TERMS>(a, f, slots, kt + 2, lane, wm, wn, acc);
  } else {
    for (; kt + 3 <= nk; kt += 3) {
      stage<0, AM, TERMS>(a, f, slots, kt, lane, wm, wn, acc);
      stage<1, AM, TERMS>(a, f, slots, kt + 1, lane, wm, wn, acc);
      stage<2, AM, TERMS>(a, f, slots, kt + 2, lane, wm, wn, acc);
    }
    const int rem = nk - kt;
    if (rem > 0) stage<0, AM, TERMS>(a, f, slots, kt, lane, wm, wn, acc);
    if (rem > 1) stage<1, AM, TERMS>(a, f, slots, kt + 1, lane, wm, wn, acc);
  }
}

// the tile map of BM-row tiles (as the bf16 kernel's)
__device__ __forceinline__ Item decode(const GemmArgs& p, int64_t item, int nb, const int* tend) {
  const int t = (int)(item / nb);
  Item it;
  it.nblk = (int)(item - (int64_t)t * nb);
  int e, mrows;
  int64_t row0;
  decode_tile(p.offsets, p.rows, p.E, BM, tend, t, e, row0, mrows);
  it.e = e;
  it.row0 = row0;
  it.mrows = mrows;
  it.n0 = it.nblk * BN;
  return it;
}

template <int NRB, int TERMS>
__global__ __launch_bounds__(kThreads, 1) void fp8_gemm_kernel(Args a) {
  constexpr int RP = NRB * 16;
  constexpr int LP = RP + 8;
  constexpr int SB = Slot<NRB, TERMS>::kBytes;
  constexpr int ST = Cfg<TERMS>::STAGES;
  __shared__ __attribute__((aligned(16))) uint8_t slot0[SB];
  __shared__ __attribute__((aligned(16))) uint8_t slot1[SB];
  __shared__ __attribute__((aligned(16))) uint8_t slot2[SB];
  __shared__ __attribute__((aligned(16))) uint8_t slot3[ST == 4 ? SB : 16];
  extern __shared__ __attribute__((aligned(16))) int tend[];
  static_assert(BM * LP * 2 <= SB && BN * LP * 2 <= SB, "the epilogue's tiles fit in a slot");
  uint8_t* const slots[4] = {slot0, slot1, slot2, ST == 4 ? slot3 : slot0};  // three slots: the fourth unused
  const GemmArgs& p = a.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  bf16* Ls = (bf16*)slot0;
  bf16* Lb = (bf16*)slot1;

  tile_ends<kThreads>(p.offsets, p.rows, p.E, BM, tend, tid);
  const int nb = (p.N + BN - 1) / BN;
  const int64_t total = (int64_t)__builtin_amdgcn_readfirstlane(tend[p.E - 1]) * nb;
  const int xcd = blockIdx.x % kXcds, wg_slot = blockIdx.x / kXcds, per_xcd = gridDim.x / kXcds;
  const int64_t chunk = (total + kXcds - 1) / kXcds;
  const int64_t beg = xcd * chunk, end = min(beg + chunk, total);
  const int nk = (p.K + BK - 1) / BK;

  for (int64_t item = beg + wg_slot; item < end; item += per_xcd) {
    const Item it = decode(p, item, nb, tend);
    const int e = it.e, n0 = it.n0, mrows = it.mrows;
    const int64_t row0 = it.row0;
    const int mb = (mrows + 31) >> 5;
    const int am = min(FM, max(0, (mb - wm + WAVES_M - 1) / WAVES_M));
    Feed<TERMS> f;
    f.init(a, row0, mrows, e, n0, wave, lane);
    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

    __syncthreads();  // the previous item's epilogue is done with the LDS
#pragma unroll
    for (int s = 0; s < ST - 1; ++s) f.issue(a, slots[s], s);
    switch (am) {
      case 4: kloop<4, TERMS>(a, f, slots, nk, lane, wm, wn, acc); break;
      case 3: kloop<3, TERMS>(a, f, slots, nk, lane, wm, wn, acc); break;
      case 2: kloop<2, TERMS>(a, f, slots, nk, lane, wm, wn, acc); break;
      case 1: kloop<1, TERMS>(a, f, slots, nk, lane, wm, wn, acc); break;
      default: kloop<0, TERMS>(a, f, slots, nk, lane, wm, wn, acc); break;
    }
    wait_vm<0>();
    __syncthreads();

    // ---- epilogue (as the bf16 kernel's; the low tile comes from fp8_prep) ----
    const int col_l = 4 * (lane >> 5);
    f32x4 cs[FN][4];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (p.scale_kind == MLORA_SCALE_EXPERT) {
          const float c = p.scale[e];
          cs[j][g] = f32x4{c, c, c, c};
        } else if (p.scale_kind == MLORA_SCALE_ROW) {
          const int n = n0 + (wn * FN + j) * 32 + 8 * g + col_l;
          cs[j][g] = n < p.N ? *(const f32x4*)(p.scale + (int64_t)e * p.scale_se + n) : f32x4{};
        } else {
          cs[j][g] = f32x4{1.f, 1.f, 1.f, 1.f};
        }
      }
    const bool lora_on = NRB > 0 && a.lowin != nullptr && p.scaling != 0.f;
    if constexpr (NRB > 0) {
      if (lora_on) {
        for (int c = tid; c < BM * RP / 8; c += kThreads) {
          const int m = c / (RP / 8), rc = (c - m * (RP / 8)) * 8;
          *(u32x4*)(Ls + m * LP + rc) = m < mrows ? *(const u32x4*)(a.lowin + (row0 + m) * a.ldli + rc) : u32x4{0u, 0u, 0u, 0u};
        }
        const rsrc_t rbt = make_rsrc(p.bt + (int64_t)e * p.bt_se, (int64_t)p.N * p.bt_sn * 2);
        for (int c = tid; c < BN * RP / 8; c += kThreads) {
          const int nn = c / (RP / 8), rc = (c - nn * (RP / 8)) * 8;
          const int n = n0 + nn;
          *(u32x4*)(Lb + nn * LP + rc) = ld128(rbt, n < p.N ? (uint32_t)((n * p.bt_sn + rc) * 2) : kOob);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = (i * WAVES_M + wm) * 32 + (lane & 31);
      if (i >= am) continue;
      bf16* orow = p.out + (row0 + row) * p.ldo;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        f32x16 t = f32x16{};
        if constexpr (NRB > 0) {
          if (lora_on) {
#pragma unroll
            for (int rk = 0; rk < NRB; ++rk) {
              const bf16x8 lf = *(const bf16x8*)(Ls + row * LP + rk * 16 + (lane >> 5) * 8);
              const bf16x8 bfr = *(const bf16x8*)(Lb + ((wn * FN + j) * 32 + (lane & 31)) * LP + rk * 16 + (lane >> 5) * 8);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr, lf, t, 0, 0, 0);
            }
          }
        }
        if (row >= mrows) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + (wn * FN + j) * 32 + 8 * g + col_l;
          if (n >= p.N) continue;
          f32x4 bias = {0.f, 0.f, 0.f, 0.f};
          if (p.bias != nullptr) {
            const bf16* bp = p.bias + (int64_t)e * p.bias_se + n;
            bias = f32x4{(float)bp[0], (float)bp[1], (float)bp[2], (float)bp[3]};
          }
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = acc[i][j][4 * g + q] * cs[j][g][q] + p.scaling * t[4 * g + q] + bias[q];
          u32x2 v;
          v[0] = pack_bf16x2(o[0], o[1]);
          v[1] = pack_bf16x2(o[2], o[3]);
          *(u32x2*)(orow + n) = v;
        }
      }
    }
  }
}

// every variant instantiated here: clang otherwise left some host stubs undefined (the library then fails to load)
template __global__ void fp8_gemm_kernel<0, 1>(Args);
template __global__ void fp8_gemm_kernel<1, 1>(Args);
template __global__ void fp8_gemm_kernel<2, 1>(Args);
template __global__ void fp8_gemm_kernel<3, 1>(Args);
template __global__ void fp8_gemm_kernel<4, 1>(Args);
template __global__ void fp8_gemm_kernel<0, 2>(Args);
template __global__ void fp8_gemm_kernel<1, 2>(Args);
template __global__ void fp8_gemm_kernel<2, 2>(Args);
template __global__ void fp8_gemm_kernel<3, 2>(Args);
template __global__ void fp8_gemm_kernel<4, 2>(Args);

template <int NRB, int TERMS>
static int launch_gemm(const Args& a, hipStream_t s) {
  auto kern = fp8_gemm_kernel<NRB, TERMS>;
  const size_t lds = (size_t)a.g.E * sizeof(int);
  static std::mutex mu;
  static std::unordered_map<int64_t, int> grid_cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail("fp8_gemm: hipGetDevice failed");
  int grid = 0;
  {
    std::lock_guard<std::mutex> g(mu);
    const int64_t key = ((int64_t)dev << 32) | (int64_t)lds;
    auto it = grid_cache.find(key);
    if (it != grid_cache.end()) {
      grid = it->second;
    } else {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail("fp8_gemm: cannot grant %zu bytes of LDS", lds);
      int cus = 0, per_cu = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return fail("fp8_gemm: cannot read the compute unit count");
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kern, kThreads, lds) != hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      grid = (cus * per_cu + kXcds - 1) / kXcds * kXcds;
      grid_cache[key] = grid;
    }
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, s, a);
  return launch_status("fp8_gemm");
}

}  // namespace f8
}  // namespace mlora

using namespace mlora;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int mlora_fp8_prep(const void* x, int64_t ldx, int64_t rows, int K, int terms, const float* colscale, int64_t cs_se,
                              void* x8, int64_t ld8, int32_t* xs, int64_t ldxs, const void* at, int64_t at_se,
                              int64_t at_sr, int rank, void* low, int64_t ldl, const int32_t* offsets, int E,
                              void* stream) {
  clear_error();
  if (rows < 0) return fail("fp8_prep: rows=%lld is negative", (long long)rows);
  if (E < 1 || E > 4096) return fail("fp8_prep: E=%d outside [1, 4096]", E);
  if (K < 16 || K % 16) return fail("fp8_prep: K=%d must be a positive multiple of 16", K);
  if (terms != 1 && terms != 2) return fail("fp8_prep: terms=%d is neither 1 nor 2", terms);
  const int64_t kpad = (int64_t)(K + 63) / 64 * 64;
  if (ldx < K || ldx % 8 || !aligned16(x)) return fail("fp8_prep: x needs 16-byte aligned rows of >= K values");
  if (ld8 < terms * kpad || ld8 % 16 || !aligned16(x8))
    return fail("fp8_prep: x8 needs 16-byte aligned rows of >= %lld bytes", (long long)(terms * kpad));
  if (ldxs < rows || ((uintptr_t)xs & 3u)) return fail("fp8_prep: xs needs a block stride >= rows");
  if (at != nullptr) {
    if (rank < 16 || rank > kMaxRank || rank % 16) return fail("fp8_prep: rank=%d must be 16, 32, 48 or 64", rank);
    if (at_sr < K || at_sr % 8 || at_se % 8 || !aligned16(at)) return fail("fp8_prep: A^T needs 16-byte aligned rows of >= K values");
    if (low == nullptr || ldl < rank || ldl % 8 || !aligned16(low)) return fail("fp8_prep: low needs 16-byte aligned rows of >= rank values");
  }
  if (rows == 0) return 0;
  if (rows > 0x7FFFFFFFLL - (int64_t)E * 64) return fail("fp8_prep: rows=%lld too large", (long long)rows);
  f8::PrepArgs p;
  p.x = (const bf16*)x; p.ldx = ldx; p.rows = rows; p.K = K;
  p.colscale = colscale; p.cs_se = cs_se;
  p.x8 = (uint8_t*)x8; p.ld8 = ld8; p.xs = xs; p.ldxs = ldxs;
  p.at = (const bf16*)at; p.at_se = at_se; p.at_sr = at_sr; p.low = (bf16*)low; p.ldl = ldl;
  p.offsets = offsets; p.E = E;
  const int grid = (int)(rows / f8::PR + E);
  const size_t lds = (size_t)E * sizeof(int);
  hipStream_t s = as_stream(stream);
#define MLORA_PREP(NRB)                                                                      \
  do {                                                                                       \
    if (terms == 2) hipLaunchKernelGGL((f8::fp8_prep_kernel<NRB, 2>), dim3(grid), dim3(f8::PT), lds, s, p); \
    else hipLaunchKernelGGL((f8::fp8_prep_kernel<NRB, 1>), dim3(grid), dim3(f8::PT), lds, s, p);            \
  } while (0)
  switch (at == nullptr ? 0 : rank / 16) {
    case 0: MLORA_PREP(0); break;
    case 1: MLORA_PREP(1); break;
    case 2: MLORA_PREP(2); break;
    case 3: MLORA_PREP(3); break;
    default: MLORA_PREP(4); break;
  }
#undef MLORA_PREP
  return launch_status("fp8_prep");
}

extern "C" int mlora_fp8_gemm(const void* x8, int64_t ld8, const int32_t* xs, int64_t ldxs, int64_t rows, int K, int terms,
                              int N,
                              const void* w, int64_t w_se, int64_t w_sn, const float* scale, int scale_kind,
                              int64_t scale_se, const void* low, int64_t ldli, const void* bt, int64_t bt_se,
                              int64_t bt_sn, int rank, float scaling, const void* bias, int64_t bias_se, void* out,
                              int64_t ldo, const int32_t* offsets, int E, void* stream) {
  clear_error();
  if (rows < 0) return fail("fp8_gemm: rows=%lld is negative", (long long)rows);
  if (E < 1 || E > 4096) return fail("fp8_gemm: E=%d outside [1, 4096]", E);
  if (K < 16 || K % 16) return fail("fp8_gemm: K=%d must be a positive multiple of 16", K);
  if (terms != 1 && terms != 2) return fail("fp8_gemm: terms=%d is neither 1 nor 2", terms);
  if (terms == 2 && E > f8::kMaxE2) return fail("fp8_gemm: E=%d past the %d experts of the two-term tile map", E, f8::kMaxE2);
  if (N < 8 || N % 8) return fail("fp8_gemm: N=%d must be a positive multiple of 8", N);
  const int64_t kpad = (int64_t)(K + 63) / 64 * 64;
  if (ld8 < terms * kpad || ld8 % 16 || !aligned16(x8))
    return fail("fp8_gemm: x8 needs 16-byte aligned rows of >= %lld bytes", (long long)(terms * kpad));
  if ((int64_t)f8::BM * ld8 > 0x7FFFFFF0) return fail("fp8_gemm: x8 row stride %lld too large", (long long)ld8);
  if (ldxs < rows || ((uintptr_t)xs & 3u)) return fail("fp8_gemm: xs needs a block stride >= rows");
  if (ldxs * (kpad / 64) * 4 > 0x7FFFFFF0) return fail("fp8_gemm: the scale words exceed 2 GiB");
  if (w_sn < K || w_sn % 16 || w_se % 16 || !aligned16(w)) return fail("fp8_gemm: the stack needs 16-byte aligned rows of >= K bytes, k contiguous");
  if (w_se > 0x7FFFFFF0) return fail("fp8_gemm: one expert's weights exceed 2 GiB");
  if (scale_kind < 0 || scale_kind > 2) return fail("fp8_gemm: scale_kind %d unknown", scale_kind);
  if (scale_kind != MLORA_SCALE_NONE && scale == nullptr) return fail("fp8_gemm: scale_kind %d without a scale", scale_kind);
  if (scale_kind == MLORA_SCALE_ROW && (scale_se < N || ((uintptr_t)scale & 15u)))
    return fail("fp8_gemm: a per-row scale needs 16-byte aligned rows of >= N values");
  if (ldo < N || ldo % 8 || !aligned16(out)) return fail("fp8_gemm: out needs 16-byte aligned rows of >= N values");
  if (low != nullptr) {
    if (bt == nullptr) return fail("fp8_gemm: low without B");
    if (rank < 16 || rank > kMaxRank || rank % 16) return fail("fp8_gemm: rank=%d must be 16, 32, 48 or 64", rank);
    if (ldli < rank || ldli % 8 || !aligned16(low)) return fail("fp8_gemm: low needs 16-byte aligned rows of >= rank values");
    if (bt_sn < rank || bt_sn % 8 || bt_se % 8 || !aligned16(bt)) return fail("fp8_gemm: B^T needs 16-byte aligned rows of >= rank values");
  }
  if (rows == 0) return 0;
  f8::Args a{};
  GemmArgs& g = a.g;
  g.x = nullptr; g.ldx = 0; g.gather = nullptr; g.gk = 1; g.xrows = 0; g.row_scale = nullptr; g.row_scale_dt = 0;
  g.w = (const uint8_t*)w; g.w_se = w_se; g.w_sk = 1; g.w_sn = w_sn;
  g.scale = scale; g.scale_se = scale_se; g.scale_kind = scale_kind;
  g.nf4_q = nullptr; g.nf4_absmax2 = nullptr; g.nf4_code2 = nullptr; g.nf4_offset = nullptr; g.nf4_code = nullptr;
  g.at = nullptr; g.at_se = 0; g.at_sr = 0;
  g.bt = (const bf16*)bt; g.bt_se = bt_se; g.bt_sn = bt_sn;
  g.rank = low != nullptr ? rank : 0; g.scaling = scaling;
  g.bias = (const bf16*)bias; g.bias_se = bias_se;
  g.out = (bf16*)out; g.ldo = ldo; g.low = nullptr; g.ldl = 0;
  g.offsets = offsets; g.rows = rows; g.E = E; g.K = K; g.N = N;
  a.x8 = (const uint8_t*)x8; a.ld8 = ld8; a.xs = xs; a.ldxs = ldxs;
  a.lowin = (const bf16*)low; a.ldli = ldli;
  hipStream_t s = as_stream(stream);
#define MLORA_F8(NRB) return terms == 2 ? f8::launch_gemm<NRB, 2>(a, s) : f8::launch_gemm<NRB, 1>(a, s)
  switch (low == nullptr ? 0 : rank / 16) {
    case 0: MLORA_F8(0);
    case 1: MLORA_F8(1);
    case 2: MLORA_F8(2);
    case 3: MLORA_F8(3);
    default: MLORA_F8(4);
  }
#undef MLORA_F8
}
