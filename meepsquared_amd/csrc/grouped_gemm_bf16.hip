// The grouped product for bf16 stacks, fed by LDS DMA through a multi-stage ring (gfx950).
//
//   out_e = c · x_e W_e + scaling · bf16(x_e A_e) B_e + bias_e         for every expert e
//
// (with gathered rows, each output row may be multiplied by a per-row scale before the bias)
//
// Same work decomposition as the register-staged kernel (grouped_gemm.hip): a persistent grid,
// each workgroup deriving the tile map in LDS, items split into one contiguous range per XCD.
// What differs is how operands reach LDS and how deep the pipeline is:
//   * x tiles, W tiles and A_e^T tiles are copied from HBM/L2 straight into LDS by
//     buffer_load_dwordx4 ... lds (16 bytes per lane, lane-linear in LDS): no staging registers,
//     no ds_write, and the copy runs asynchronously behind the MFMAs;
//   * a ring of STAGES BK-deep stages: the copy of stage kt + STAGES - 1 is issued while stage kt is
//     multiplied, so each copy has STAGES - 1 iterations of MFMA work to hide its latency; a wave
//     waits (s_waitcnt vmcnt) only for its own copies of the stage it is about to read, then one
//     barrier per stage publishes every wave's copies;
//   * a stack with k contiguous (the forward pass of an (E, out, in) stack) is held as [n][k]; a
//     stack with n contiguous (the input-gradient pass) is held as it lies in memory, [k][n], and
//     read with ds_read_b64_tr_b16, which returns each lane four consecutive k of one column: the
//     MFMA operand, with no transpose pass;
//   * the global addresses of each DMA lane are chosen so that the lane-linear LDS image is
//     XOR-swizzled: MFMA operand reads (16 lanes per cycle) hit 16 distinct bank groups.
// Waves are WAVES_M x WAVES_N; wave (wm, wn) owns the interleaved 32-row blocks i*WAVES_M + wm and
// 32-column blocks j*WAVES_N + wn; the K loop is specialised on the number of its row blocks that
// hold rows of the expert (the last tile of an expert is usually partial), with no branch inside.
// An expert's last tile of at most XR rows past a full one is merged into it (a "tall" item, the
// TALL instantiation): each wave then also multiplies the extra rows by its column block wm*WAVES_N+wn.
//
// Reference behaviour: src/meepsquared/_grouped.py:120-221 (_grouped_gemm_kernel), :313-345 (_launch).
#include <mutex>
#include <unordered_map>

#include "gemm_common.hpp"

namespace mlora {
namespace dma {

#ifndef MLORA_DMA_WM
#define MLORA_DMA_WM 2
#endif
#ifndef MLORA_DMA_WN
#define MLORA_DMA_WN 4
#endif
#ifndef MLORA_DMA_OCC
#define MLORA_DMA_OCC 1
#endif

#ifndef MLORA_DMA_BK
#define MLORA_DMA_BK 64
#endif
#ifndef MLORA_DMA_STAGES
#define MLORA_DMA_STAGES 2
#endif
constexpr int BM = 256, BN = 256, BK = MLORA_DMA_BK, STAGES = MLORA_DMA_STAGES;
constexpr int CPR = BK / 8;  // 16-byte chunks per [row][k] tile row
static_assert((BK == 32 && STAGES == 4) || (BK == 64 && STAGES == 2), "ring shapes");
constexpr int WAVES_M = MLORA_DMA_WM, WAVES_N = MLORA_DMA_WN;
constexpr int NW = WAVES_M * WAVES_N, kThreads = 64 * NW;
constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
constexpr int FM = WTM / 32, FN = WTN / 32;
constexpr int kLS = 2 * FM / WAVES_N;          // 16-row halves of x·A_e per wave
constexpr int XCH = BM * BK / 8, WCH = BN * BK / 8;  // 16-byte chunks per stage
constexpr int XI = XCH / (64 * NW), WI = WCH / (64 * NW);  // DMA instructions per wave per stage
static_assert(XCH % (64 * NW) == 0 && WCH % (64 * NW) == 0, "stages must split evenly over the waves");
static_assert(FM >= 1 && FN >= 1 && (2 * FM) % WAVES_N == 0, "tile shape");

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kSmallLastE = 1024;  // experts up to which the small last tiles are scheduled last
// Tall items: an expert whose rows leave a last tile of at most XR rows after its full tiles has that
// remainder merged into its last full tile, which then holds BM + XR rows at most; each wave takes one
// more 32 x 32 block (the extra rows x its column block wm * WAVES_N + wn), +12.5 % MFMA work on that
// item instead of a near-empty item of its own (which costs most of a full one: its stages are bound
// by the copy latency).  The extra rows' x tile sits at the end of each ring slot.
constexpr int XR = 32;

// The product's column (the stack's row) at column c of the tile whose first column is n0.  With SwiGLU
// fused (swi = half the columns), tile t's first half is gate columns 128 t .. and its second half the up
// columns swi + 128 t .. that pair with them, so that each wave's two 32-column blocks j = 0, 1 hold a gate
// block and its up block in the same lanes.
template <bool SWI>
__device__ __forceinline__ int tile_col(const GemmArgs& p, int n0, int c) {
  if constexpr (!SWI) return n0 + c;
  else return c < BN / 2 ? (n0 >> 1) + c : p.swi + (n0 >> 1) + (c - BN / 2);
}
constexpr bool kSwiOn = FN == 2 && WAVES_N * 64 == BN;  // the pairing above needs these shapes

// [row][k] tiles (rows of BK bf16, CPR chunks of 16 bytes): chunk c of row r in slot c ^ f(r), with f
// spreading the 16 rows one MFMA operand read touches over 16 distinct 16-byte bank groups
__device__ __forceinline__ int swz_f(int row) { return (row >> (CPR == 4 ? 2 : 1)) & (CPR - 1); }
__device__ __forceinline__ int swz_rk(int row, int chunk) { return row * BK + ((chunk ^ swz_f(row)) << 3); }
// [k][n] tiles (rows of BN bf16): chunk c of row k in slot c ^ ((k & 3) << 2)
__device__ __forceinline__ int swz_kn(int k, int chunk) { return k * BN + ((chunk ^ ((k & 3) << 2)) << 3); }

__device__ __forceinline__ void dma16(rsrc_t r, const bf16* lds_dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_dst, 16, voff, 0, 0, 0);
}
// the same with a wave-uniform scalar offset added to the lane's
__device__ __forceinline__ void dma16s(rsrc_t r, const bf16* lds_dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_dst, 16, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left free
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// A workgroup barrier that waits for nothing but this wave's LDS reads: the DMA copies still in
// flight stay in flight (a __syncthreads would wait for them all).  The empty asm statements keep
// the compiler from moving memory accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The tile map in LDS, one int per expert: tend[e] = the number of BM-row tiles of experts 0..e
// (an inclusive scan; tend[E-1] is the tile count).  With tall items an expert's remainder of at most XR
// rows past its full tiles joins its last tile (BM + XR rows at most); with tall2, a larger remainder of at
// most n XR rows past n >= 2 full tiles is spread over the last m = ceil(rem / XR) of them (the first of those
// takes rem - (m - 1) XR extra rows, the others XR each), so that no partial tile of its own is left: a tall
// item costs a few % more than a full one, a partial tile most of one, and near-empty ones fill the launch's
// last round.  Expert e's rows are [start(e), start(e+1)) with
// start(e) = offsets[e-1] clamped into [0, rows] (start(0) = 0), read from global memory when needed.
// With small_last, an expert's last tile when it holds at most BM/2 rows is counted apart, in sfx[e]
// (0 or 1, scanned the same way): those tiles are scheduled after all the others, so that they fill
// the last rounds of the workgroups instead of landing at random (a near-empty tile still costs most
// of a full one: its stages are bound by the copy latency).
__device__ __forceinline__ int64_t row_start(const GemmArgs& p, int e) {
  if (e == 0) return 0;
  const int64_t o = p.offsets[e - 1];
  return o < 0 ? 0 : (o > p.rows ? p.rows : o);
}

__device__ __forceinline__ void scan_wave(int* v, int E, int lane) {  // inclusive scan by one wave
  int run = 0;
  for (int base = 0; base < E; base += 64) {
    const int e = base + lane;
    int incl = e < E ? v[e] : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (lane >= o) incl += u;
    }
    if (e < E) v[e] = run + incl;
    run += __shfl(incl, 63, 64);
  }
}

__device__ __forceinline__ void build_tile_ends(const GemmArgs& p, int* tend, int* sfx, bool small_last, bool tall,
                                                bool tall2, int tid) {
  const int E = p.E;
  for (int e = tid; e < E; e += kThreads) {
    const int64_t c = row_start(p, e + 1) - row_start(p, e);
    int nt = c > 0 ? (int)((c + BM - 1) / BM) : 0;
    if (tall && nt >= 2 && c - (int64_t)(nt - 1) * BM <= XR) --nt;  // the remainder joins the last full tile
    else if (tall2 && nt >= 3 && c - (int64_t)(nt - 1) * BM <= (int64_t)(nt - 1) * XR) --nt;  // ... or the last m
    const int small = small_last && nt > 0 && c - (int64_t)(nt - 1) * BM <= BM / 2;
    tend[e] = nt - small;
    if (small_last) sfx[e] = small;
  }
  __syncthreads();
  if (tid < 64) scan_wave(tend, E, tid);
  else if (small_last && tid < 128) scan_wave(sfx, E, tid - 64);
  __syncthreads();
}

__device__ __forceinline__ int first_above(const int* v, int E, int t) {  // the e with v[e-1] <= t < v[e]
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (v[mid] > t) hi = mid; else lo = mid + 1;
  }
  return __builtin_amdgcn_readfirstlane(lo);
}

// work item (tile t, column block) -> wave-uniform expert, rows and columns; small: t counts the
// small last tiles
// Launches with more than kGroupNb column blocks take their full tiles' items in groups of kGroupRows row
// tiles, column block by column block: the workgroups of one XCD then run a few column blocks of several row
// tiles at a time, each stack tile shared by up to kGroupRows items, instead of one row tile against as many
// column blocks (as many distinct stack tiles per stage as workgroups).  A permutation of [0, T nb): group g
// holds rows = min(kGroupRows, T - g kGroupRows) row tiles, its r-th item is column block r / rows of row
// tile g kGroupRows + r % rows.
constexpr int kGroupRows = 4, kGroupNb = 16;  // (4 measured faster than 2 or 8; at 16 column blocks the row-tile order)
__device__ __forceinline__ int64_t grouped_item(int64_t item, int64_t T, int nb) {
  const int64_t gsz = (int64_t)kGroupRows * nb, g = item / gsz, r = item - g * gsz;
  const int64_t rows = min((int64_t)kGroupRows, T - g * kGroupRows), c = r / rows;
  return (g * kGroupRows + (r - c * rows)) * nb + c;
}

__device__ __forceinline__ Item decode(const GemmArgs& p, int64_t item, int nb, const int* tend, const int* sfx,
                                       bool small, bool tall, bool tall2) {
  const int t = (int)(item / nb);
  Item it;
  it.nblk = (int)(item - (int64_t)t * nb);
  if (!small) {
    it.e = first_above(tend, p.E, t);
    const int t0 = it.e == 0 ? 0 : __builtin_amdgcn_readfirstlane(tend[it.e - 1]);
    it.row0 = row_start(p, it.e) + (int64_t)(t - t0) * BM;
  } else {
    it.e = first_above(sfx, p.E, t);
    const int big = __builtin_amdgcn_readfirstlane(tend[it.e]) -
                    (it.e == 0 ? 0 : __builtin_amdgcn_readfirstlane(tend[it.e - 1]));
    it.row0 = row_start(p, it.e) + (int64_t)big * BM;
  }
  // an item left with at most BM + XR rows is the expert's last (a tall one when it has more than BM)
  const int64_t left = row_start(p, it.e + 1) - it.row0;
  it.mrows = (int)(left <= BM + (tall ? XR : 0) ? left : (int64_t)BM);
  if (tall2 && !small) {  // the expert's remainder spread over its last m tiles (as build_tile_ends counts)
    const int t0 = it.e == 0 ? 0 : __builtin_amdgcn_readfirstlane(tend[it.e - 1]);
    const int nt = __builtin_amdgcn_readfirstlane(tend[it.e]) - t0, j = (int)((it.row0 - row_start(p, it.e)) / BM);
    const int64_t rem = row_start(p, it.e + 1) - row_start(p, it.e) - (int64_t)nt * BM;
    if (nt >= 2 && rem > XR && rem <= (int64_t)nt * XR) {
      const int m = (int)((rem + XR - 1) / XR), first = nt - m, a = (int)(rem - (int64_t)(m - 1) * XR);
      if (j >= first) {
        it.row0 += j == first ? 0 : a + (j - first - 1) * XR;
        it.mrows = BM + (j == first ? a : XR);
      }
    }
  }
  it.n0 = it.nblk * BN;
  return it;
}

// One ring slot: the x tile [BM][BK], the stack tile ([BN][BK] or [BK][BN]) and the A_e^T tile
// [RP][BK].  Each slot is its own LDS object, so the compiler can tell a read of one slot from the
// copies still landing in the others and does not wait for those.
// The A^T tile is copied with RD rows: the rank padded so that the copies split over the eight
// waves in whole runs of lanes (rank 48 is copied as 64 rows, the last 16 read as zeros).
// The stack's element type in LDS: bf16, or fp8 e4m3 / NF4 copied as stored (k contiguous) and
// decoded to bf16 in registers as each MFMA operand is read.
// kWFp8K: fp8 with a per-row stack scale that lies along k here (the input-gradient product of a
// stack with one scale per output row, read through its k-contiguous copy): the stage's BK scales are
// copied beside the tile and applied in the decode, bf16(e4m3 · s_k), as the register-staged kernel does.
// kWNf4T: NF4 codes packed along k whose absmax varies with k (the input-gradient product of an NF4
// stack, read through its transposed copy): the stage's absmax tile, one fp32 per (64 columns, k), is
// copied beside the codes, and each value decodes as bf16(code[nibble] · absmax) from fp32 codes.
enum : int { kWBf16 = 0, kWFp8 = 1, kWNf4 = 2, kWFp8K = 3, kWNf4T = 4 };
template <int WT>
struct WTile {
  static constexpr bool kFp8 = WT == kWFp8 || WT == kWFp8K;
  static constexpr int RowBytes = WT == kWBf16 ? BK * 2 : kFp8 ? BK : BK / 2;         // one row of the stage
  static constexpr int Chunks = RowBytes / 16;                                         // 16-byte chunks per row
  static constexpr int Bytes = BN * RowBytes;                                          // the tile
  static constexpr int Elems = Bytes / 2 + (WT == kWFp8K ? BK * 2 : WT == kWNf4T ? (BN / 64) * BK * 2 : 0);
  //                          bf16 slots of LDS (+ the scales along k, or the absmax tile [BN / 64][BK] fp32)
  static constexpr int WI = BN * Chunks / (64 * NW);                                   // copies per wave
  static_assert(BN * Chunks % (64 * NW) == 0, "the stack tile splits evenly over the waves");
  static_assert((WT != kWFp8K && WT != kWNf4T) || BK == 64, "one dword copy of 64 lanes carries a row of scales");
};
// [n][k] byte tiles of fp8 (4 chunks per row) and NF4 (2): chunk c of row n in slot c ^ g(n)
template <int WT>
__device__ __forceinline__ int swz_q(int n) { return WTile<WT>::kFp8 ? (n >> 2) & 3 : (n >> 3) & 1; }

template <int NRB, int WT = kWBf16, bool TALL = false>
struct SlotSize {
  static constexpr int RD = (NRB == 3 ? 4 : NRB) * 16;
  static constexpr int kXOff = BM * BK + WTile<WT>::Elems + RD * BK;  // the tall rows' x tile [XR][BK]
  static constexpr int kElems = kXOff + (TALL ? XR * BK : 0);
};

// Per-lane DMA addressing of one item, fixed for its whole K loop: each lane's byte offsets at k = 0.
// A stage that lies wholly inside K (every stage when K is a multiple of BK) adds its k offset as the
// copy's scalar offset, with no per-lane test; only a stage that crosses the end of K re-derives each
// lane's k from its lane index and sends the lanes past K out of range (zeros).  Stack columns past N
// are read like the others (inside the stack's buffer range, or zeros past its end) and never stored.
template <bool BKC, int NRB, int WT, bool TALL = false, bool DB = false, bool SWI = false>
struct Feed {
  static_assert(WT == kWBf16 || BKC, "fp8 and NF4 stacks are read with k contiguous");
  static_assert(!DB || (WT == kWBf16 && NRB == 1 && STAGES == 2), "the fused adapter gradient: bf16, rank 16, two slots");
  static constexpr bool kDB = DB;
  static constexpr int RP = NRB * 16;
  static constexpr int CPW = SlotSize<NRB, WT>::RD * BK / 8 / NW;  // A^T chunks per wave per stage
  static_assert(NRB == 0 || (CPW > 0 && 64 % CPW == 0), "each wave's A^T chunks lie in one 64-lane copy");
  static constexpr int WI = WTile<WT>::WI;
  // this wave's copies per stage: XI of x, WI of the stack, one (lane-masked) of A^T
  static constexpr int PS = XI + WI + (NRB > 0 ? 1 : 0);
  rsrc_t rx, rw, ra, rs;  // rs: the expert's scales along k (kWFp8K)
  // TALL: the extra rows' x tile, copied by waves 0 .. XR * CPR / 64 - 1 (one instruction each) when the
  // item holds more than BM rows.  Waves issue different counts then: the ring waits for every copy
  // of a wave (vmcnt 0) with two slots, so the counts need not match.
  static constexpr int kTallWaves = XR * CPR / 64;
  static_assert(!TALL || (STAGES == 2 && (XR * CPR) % 64 == 0 && kTallWaves <= NW), "tall rows' copies");
  uint32_t to;
  int td;
  bool t_on;
  uint32_t xo[XI], wo[WI], ao;
  int xd[XI], wd[WI], ad;  // LDS element offset of each instruction's 64 lanes within the slot
  bool a_on;
  int lane_, wave_, n0_;
  int64_t wstep;           // bytes the stack offset advances per k (BKC: 2; else 2 * w_sk)
  // DB: the item's share of the fused adapter gradient.  Stage kt is this item's when kt % nb == nblk
  // (the column blocks of a row tile take turns), and on the item's j-th such stage the waves of row
  // group j % 2 (waves 0-3 or 4-7, in turn) each sum 16 of its 64 columns over all the tile's rows.
  const bf16* dbt_;        // LDS [BM + XR][16]: l of the tile's rows, zeros past its rows
  rsrc_t rdbw;             // the tile's partial sums in the workspace, [16][K] fp32
  int nb_, nblk_, mrows_;
  mutable int db_next_, db_j_;  // the item's next such stage and how many came before it
  // whether this wave sums on stage kt; called once per stage, in order (kt = 0, 1, ...)
  __device__ __forceinline__ bool db_step(int kt) const {
    if constexpr (!DB) {
      return false;
    } else {
      const bool hit = kt == db_next_;
      const bool mine = hit && (db_j_ & 1) == (wave_ >> 2);
      db_j_ += hit ? 1 : 0;
      db_next_ += hit ? nb_ : 0;
      return mine;
    }
  }

  // the k (within a stage) of this lane's chunk in copy q of the x tile, the stack tile, the A^T tile
  // and the tall rows' tile
  __device__ __forceinline__ static int x_k(int wave, int q, int lane) {
    const int ci = (wave * XI + q) * 64 + lane, row = ci / CPR;
    return ((ci % CPR) ^ swz_f(row)) * 8;
  }
  __device__ __forceinline__ static int w_k(int wave, int q, int lane) {
    const int ci = (wave * WI + q) * 64 + lane;
    if constexpr (WT != kWBf16) {
      constexpr int CH = WTile<WT>::Chunks;
      const int row = ci / CH;
      return ((ci % CH) ^ swz_q<WT>(row)) * (WTile<WT>::kFp8 ? 16 : 32);
    } else if constexpr (BKC) {
      const int row = ci / CPR;
      return ((ci % CPR) ^ swz_f(row)) * 8;
    } else {
      return ci / (BN / 8);
    }
  }
  __device__ __forceinline__ static int a_k(int wave, int lane) {
    const int ci = ((wave * CPW) >> 6) * 64 + lane, r = ci / CPR;
    return ((ci % CPR) ^ swz_f(r)) * 8;
  }
  __device__ __forceinline__ static int t_k(int wave, int lane) {
    const int ci = wave * 64 + lane, row = ci / CPR;
    return ((ci % CPR) ^ swz_f(row)) * 8;
  }

  __device__ __forceinline__ void init(const GemmArgs& p, int n0, int64_t row0, int mrows, int wave, int lane) {
    lane_ = lane;
    wave_ = wave;
    n0_ = n0;
#pragma unroll
    for (int q = 0; q < XI; ++q) {
      const int instr = wave * XI + q, ci = instr * 64 + lane;
      const int row = ci / CPR, c = (ci % CPR) ^ swz_f(row);
      if (p.gather == nullptr) {
        xo[q] = (uint32_t)((row * p.ldx + c * 8) * 2);
      } else {  // the row's source row of x (x's resource spans all of x)
        // (32-bit division: the routed rows number below 2^32, checked at the ABI)
        const int64_t src = row < mrows ? (int64_t)((uint32_t)p.gather[row0 + row] / (uint32_t)p.gk) : -1;
        xo[q] = src >= 0 ? (uint32_t)((src * p.ldx + c * 8) * 2) : kOob;
      }
      xd[q] = instr * 512;
    }
#pragma unroll
    for (int q = 0; q < WI; ++q) {
      const int instr = wave * WI + q, ci = instr * 64 + lane;
      if constexpr (WT != kWBf16) {  // [n][k] bytes: fp8 one per k, NF4 one per two k
        constexpr int CH = WTile<WT>::Chunks;
        const int row = ci / CH, c = (ci % CH) ^ swz_q<WT>(row);
        const int n = tile_col<SWI>(p, n0, row);
        const int64_t rowb = WTile<WT>::kFp8 ? (int64_t)n * p.w_sn : (int64_t)n * p.w_sn / 2;
        wo[q] = (uint32_t)(rowb + c * 16);
      } else if constexpr (BKC) {  // [n][k]
        const int row = ci / CPR, c = (ci % CPR) ^ swz_f(row);
        const int n = tile_col<SWI>(p, n0, row);
        wo[q] = (uint32_t)(((int64_t)n * p.w_sn + c * 8) * 2);
      } else {  // [k][n]
        const int kr = ci / (BN / 8), c = (ci % (BN / 8)) ^ ((kr & 3) << 2);
        const int n = tile_col<SWI>(p, n0, c * 8);
        wo[q] = (uint32_t)(((int64_t)kr * p.w_sk + n) * 2);
      }
      wd[q] = BM * BK + instr * 512;
    }
    wstep = WTile<WT>::kFp8 ? 1 : BKC ? 2 : 2 * p.w_sk;
    if constexpr (TALL) {
      t_on = mrows > BM && wave < kTallWaves;
      const int ci = wave * 64 + lane, row = ci / CPR, c = (ci % CPR) ^ swz_f(row);
      if (p.gather == nullptr) {
        to = (uint32_t)(((BM + row) * p.ldx + c * 8) * 2);  // rows past the item: past its resource, zeros
      } else {
        const int64_t src = BM + row < mrows ? (int64_t)((uint32_t)p.gather[row0 + BM + row] / (uint32_t)p.gk) : -1;
        to = src >= 0 ? (uint32_t)((src * p.ldx + c * 8) * 2) : kOob;
      }
      td = SlotSize<NRB, WT, true>::kXOff + wave * 512;
    }
    if constexpr (NRB > 0) {
      // wave w copies chunks [w * CPW, (w + 1) * CPW) of the A^T tile: lanes of one 64-chunk
      // instruction block, the others masked off (their LDS bytes belong to other waves)
      const int c0 = wave * CPW, blk = c0 >> 6;
      const int ci = blk * 64 + lane;
      const int r = ci / CPR, c = (ci % CPR) ^ swz_f(r);
      ao = (uint32_t)((r * p.at_sr + c * 8) * 2);
      ad = BM * BK + WTile<WT>::Elems + blk * 512;
      a_on = lane >= (c0 & 63) && lane < (c0 & 63) + CPW;
    }
  }

  // the copies of stage kt into `slot` (past the end of K they read zeros, so the count per stage
  // never changes), in three parts that the K loop spreads over a stage's MFMAs: the x tile, the
  // stack tile (with its scales), the A^T tile
  __device__ __forceinline__ void issue(const GemmArgs& p, bf16* slot, int kt) const {
    issue_part<0>(p, slot, kt);
    issue_part<1>(p, slot, kt);
    issue_part<2>(p, slot, kt);
  }
  template <int PART>
  __device__ __forceinline__ void issue_part(const GemmArgs& p, bf16* slot, int kt) const {
    const int k0 = kt * BK;
    const uint32_t wk0 = WT == kWNf4 || WT == kWNf4T ? (uint32_t)(k0 / 2) : (uint32_t)(k0 * wstep);
    if (k0 + BK <= p.K) {  // the whole stage inside K: the k offset rides in the scalar offset
      if constexpr (PART == 0) {
#pragma unroll
        for (int q = 0; q < XI; ++q) dma16s(rx, slot + xd[q], xo[q], (uint32_t)(k0 * 2));
        if constexpr (TALL) {
          if (t_on) dma16s(rx, slot + td, to, (uint32_t)(k0 * 2));
        }
      }
      if constexpr (PART == 1) {
#pragma unroll
        for (int q = 0; q < WI; ++q) dma16s(rw, slot + wd[q], wo[q], wk0);
      }
      if constexpr (PART == 2 && NRB > 0) {
        if (a_on) dma16s(ra, slot + ad, ao, (uint32_t)(k0 * 2));
      }
    } else {  // the stage crosses the end of K: each lane's k, from its lane index (kept out of the loop)
      int lane = lane_;
      asm volatile("" : "+v"(lane));
      if constexpr (PART == 0) {
#pragma unroll
        for (int q = 0; q < XI; ++q)
          dma16(rx, slot + xd[q], x_k(wave_, q, lane) + k0 < p.K ? xo[q] + (uint32_t)(k0 * 2) : kOob);
        if constexpr (TALL) {
          if (t_on) dma16(rx, slot + td, t_k(wave_, lane) + k0 < p.K ? to + (uint32_t)(k0 * 2) : kOob);
        }
      }
      if constexpr (PART == 1) {
#pragma unroll
        for (int q = 0; q < WI; ++q) dma16(rw, slot + wd[q], w_k(wave_, q, lane) + k0 < p.K ? wo[q] + wk0 : kOob);
      }
      if constexpr (PART == 2 && NRB > 0) {
        if (a_on) dma16(ra, slot + ad, a_k(wave_, lane) + k0 < p.K ? ao + (uint32_t)(k0 * 2) : kOob);
      }
    }
    if constexpr (PART == 1 && WT == kWNf4T) {  // waves 0 .. BN/64 - 1: one row of the absmax tile each
      if (wave_ < BN / 64) {
        const int nbg = tile_col<SWI>(p, n0_, wave_ * 64) / 64;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void*)(slot + BM * BK + WTile<WT>::Bytes / 2 + wave_ * BK * 2), 4,
            nbg < p.N / 64 && k0 + lane_ < p.K ? (uint32_t)(((int64_t)nbg * p.K + k0 + lane_) * 4) : kOob, 0, 0, 0);
      }
    }
    if constexpr (PART == 1 && WT == kWFp8K) {  // every wave copies the same 64 scales (one dword per lane)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(slot + BM * BK + WTile<WT>::Bytes / 2), 4,
                                               k0 + lane_ < p.K ? (uint32_t)((k0 + lane_) * 4) : kOob, 0, 0, 0);
    }
  }

  // DB: this stage's part of the adapter gradient, columns 16 (wave % 4) .. + 15 of the stage's x tile
  // summed over the tile's rows against l: a 16 x 16 block (column x rank) from 32-row chunks on
  // v_mfma_f32_16x16x32_bf16, both operands read with ds_read_b64_tr_b16 (each lane gets eight rows of one
  // column of x, or of one rank of l), then one 16-byte store per lane into the workspace ([rank][k]: lane
  // l holds columns 4 (l / 16) .. + 3 of rank l % 16).  Every stage runs this and stores (out of range when
  // the stage is not this wave's, the chunk loop then running no iteration): a store under a condition, in
  // each unrolled stage, made the register allocator spill the accumulators.  The store follows the
  // stage's copies, so the next stage's wait leaves it in flight; the prologue issues one too (db_none), so
  // that exactly one store follows every stage's copies.
  __device__ __forceinline__ void db_sum(const GemmArgs& p, const bf16* slot, int kt, int lane) const {
    if constexpr (DB) {
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const bool mine = db_step(kt);
      const int nch = mine ? (mrows_ + 31) >> 5 : 0;  // at most BM / 32 + 1 (a tall item's extra rows)
      f32x4 c0 = f32x4{}, c1 = f32x4{};
      // two chunks per iteration into two accumulators; the addresses are formed inside the loop from the
      // lane index taken afresh (opaque), so that stages that sum nothing spend nothing on them
      for (int ch0 = 0; ch0 < nch; ch0 += 2) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int G = ln >> 4, sl = ln & 15, col = (wave_ & 3) * 16 + 4 * (sl & 3);
        bf16x8 a[2], b[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int ch = min(ch0 + u, nch - 1);  // (a chunk past nch: read, not summed)
          const bf16* xt = ch < BM / 32 ? slot : slot + SlotSize<NRB, WT, true>::kXOff;
          const int xr = (ch < BM / 32 ? ch * 32 : 0) + 8 * G + (sl >> 2);
          const int lr = ch * 32 + 8 * G + (sl >> 2);
          const s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)(xt + swz_rk(xr, col >> 3) + (col & 7)));
          const s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)(xt + swz_rk(xr + 4, col >> 3) + (col & 7)));
          const s16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)(dbt_ + lr * 16 + 4 * (sl & 3)));
          const s16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_void*)(dbt_ + (lr + 4) * 16 + 4 * (sl & 3)));
          a[u] = __builtin_bit_cast(bf16x8, (s16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]}));
          b[u] = __builtin_bit_cast(bf16x8, (s16x8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]}));
        }
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], c0, 0, 0, 0);
        if (ch0 + 1 < nch) c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], c1, 0, 0, 0);
      }
      c0 += c1;
      const int k = kt * BK + (wave_ & 3) * 16 + 4 * (lane >> 4);  // K is a multiple of 8: four columns all in or all out
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, c0), rdbw,
                                             mine && k < p.K ? (uint32_t)(((lane & 15) * p.K + k) * 4) : kOob, 0, 0);
    }
  }
  __device__ __forceinline__ void db_none() const {  // the prologue's store: out of range, no effect
    if constexpr (DB) __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rdbw, kOob, 0, 0);
  }
};

// the stack's fragment for MFMA (32 columns n at nb, 8 consecutive k at kb + 8*(lane/32))
template <bool BKC, int WT = kWBf16>
__device__ __forceinline__ bf16x8 w_frag(const bf16* bs, int nb, int kk, int lane) {
  if constexpr (WT == kWFp8K) {
    // as kWFp8, each value then multiplied by its k's scale in fp32 and rounded once to bf16
    const int n = nb + (lane & 31);
    const u32x2 v = *(const u32x2*)((const uint8_t*)bs + n * BK + ((kk ^ swz_q<WT>(n)) << 4) + 8 * (lane >> 5));
    const float* sc = (const float*)((const uint8_t*)bs + WTile<WT>::Bytes) + kk * 16 + 8 * (lane >> 5);
    const f32x4 s0 = *(const f32x4*)sc, s1 = *(const f32x4*)(sc + 4);
    const unsigned d[4] = {__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.f, false)),
                           __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.f, true)),
                           __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.f, false)),
                           __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.f, true))};
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16_bits_to_f32(d[i] & 0xFFFFu), b = bf16_bits_to_f32(d[i] >> 16);
      const float sa = i < 2 ? s0[2 * i] : s1[2 * i - 4], sb = i < 2 ? s0[2 * i + 1] : s1[2 * i - 3];
      w[i] = pack_bf16x2(a * sa, b * sb);
    }
    typedef unsigned u32x4_ __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8, (u32x4_{w[0], w[1], w[2], w[3]}));
  } else if constexpr (WT == kWFp8) {
    // eight e4m3 bytes of row n (16-byte chunk kk, half lane/32), converted exactly to bf16
    const int n = nb + (lane & 31);
    const u32x2 v = *(const u32x2*)((const uint8_t*)bs + n * BK + ((kk ^ swz_q<WT>(n)) << 4) + 8 * (lane >> 5));
    typedef unsigned u32x4_ __attribute__((ext_vector_type(4)));
    const u32x4_ w = {__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.f, false)),
                      __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[0], 1.f, true)),
                      __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.f, false)),
                      __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[1], 1.f, true))};
    return __builtin_bit_cast(bf16x8, w);
  } else if constexpr (BKC) {
    return *(const bf16x8*)(bs + swz_rk(nb + (lane & 31), kk * 2 + (lane >> 5)));
  } else {
    // ds_read_b64_tr_b16: in each group of 16 lanes, source lane s points at (k0 + s/4, n0 + 4*(s%4))
    // and lane i receives the four values (k0 .. k0+3, n0 + i)
    const int g = lane >> 4, s = lane & 15;
    const int n = nb + 16 * (g & 1) + 4 * (s & 3);
    const int k = kk * 16 + 8 * (g >> 1) + (s >> 2);
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const bf16* p0 = bs + swz_kn(k, n >> 3) + (n & 7);
    const bf16* p1 = bs + swz_kn(k + 4, n >> 3) + (n & 7);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(lds_void*)p0);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(lds_void*)p1);
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  }
}

// ---- NF4 ----
// A stage is one 64-k block of every stack row, so a lane needs one absmax per column block per
// stage: absmax = code2[q] · absmax2 + offset (rounded after the product and after the sum, as the
// standalone dequantiser), with q and absmax2 loaded a stage ahead.  From it the lane builds its
// table of the sixteen decoded values bf16(code[c] · absmax), kept as a low-byte and a high-byte
// plane (four dwords each), and decodes eight nibbles with byte permutes: four values per lookup.
struct Nf4Pipe {
  int64_t blk[FN];  // the block index of this lane's column j at k = 0, or -1 past N
  uint32_t q[FN];
  float a2[FN];
  uint32_t pl[4][4];  // kWNf4T: byte p of code[4m .. 4m+3] in pl[p][m]
  __device__ __forceinline__ void planes(const float* code) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f32x4 c = *(const f32x4*)(code + 4 * m);
      const uint32_t b0 = __float_as_uint(c[0]), b1 = __float_as_uint(c[1]), b2 = __float_as_uint(c[2]),
                     b3 = __float_as_uint(c[3]);
      const uint32_t l01 = __builtin_amdgcn_perm(b1, b0, 0x05010400u), h01 = __builtin_amdgcn_perm(b1, b0, 0x07030602u);
      const uint32_t l23 = __builtin_amdgcn_perm(b3, b2, 0x05010400u), h23 = __builtin_amdgcn_perm(b3, b2, 0x07030602u);
      pl[0][m] = __builtin_amdgcn_perm(l23, l01, 0x05040100u);  // bytes 0 of entries 4m .. 4m+3
      pl[1][m] = __builtin_amdgcn_perm(l23, l01, 0x07060302u);
      pl[2][m] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
      pl[3][m] = __builtin_amdgcn_perm(h23, h01, 0x07060302u);
    }
  }
  template <bool SWI>
  __device__ __forceinline__ void init(const GemmArgs& p, int e, int n0, int wn, int lane) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = tile_col<SWI>(p, n0, (j * WAVES_N + wn) * 32 + (lane & 31));
      blk[j] = n < p.N ? ((int64_t)e * p.w_se + (int64_t)n * p.w_sn) >> 6 : -1;
    }
  }
  __device__ __forceinline__ void load(const GemmArgs& p, int kt) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const bool ok = blk[j] >= 0 && kt * BK < p.K;
      const int64_t b = blk[j] + kt;
      q[j] = ok ? p.nf4_q[b] : 0u;
      a2[j] = ok ? p.nf4_absmax2[b >> 8] : 0.f;
    }
  }
};

__device__ __forceinline__ float nf4_absmax(float c2, float a2, float off) {
#pragma clang fp contract(off)
  return c2 * a2 + off;
}

// the decoded values of one block: lo[m] / hi[m] hold the low / high bytes of entries 4m .. 4m+3
__device__ __forceinline__ void nf4_table(const float* code, float absmax, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x4 c = *(const f32x4*)(code + 4 * m);
    const uint32_t p0 = pack_bf16x2(c[0] * absmax, c[1] * absmax), p1 = pack_bf16x2(c[2] * absmax, c[3] * absmax);
    lo[m] = __builtin_amdgcn_perm(p1, p0, 0x06040200u);
    hi[m] = __builtin_amdgcn_perm(p1, p0, 0x07050301u);
  }
}

// four byte-sized indices (0..15) -> their entries' low and high bytes
__device__ __forceinline__ void nf4_look(uint32_t g, const uint32_t (&lo)[4], const uint32_t (&hi)[4], uint32_t& lb,
                                         uint32_t& hb) {
  const uint32_t sel = g & 0x07070707u;
  // 0xFF in the bytes whose index is 8 or more (permute selector 13), 0x00 elsewhere (selector 12)
  const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((g >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
  lb = __builtin_amdgcn_perm(lo[1], lo[0], sel);
  hb = __builtin_amdgcn_perm(hi[1], hi[0], sel);
  lb = (__builtin_amdgcn_perm(lo[3], lo[2], sel) & m) | (lb & ~m);
  hb = (__builtin_amdgcn_perm(hi[3], hi[2], sel) & m) | (hb & ~m);
}

// four byte-sized indices (0..15) -> the four fp32 codes they name, from the code's byte planes
__device__ __forceinline__ void nf4_code4(uint32_t g, const uint32_t (&pl)[4][4], float (&f)[4]) {
  const uint32_t sel = g & 0x07070707u;
  const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((g >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
  uint32_t t[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    t[b] = (__builtin_amdgcn_perm(pl[b][3], pl[b][2], sel) & m) | (__builtin_amdgcn_perm(pl[b][1], pl[b][0], sel) & ~m);
  // t[b] holds byte b of the four codes; gather each code's four bytes
  const uint32_t l01 = __builtin_amdgcn_perm(t[1], t[0], 0x05010400u), h01 = __builtin_amdgcn_perm(t[1], t[0], 0x07030602u);
  const uint32_t l23 = __builtin_amdgcn_perm(t[3], t[2], 0x05010400u), h23 = __builtin_amdgcn_perm(t[3], t[2], 0x07030602u);
  f[0] = __uint_as_float(__builtin_amdgcn_perm(l23, l01, 0x05040100u));
  f[1] = __uint_as_float(__builtin_amdgcn_perm(l23, l01, 0x07060302u));
  f[2] = __uint_as_float(__builtin_amdgcn_perm(h23, h01, 0x05040100u));
  f[3] = __uint_as_float(__builtin_amdgcn_perm(h23, h01, 0x07060302u));
}

// eight NF4 codes with one absmax per value (a0: values 0-3, a1: 4-7) -> eight bf16(code · absmax)
__device__ __forceinline__ bf16x8 nf4t_decode(uint32_t x, const uint32_t (&pl)[4][4], f32x4 a0, f32x4 a1) {
  float fe[4], fo[4];
  nf4_code4((x >> 4) & 0x0F0F0F0Fu, pl, fe);  // elements 0, 2, 4, 6
  nf4_code4(x & 0x0F0F0F0Fu, pl, fo);         // elements 1, 3, 5, 7
  typedef unsigned u32x4_ __attribute__((ext_vector_type(4)));
  const u32x4_ w = {pack_bf16x2(fe[0] * a0[0], fo[0] * a0[1]), pack_bf16x2(fe[1] * a0[2], fo[1] * a0[3]),
                    pack_bf16x2(fe[2] * a1[0], fo[2] * a1[1]), pack_bf16x2(fe[3] * a1[2], fo[3] * a1[3])};
  return __builtin_bit_cast(bf16x8, w);
}

// eight NF4 codes (byte j: element 2j in the high nibble, 2j+1 in the low) -> eight bf16
__device__ __forceinline__ bf16x8 nf4_decode(uint32_t x, const uint32_t (&lo)[4], const uint32_t (&hi)[4]) {
  uint32_t el, eh, ol, oh;
  nf4_look((x >> 4) & 0x0F0F0F0Fu, lo, hi, el, eh);  // elements 0, 2, 4, 6
  nf4_look(x & 0x0F0F0F0Fu, lo, hi, ol, oh);         // elements 1, 3, 5, 7
  const uint32_t e02 = __builtin_amdgcn_perm(eh, el, 0x05010400u), e46 = __builtin_amdgcn_perm(eh, el, 0x07030602u);
  const uint32_t o13 = __builtin_amdgcn_perm(oh, ol, 0x05010400u), o57 = __builtin_amdgcn_perm(oh, ol, 0x07030602u);
  typedef unsigned u32x4_ __attribute__((ext_vector_type(4)));
  const u32x4_ w = {__builtin_amdgcn_perm(o13, e02, 0x05040100u), __builtin_amdgcn_perm(o13, e02, 0x07060302u),
                    __builtin_amdgcn_perm(o57, e46, 0x05040100u), __builtin_amdgcn_perm(o57, e46, 0x07060302u)};
  return __builtin_bit_cast(bf16x8, w);
}

// The MFMAs of one stage held in `slot` for a wave with AM live row blocks.
// The copies of the next stage (into nslot) are issued in three parts after the first MFMA steps:
// issued back to back they fill the texture unit's queues and hold the wave in front of its MFMAs.
// TL: a tall item (BM + up to XR rows): one more MFMA per step into tacc, the extra rows x this wave's
// column block wm (and their x A_e in tlacc, by waves (0, 0) and (0, 1), one 16-row half each)
template <int AM, bool BKC, int NRB, int WT, bool TL, class F>
__device__ __forceinline__ void compute(const GemmArgs& p, const bf16* slot, int lane0, int wm, int wn,
                                        f32x16 (&acc)[FM][FN], f32x4 (&lacc)[kLS][NRB > 0 ? NRB : 1],
                                        f32x16& tacc, f32x4 (&tlacc)[NRB > 0 ? NRB : 1],
                                        Nf4Pipe& nf, const float* code, float off, int kt,
                                        const F& f, bf16* nslot, int nkt) {
  // With the fused adapter gradient, a tall item's stages take the lane index afresh (opaque): the LDS
  // addresses of the fragments are formed in the stage that reads them, not hoisted out of the K loop
  // into registers held through it (the gradient's state then spills the tall accumulators).  Elsewhere
  // the hoisted addresses are faster (4 % of the product).
  int lane = lane0;
  if constexpr (F::kDB && TL) asm volatile("" : "+v"(lane));
  static_assert(!TL || (AM == FM && FN == 2 && WAVES_M == 2 && WAVES_N >= 2), "tall items: 2 x 4 waves, full row blocks");
  constexpr int kXOff = SlotSize<NRB, WT, true>::kXOff;
  const bf16* as = slot;
  const bf16* bs = slot + BM * BK;
  uint32_t tlo[WT == kWNf4 ? FN : 1][4], thi[WT == kWNf4 ? FN : 1][4];
  if constexpr (WT == kWNf4) {  // this stage's tables, then the next stage's block scales
#pragma unroll
    for (int j = 0; j < FN; ++j) nf4_table(code, nf4_absmax(code[16 + nf.q[j]], nf.a2[j], off), tlo[j], thi[j]);
    nf.load(p, kt + 1);
  }
  // With two slots every wait is for all of a wave's copies, so the stage past the end of K is not
  // queued at all (the four-slot ring queues zero-filled copies to keep its wait counts constant)
  const bool queue = STAGES != 2 || nkt * BK < p.K;
  if constexpr (AM == 0) {
    if (queue) f.issue(p, nslot, nkt);
  }
  if constexpr (AM > 0) {
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      auto read_a = [&](int i) -> bf16x8 {
        return *(const bf16x8*)(as + swz_rk((i * WAVES_M + wm) * 32 + (lane & 31), kk * 2 + (lane >> 5)));
      };
      auto read_b = [&](int j) -> bf16x8 {
        if constexpr (WT == kWNf4T) {
          const int n = (j * WAVES_N + wn) * 32 + (lane & 31);
          const uint32_t x = *(const uint32_t*)((const uint8_t*)bs + n * (BK / 2) +
                                                (((kk >> 1) ^ swz_q<WT>(n)) << 4) + (kk & 1) * 8 + 4 * (lane >> 5));
          const float* a = (const float*)((const uint8_t*)bs + WTile<WT>::Bytes) + (n >> 6) * BK + kk * 16 + 8 * (lane >> 5);
          return nf4t_decode(x, nf.pl, *(const f32x4*)a, *(const f32x4*)(a + 4));
        } else if constexpr (WT == kWNf4) {
          // eight codes: byte 8kk/2 + 4(lane/32) of row n (16-byte chunk kk/2)
          const int n = (j * WAVES_N + wn) * 32 + (lane & 31);
          const uint32_t x = *(const uint32_t*)((const uint8_t*)bs + n * (BK / 2) +
                                                (((kk >> 1) ^ swz_q<WT>(n)) << 4) + (kk & 1) * 8 + 4 * (lane >> 5));
          return nf4_decode(x, tlo[j], thi[j]);
        } else {
          return w_frag<BKC, WT>(bs, (j * WAVES_N + wn) * 32, kk, lane);
        }
      };
      // the reads in the order the MFMAs consume them (LDS returns them in order): the first MFMA
      // waits for two fragments, each later one for at most one more
      bf16x8 af[AM], bfr[FN];
      bfr[0] = read_b(0);
      af[0] = read_a(0);
#pragma unroll
      for (int j = 1; j < FN; ++j) bfr[j] = read_b(j);
#pragma unroll
      for (int i = 1; i < AM; ++i) af[i] = read_a(i);
      // the step's MFMAs at raised wave priority: of the two waves on a SIMD, the one with MFMAs ready
      // wins the issue slot over the other's LDS reads and copies (-0.85 % product time)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < AM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
      if constexpr (TL) {
        const bf16x8 at = *(const bf16x8*)(slot + kXOff + swz_rk(lane & 31, kk * 2 + (lane >> 5)));
        tacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wm == 0 ? bfr[0] : bfr[1], at, tacc, 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
      constexpr int last = BK / 16 - 1;
      if (kk <= 2 || kk == last) __builtin_amdgcn_sched_barrier(0);
      if (queue) {
        if (kk == 0) f.template issue_part<0>(p, nslot, nkt);
        if (kk == 1 || (kk == last && last < 1)) f.template issue_part<1>(p, nslot, nkt);
        if (kk == 2 || (kk == last && last < 2)) f.template issue_part<2>(p, nslot, nkt);
      }
      if (kk <= 2 || kk == last) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NRB > 0) {
      const bf16* aa = slot + BM * BK + WTile<WT>::Elems;
#pragma unroll
      for (int ls = 0; ls < BK / 32; ++ls) {
        bf16x8 ar[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) ar[rb] = *(const bf16x8*)(aa + swz_rk(rb * 16 + (lane & 15), ls * 4 + (lane >> 4)));
#pragma unroll
        for (int q = 0; q < kLS; ++q) {
          const int sh = wn + WAVES_N * q;  // this wave's 16-row half: block sh / 2, half sh % 2
          if ((sh >> 1) < AM) {
            const int rbase = ((sh >> 1) * WAVES_M + wm) * 32 + (sh & 1) * 16;
            const bf16x8 xf = *(const bf16x8*)(as + swz_rk(rbase + (lane & 15), ls * 4 + (lane >> 4)));
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
              lacc[q][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, ar[rb], lacc[q][rb], 0, 0, 0);
          }
        }
        if constexpr (TL) {
          if (wm == 0 && wn < 2) {
            const bf16x8 xf = *(const bf16x8*)(slot + kXOff + swz_rk(wn * 16 + (lane & 15), ls * 4 + (lane >> 4)));
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
              tlacc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, ar[rb], tlacc[rb], 0, 0, 0);
          }
        }
      }
    }
  }
  if constexpr (F::kDB) {
    f.db_sum(p, slot, kt, lane);
  }
}

// One iteration of the K loop: wait for this wave's copies of stage kt (slot S), publish every
// wave's with a barrier, queue stage kt + STAGES - 1 into the slot read one iteration ago, multiply.
template <int S, int AM, bool BKC, int NRB, int WT, bool TL, class F>
__device__ __forceinline__ void stage(const GemmArgs& p, const F& f, bf16* const (&slots)[STAGES], int kt,
                                      int lane, int wm, int wn, f32x16 (&acc)[FM][FN],
                                      f32x4 (&lacc)[kLS][NRB > 0 ? NRB : 1], f32x16& tacc,
                                      f32x4 (&tlacc)[NRB > 0 ? NRB : 1], Nf4Pipe& nf, const float* code, float off) {
  // (stages kt+1, kt+2 may stay in flight; with the fused adapter gradient, the previous stage's store
  // of its partial sums, issued after every copy, too)
  wait_vm<F::PS * (STAGES - 2) + (F::kDB ? 1 : 0)>();
  stage_barrier();
  compute<AM, BKC, NRB, WT, TL>(p, slots[S], lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off, kt, f,
                                slots[(S + STAGES - 1) % STAGES], kt + STAGES - 1);
}

// The K loop of one item, unrolled by the ring depth so every slot index is a constant.
template <int AM, bool BKC, int NRB, int WT, bool TL = false, class F>
__device__ __forceinline__ void kloop(const GemmArgs& p, const F& f, bf16* const (&slots)[STAGES], int nk,
                                      int lane, int wm, int wn, f32x16 (&acc)[FM][FN],
                                      f32x4 (&lacc)[kLS][NRB > 0 ? NRB : 1], f32x16& tacc,
                                      f32x4 (&tlacc)[NRB > 0 ? NRB : 1], Nf4Pipe& nf, const float* code, float off) {
  int kt = 0;
  if constexpr (STAGES == 4) {
    for (; kt + STAGES <= nk; kt += STAGES) {
      stage<0, AM, BKC, NRB, WT, TL>(p, f, slots, kt, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
      stage<1, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 1, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
      stage<2, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 2, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
      stage<3, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 3, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
    }
    const int rem = nk - kt;  // 0 .. 3 stages left
    if (rem > 0) stage<0, AM, BKC, NRB, WT, TL>(p, f, slots, kt, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
    if (rem > 1) stage<1, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 1, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
    if (rem > 2) stage<2, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 2, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
  } else {
    for (; kt + 2 <= nk; kt += 2) {
      stage<0, AM, BKC, NRB, WT, TL>(p, f, slots, kt, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
      stage<1, AM, BKC, NRB, WT, TL>(p, f, slots, kt + 1, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
    }
    if (kt < nk) stage<0, AM, BKC, NRB, WT, TL>(p, f, slots, kt, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
  }
}

// One 32 x 32 block of bf16 results (rows rbase .., columns col ..) from the MFMA layout: lane l holds
// columns 8g + 4(l/32) .. +3 of row l % 32 in v[g], g = 0..3.  One swap of the lanes' halves per pair of
// groups gives lane l < 32 columns 0-7 (x) and 16-23 (y) of row l, lane l + 32 columns 8-15 and 24-31; in
// 16-lane rows, x = [r0-15 c0-7, r16-31 c0-7, r0-15 c8-15, r16-31 c8-15] and y likewise for c16-31.  A
// 32-lane swap then a 16-lane swap regroup them into a = [c0-7, c8-15, c16-23, c24-31] of rows 0-15 and b
// the same of rows 16-31: each store writes 64 contiguous bytes of 16 rows.  Rows past the resource's
// range are dropped by it; columns from ncols on are not stored.
__device__ __forceinline__ void store_block32(const u32x2 (&v)[4], rsrc_t r, int rbase, int64_t ld, int col,
                                              int ncols, int lane) {
  u32x2 pk[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const auto sw = __builtin_amdgcn_permlane32_swap(pk[2 * h][d], pk[2 * h + 1][d], false, false);
      pk[2 * h][d] = sw[0];
      pk[2 * h + 1][d] = sw[1];
    }
  uint32_t xa[4] = {pk[0][0], pk[0][1], pk[1][0], pk[1][1]}, yb[4] = {pk[2][0], pk[2][1], pk[3][0], pk[3][1]};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const auto s1 = __builtin_amdgcn_permlane32_swap(xa[q], yb[q], false, false);
    const auto s2 = __builtin_amdgcn_permlane16_swap(s1[0], s1[1], false, false);
    xa[q] = s2[0];
    yb[q] = s2[1];
  }
  const int n = col + 8 * (lane >> 4);
  const uint32_t o = (uint32_t)((rbase + (lane & 15)) * ld * 2) + (uint32_t)n * 2;
  if (n < ncols) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{xa[0], xa[1], xa[2], xa[3]}, r, o, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{yb[0], yb[1], yb[2], yb[3]}, r, o + (uint32_t)(16 * ld * 2), 0, 0);
  }
}

// SwiGLU of two packed bf16 gate values and their up values, as mlora_swiglu computes each one
__device__ __forceinline__ uint32_t swiglu_bf16x2(uint32_t g2, uint32_t u2) {
  const float g0 = bf16_bits_to_f32(g2 & 0xFFFFu), g1 = bf16_bits_to_f32(g2 >> 16);
  const float u0 = bf16_bits_to_f32(u2 & 0xFFFFu), u1 = bf16_bits_to_f32(u2 >> 16);
  return pack_bf16x2(g0 * sigmoidf_(g0) * u0, g1 * sigmoidf_(g1) * u1);
}

template <bool BKC, int NRB, int WT, bool TALL = false, bool DB = false, bool SWI = false>
__global__ __launch_bounds__(kThreads, MLORA_DMA_OCC) void grouped_gemm_bf16_kernel(GemmArgs p) {
  constexpr int RP = NRB * 16;
  constexpr int LP = RP + 8;
  constexpr int SE = SlotSize<NRB, WT, TALL>::kElems;
  constexpr int BMT = BM + (TALL ? XR : 0);  // the most rows an item holds
  static_assert(BMT * LP <= SE && BN * LP + (STAGES == 4 ? 0 : BN * 3) <= SE,
                "the epilogue's low, B^T, column-scale and bias tiles fit in the slots they reuse");
  __shared__ __attribute__((aligned(16))) bf16 slot0[SE];
  __shared__ __attribute__((aligned(16))) bf16 slot1[SE];
#if MLORA_DMA_STAGES == 4
  __shared__ __attribute__((aligned(16))) bf16 slot2[SE];
  __shared__ __attribute__((aligned(16))) bf16 slot3[SE];
  bf16* const slots[STAGES] = {slot0, slot1, slot2, slot3};
#else
  bf16* const slots[STAGES] = {slot0, slot1};
#endif
  extern __shared__ __attribute__((aligned(16))) int tile_map[];
  const int tid0 = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid0 >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int E = p.E;

  bf16* Ls = slot0;  // epilogue: [BM][LP] and [BN][LP], in slots the ring has finished with
  bf16* Lb = slot1;
  // With one 16-rank block, B_e^T's tile (BN rows of 32 bytes) is copied by DMA at the start of each
  // item into an LDS region of its own, so the epilogue waits on no load for it.  The two 16-byte
  // halves of row n sit swapped when bit 2 of n is set: the epilogue's 16-byte reads of 32
  // consecutive rows then spread over the banks.
  constexpr bool kPreB = NRB == 1;
  __shared__ __attribute__((aligned(16))) bf16 lbt[kPreB ? BN * 16 : 8];
  // DB: l of the item's rows, [BM + XR][16] (the summed operand of the fused adapter gradient)
  __shared__ __attribute__((aligned(16))) bf16 dbt[DB ? (BM + XR) * 16 : 8];

  // the small-tile counts after the tile map (experts up to kSmallLastE), then the NF4 code book (16)
  // and absmax code book (256)
  const bool small_last = E <= kSmallLastE;
  int* sfx = tile_map + ((E + 3) & ~3);
  float* code = (float*)(sfx + (small_last ? ((E + 3) & ~3) : 0));
  float off = 0.f;
  if constexpr (WT == kWNf4) {
    for (int c = tid0; c < 16 + 256; c += kThreads) code[c] = c < 16 ? p.nf4_code[c] : p.nf4_code2[c - 16];
    off = p.nf4_offset[0];
  }
  if constexpr (WT == kWNf4T) {
    for (int c = tid0; c < 16; c += kThreads) code[c] = p.nf4_code[c];
  }
  build_tile_ends(p, tile_map, sfx, small_last, TALL, TALL && !DB, tid0);
  const int nb = (p.N + BN - 1) / BN;
  // each XCD takes one contiguous eighth of the full tiles' items, then one eighth of the small tiles'
  const int64_t nbig = (int64_t)__builtin_amdgcn_readfirstlane(tile_map[E - 1]) * nb;
  const int64_t nsmall = small_last ? (int64_t)__builtin_amdgcn_readfirstlane(sfx[E - 1]) * nb : 0;
  const int xcd = blockIdx.x % kXcds, wg_slot = blockIdx.x / kXcds, per_xcd = gridDim.x / kXcds;
  const int64_t cbig = (nbig + kXcds - 1) / kXcds, csmall = (nsmall + kXcds - 1) / kXcds;
  const int64_t bbeg = min(xcd * cbig, nbig), bcnt = min(bbeg + cbig, nbig) - bbeg;
  const int64_t sbeg = min(xcd * csmall, nsmall), scnt = min(sbeg + csmall, nsmall) - sbeg;
  const int nk = (p.K + BK - 1) / BK;

  for (int64_t j = wg_slot; j < bcnt + scnt; j += per_xcd) {
    const bool small = j >= bcnt;
    int64_t item = small ? sbeg + (j - bcnt) : bbeg + j;
    if (!small && nb > kGroupNb) item = grouped_item(item, nbig / nb, nb);
    // the thread index taken afresh for every item: values derived from it are computed where they
    // are used, not hoisted out of this loop to hold registers through every K loop and epilogue
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const Item it = decode(p, item, nb, tile_map, sfx, small, TALL, TALL && !DB);
    const int e = it.e, n0 = it.n0, mrows = it.mrows;
    const int64_t row0 = it.row0;
    const int ncols = min(BN, p.N - n0);
    const int mb = (mrows + 31) >> 5, nbk = (ncols + 31) >> 5;
    const int am = min(FM, max(0, (mb - wm + WAVES_M - 1) / WAVES_M));
    const int an = min(FN, max(0, (nbk - wn + WAVES_N - 1) / WAVES_N));

    Feed<BKC, NRB, WT, TALL, DB, SWI> f;
    f.rx = p.gather == nullptr ? make_rsrc(p.x + row0 * p.ldx, (int64_t)mrows * p.ldx * 2)
                               : make_rsrc(p.x, p.xrows * p.ldx * 2);
    {
      const int64_t ebytes = WT == kWBf16 ? p.w_se * 2 : WTile<WT>::kFp8 ? p.w_se : p.w_se / 2;  // one expert's stack
      f.rw = make_rsrc(p.w + (int64_t)e * ebytes, ebytes);
      if constexpr (WT == kWFp8K) f.rs = make_rsrc(p.scale + (int64_t)e * p.scale_se, (int64_t)p.K * 4);
      if constexpr (WT == kWNf4T)  // the expert's absmax table (N / 64, K)
        f.rs = make_rsrc(p.nf4_absmax2 + (int64_t)e * (p.N / 64) * p.K, (int64_t)(p.N / 64) * p.K * 4);
    }
    f.ra = f.rx;
    if constexpr (NRB > 0) f.ra = make_rsrc(p.at + (int64_t)e * p.at_se, (int64_t)RP * p.at_sr * 2);
    f.init(p, n0, row0, mrows, wave, lane);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
    f32x4 lacc[kLS][NRB > 0 ? NRB : 1];
#pragma unroll
    for (int q = 0; q < kLS; ++q)
#pragma unroll
      for (int j = 0; j < (NRB > 0 ? NRB : 1); ++j) lacc[q][j] = f32x4{};
    f32x16 tacc = f32x16{};  // a tall item's extra rows x column block wm * WAVES_N + wn
    f32x4 tlacc[NRB > 0 ? NRB : 1];
#pragma unroll
    for (int j = 0; j < (NRB > 0 ? NRB : 1); ++j) tlacc[j] = f32x4{};
    const bool tall = TALL && mrows > BM;

    Nf4Pipe nf;
    if constexpr (WT == kWNf4T) nf.planes(code);  // (the tile map's barrier published the code book)
    if constexpr (WT == kWNf4) {
      nf.template init<SWI>(p, e, n0, wn, lane);
      nf.load(p, 0);
    }
    __syncthreads();  // the previous item's epilogue is done with the LDS
    if constexpr (kPreB) {  // one 16-byte chunk per thread: row tid / 2, half (tid & 1) ^ bit 2 of the row
      static_assert(BN * 2 <= kThreads, "one chunk of the B^T tile per thread");
      if (p.scaling != 0.f && tid < BN * 2) {
        const rsrc_t rbt = make_rsrc(p.bt + (int64_t)e * p.bt_se, (int64_t)p.N * p.bt_sn * 2);
        const int row = tid >> 1, half = (tid & 1) ^ ((row >> 2) & 1), n = tile_col<SWI>(p, n0, row);
        dma16(rbt, lbt + (tid >> 6) * 512, n < p.N ? (uint32_t)((n * p.bt_sn + half * 8) * 2) : kOob);
      }
    }
    if constexpr (DB) {
      // l of the tile's rows into LDS by DMA, [row][16] (row r's 32 bytes are chunks 2r, 2r + 1, lane-linear:
      // nine copies of 64 chunks); rows past the item read out of range (zeros).  They land with the first
      // stage's copies.
      const rsrc_t rl = make_rsrc(p.dbl + row0 * p.dbl_ld, (int64_t)mrows * p.dbl_ld * 2);
      for (int q = wave; q < (BM + XR) * 2 / 64; q += NW) {
        const int c = q * 64 + lane, r = c >> 1;
        dma16(rl, dbt + q * 512, (uint32_t)((r * p.dbl_ld + (c & 1) * 8) * 2));
      }
      f.dbt_ = dbt;
      f.nb_ = nb;
      f.nblk_ = it.nblk;
      f.db_next_ = it.nblk;
      f.db_j_ = 0;
      f.mrows_ = mrows;
      // the tile's slot: expert e's tiles start at row row_start(e) + j BM, so e + row0 / BM is one per tile
      f.rdbw = make_rsrc(p.dbw + (e + row0 / BM) * 16 * (int64_t)p.K, (int64_t)16 * p.K * 4);
    }
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) f.issue(p, slots[s], s);
    f.db_none();

    switch (am) {
      case FM:
        if constexpr (TALL) {
          if (tall) {
            kloop<FM, BKC, NRB, WT, true>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
            break;
          }
        }
        kloop<FM, BKC, NRB, WT>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off);
        break;
#if (256 / MLORA_DMA_WM / 32) >= 4
      case 3: kloop<3, BKC, NRB, WT>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off); break;
#endif
#if (256 / MLORA_DMA_WM / 32) >= 3
      case 2: kloop<2, BKC, NRB, WT>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off); break;
#endif
#if (256 / MLORA_DMA_WM / 32) >= 2
      case 1: kloop<1, BKC, NRB, WT>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off); break;
#endif
      default: kloop<0, BKC, NRB, WT>(p, f, slots, nk, lane, wm, wn, acc, lacc, tacc, tlacc, nf, code, off); break;
    }
    wait_vm<0>();     // (four slots) the zero-filled copies queued past the end of K
    __syncthreads();  // every wave is done with the ring (all copies waited for in the loop)

    // ---- epilogue ----
    // Everything the stores need is read first: the adapters' tiles, the per-column stack scales and
    // the bias into LDS, the row scales into registers.  A vector-memory load issued after the first
    // output store would wait for every store before it (one in-order counter covers both), so the
    // stores run back to back with nothing but LDS reads between them.
    const int col_l = 4 * (lane >> 5);
    // [BN] per-column stack scale (MLORA_SCALE_ROW) and [BN] bias: after B^T, or in the third slot
    float* Lc = (float*)(STAGES == 4 ? slots[STAGES - 2] : Lb + BN * LP);
    bf16* Lbias = (bf16*)(Lc + BN);      // [BN] bias
    const bool col_scale = p.scale_kind == MLORA_SCALE_ROW && WT != kWFp8K, has_bias = p.bias != nullptr;
    const float cexp = p.scale_kind == MLORA_SCALE_EXPERT ? p.scale[e] : 1.f;
    if (tid < BN && (col_scale || has_bias)) {
      const int n = tile_col<SWI>(p, n0, tid);
      if (col_scale) Lc[tid] = n < p.N ? p.scale[(int64_t)e * p.scale_se + n] : 0.f;
      if (has_bias) Lbias[tid] = n < p.N ? p.bias[(int64_t)e * p.bias_se + n] : (bf16)0.f;
    }
    float rs[FM];  // each row's output scale (the combine weight of a gathered gradient row)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = (i * WAVES_M + wm) * 32 + (lane & 31);
      rs[i] = 1.f;
      if (p.row_scale != nullptr && i < am && row < mrows) {
        const int64_t si = p.gather[row0 + row];
        rs[i] = p.row_scale_dt == MLORA_DT_F32 ? ((const float*)p.row_scale)[si] : (float)((const bf16*)p.row_scale)[si];
      }
    }
    float rs_t = 1.f;  // the tall rows' output scale
    if constexpr (TALL) {
      if (tall && p.row_scale != nullptr && BM + (lane & 31) < mrows) {
        const int64_t si = p.gather[row0 + BM + (lane & 31)];
        rs_t = p.row_scale_dt == MLORA_DT_F32 ? ((const float*)p.row_scale)[si] : (float)((const bf16*)p.row_scale)[si];
      }
    }
    if constexpr (NRB > 0) {
#pragma unroll
      for (int q = 0; q < kLS; ++q) {
        const int sh = wn + WAVES_N * q;
        const int rbase = ((sh >> 1) * WAVES_M + wm) * 32 + (sh & 1) * 16;
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            Ls[(rbase + 4 * (lane >> 4) + v) * LP + rb * 16 + (lane & 15)] = (bf16)lacc[q][rb][v];
      }
      if constexpr (TALL) {
        if (tall && wm == 0 && wn < 2) {
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              Ls[(BM + wn * 16 + 4 * (lane >> 4) + v) * LP + rb * 16 + (lane & 15)] = (bf16)tlacc[rb][v];
        }
      }
      if constexpr (!kPreB) {
        const rsrc_t rbt = make_rsrc(p.bt + (int64_t)e * p.bt_se, (int64_t)p.N * p.bt_sn * 2);
        for (int c = tid; c < BN * RP / 8; c += kThreads) {
          const int nn = c / (RP / 8), rc = (c - nn * (RP / 8)) * 8;
          const int n = tile_col<SWI>(p, n0, nn);
          *(u32x4*)(Lb + nn * LP + rc) = ld128(rbt, n < p.N ? (uint32_t)((n * p.bt_sn + rc) * 2) : kOob);
        }
      }
    }
    __syncthreads();
    wait_vm<0>();  // the row scales (and every other load) are in before the first store
    if constexpr (NRB > 0) {
      if (p.low != nullptr && it.nblk == 0) {
        for (int c = tid; c < BMT * RP / 8; c += kThreads) {
          const int m = c / (RP / 8), rc = (c - m * (RP / 8)) * 8;
          if (m < mrows) *(u32x4*)(p.low + (row0 + m) * p.ldl + rc) = *(const u32x4*)(Ls + m * LP + rc);
        }
      }
    }
    const bool lora_on = NRB > 0 && p.scaling != 0.f;
    const bool plain = !col_scale && cexp == 1.f && p.row_scale == nullptr && !has_bias;
    // the item's rows of out through a buffer resource: 32-bit offsets, stores past its rows dropped
    const rsrc_t ro = make_rsrc(p.out + row0 * p.ldo, (int64_t)mrows * p.ldo * 2);
    // SwiGLU fused: act's rows of the item; wave wn's column blocks j = 0, 1 are gate columns
    // n0 / 2 + 32 wn .. and their up columns, giving act's columns n0 / 2 + 32 wn ..
    static_assert(!SWI || (kSwiOn && !DB), "the fused SwiGLU pairs blocks j = 0, 1 and takes no fused gradient");
    constexpr bool swi = SWI;
    const rsrc_t ra = make_rsrc(swi ? p.act + row0 * p.lda : p.out, swi ? (int64_t)mrows * p.lda * 2 : 0);
    const int acol = (n0 >> 1) + wn * 32;
    // a tall item's extra rows: wave (1, wn) holds the up block of wave (0, wn)'s gate block and hands
    // its values over here ([WAVES_N][64 lanes][8 dwords], past the column-scale and bias tiles)
    uint32_t* const xch = (uint32_t*)(Lb + BN * LP + BN * 4);
    (void)xch;
    (void)acol;
    static_assert(!TALL || BN * LP + BN * 4 + WAVES_N * 64 * 8 * 2 <= SE, "the tall rows' hand-over fits in its slot");
    // the output blocks: row block i (rows (i * WAVES_M + wm) * 32 ..) x column block j * WAVES_N + wn,
    // and for a tall item one more, i = FM: its extra rows x column block wm * WAVES_N + wn
#pragma unroll
    for (int i = 0; i < FM + (TALL ? 1 : 0); ++i) {
      const bool tb = TALL && i == FM;
      if (tb ? !tall : i >= am) continue;
      const int rbase = tb ? BM : (i * WAVES_M + wm) * 32;
      u32x2 pg[4];  // SwiGLU fused: the gate block's values, before the swaps
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if (j >= an || (tb && j != wm)) continue;
        const f32x16& av = tb ? tacc : acc[i < FM ? i : 0][j];
        const float rsv = tb ? rs_t : rs[i < FM ? i : 0];
        f32x16 t = f32x16{};
        if constexpr (NRB > 0) {
          if (lora_on) {
#pragma unroll
            for (int rk = 0; rk < NRB; ++rk) {
              const bf16x8 lf = *(const bf16x8*)(Ls + (rbase + (lane & 31)) * LP + rk * 16 + (lane >> 5) * 8);
              const int nr = (j * WAVES_N + wn) * 32 + (lane & 31);
              const bf16x8 bfr = kPreB ? *(const bf16x8*)(lbt + nr * 16 + (((lane >> 5) ^ ((nr >> 2) & 1)) << 3))
                                       : *(const bf16x8*)(Lb + nr * LP + rk * 16 + (lane >> 5) * 8);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr, lf, t, 0, 0, 0);
            }
          }
        }
        // lane l holds columns 8g + 4(l/32) .. +3 of row l % 32 in pk[g], g = 0..3
        u32x2 pk[4];
        if (plain) {  // no stack scale, row scale or bias: one fma per value
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = __builtin_fmaf(p.scaling, t[4 * g + q], av[4 * g + q]);
            pk[g] = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int nn = (j * WAVES_N + wn) * 32 + 8 * g + col_l;  // column within the tile
            f32x4 c = {cexp, cexp, cexp, cexp}, bias = {0.f, 0.f, 0.f, 0.f};
            if (col_scale) c = *(const f32x4*)(Lc + nn);
            if (has_bias) {
              const u32x2 b2 = *(const u32x2*)(Lbias + nn);
              bias = f32x4{bf16_bits_to_f32(b2[0] & 0xFFFFu), bf16_bits_to_f32(b2[0] >> 16),
                           bf16_bits_to_f32(b2[1] & 0xFFFFu), bf16_bits_to_f32(b2[1] >> 16)};
            }
            float o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
              o[q] = (av[4 * g + q] * c[q] + p.scaling * t[4 * g + q]) * rsv + bias[q];
            pk[g] = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          }
        }
        if constexpr (swi) {
          if (j == 0) {
#pragma unroll
            for (int g = 0; g < 4; ++g) pg[g] = pk[g];
          } else if (!tb) {
            u32x2 pa[4];
#pragma unroll
            for (int g = 0; g < 4; ++g)
              pa[g] = u32x2{swiglu_bf16x2(pg[g][0], pk[g][0]), swiglu_bf16x2(pg[g][1], pk[g][1])};
            store_block32(pa, ra, rbase, p.lda, acol, p.swi, lane);
          } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) *(u32x2*)(xch + (wn * 64 + lane) * 8 + 2 * g) = pk[g];
          }
        }
        store_block32(pk, ro, rbase, p.ldo, tile_col<SWI>(p, n0, (j * WAVES_N + wn) * 32), p.N, lane);
      }
      if constexpr (TALL && swi) {
        if (tb) {  // every wave is here (a tall item): the up blocks handed over, then act
          __syncthreads();
          if (wm == 0) {
            u32x2 pa[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const u32x2 pu = *(const u32x2*)(xch + (wn * 64 + lane) * 8 + 2 * g);
              pa[g] = u32x2{swiglu_bf16x2(pg[g][0], pu[0]), swiglu_bf16x2(pg[g][1], pu[1])};
            }
            store_block32(pa, ra, rbase, p.lda, acol, p.swi, lane);
          }
        }
      }
    }
  }
}

static size_t lds_bytes(int E, int WT) {
  const size_t ea = (size_t)((E + 3) & ~3);
  return ea * sizeof(int) * (E <= kSmallLastE ? 2 : 1) + (WT == kWNf4 ? 272 * 4 : WT == kWNf4T ? 16 * 4 : 0);
}
static_assert(BM * (kMaxRank + 8) <= SlotSize<4>::kElems &&
                  BN * (kMaxRank + 8) + (STAGES == 4 ? 0 : BN * 3) <= SlotSize<4>::kElems,
              "the epilogue's low, B^T, column-scale and bias tiles must fit in the slots they reuse");
static_assert(STAGES * SlotSize<4>::kElems * 2 + 4096 * 4 <= 163840, "the slots and the largest tile map fit in LDS");
static_assert(STAGES * SlotSize<4, kWNf4>::kElems * 2 + 4096 * 4 + 272 * 4 <= 163840, "the same with the NF4 code books");
static_assert(STAGES * SlotSize<4, kWNf4T>::kElems * 2 + 4096 * 4 + 16 * 4 <= 163840, "the same with the absmax tiles");
static_assert(STAGES * SlotSize<4>::kElems * 2 + kSmallLastE * 8 <= 163840, "the small-tile counts fit beside the slots");
static_assert(STAGES * SlotSize<1>::kElems * 2 + BN * 16 * 2 + 4096 * 4 <= 163840,
              "with one rank block: the slots, the B^T tile and the largest tile map fit in LDS");
static_assert(WTile<kWNf4>::RowBytes * 2 == 64, "an NF4 stage is one block of 64 codes per row");

// tall items: bf16 and fp8 stacks, rank 16 or none, two-slot ring, and a tile map small enough to sit beside
// the larger slots (the small-tile counts included)
static_assert(STAGES * SlotSize<1, kWBf16, true>::kElems * 2 + BN * 16 * 2 + kSmallLastE * 8 <= 163840 &&
                  STAGES * SlotSize<1, kWFp8K, true>::kElems * 2 + BN * 16 * 2 + kSmallLastE * 8 <= 163840,
              "tall items: the slots, the B^T tile and the tile map fit in LDS");
template <bool BKC, int NRB, int WT>
constexpr bool kTallOn = STAGES == 2 && (WT == kWBf16 || WT == kWFp8 || WT == kWFp8K) && NRB <= 1 && WAVES_M == 2 &&
                         WAVES_N >= 2 && FN == 2;  // (NF4 stacks: the tall block's registers spill its K loop)

// The fused adapter gradient: at most kDbMaxE experts, so that the slots, the B^T tile, l's tile and the
// tile map fit in LDS together
constexpr int kDbMaxE = 256;
static_assert(STAGES * SlotSize<1, kWBf16, true>::kElems * 2 + BN * 16 * 2 + (BM + XR) * 16 * 2 + kDbMaxE * 8 <= 163840,
              "with the fused adapter gradient: the slots, the B^T tile, l's tile and the tile map fit in LDS");

// The fused adapter gradient's last step: out[e, k, r] = bf16(scaling · sum over expert e's tiles of the
// partial sums [slot][r][k]), the tiles added in row order (deterministic).  The tiles are counted as the
// product counts them: xr = XR when a remainder of at most XR rows joined the expert's last full tile.
__global__ __launch_bounds__(256) void db_finish_kernel(const float* __restrict__ ws, const int32_t* __restrict__ offsets,
                                                        int64_t rows, int E, int K, int xr, float scaling,
                                                        bf16* __restrict__ out, int64_t o_se, int64_t o_sk,
                                                        int64_t o_sr) {
  const int e = blockIdx.y;
  auto start = [&](int x) -> int64_t {
    if (x == 0) return 0;
    const int64_t o = offsets[x - 1];
    return o < 0 ? 0 : (o > rows ? rows : o);
  };
  const int64_t es = start(e), c = start(e + 1) - es;
  int nt = c > 0 ? (int)((c + BM - 1) / BM) : 0;
  if (nt >= 2 && c - (int64_t)(nt - 1) * BM <= xr) --nt;
  const int64_t s0 = e + es / BM;
  for (int i = threadIdx.x; i < 16 * 256; i += 256) {
    const int r = i >> 8, k = blockIdx.x * 256 + (i & 255);
    if (k >= K) continue;
    float sum = 0.f;
    for (int t = 0; t < nt; ++t) sum += ws[((s0 + t) * 16 + r) * K + k];
    out[(int64_t)e * o_se + (int64_t)k * o_sk + (int64_t)r * o_sr] = (bf16)(sum * scaling);
  }
}

template <bool BKC, int NRB, int WT, bool TALL = false, bool DB = false, bool SWI = false>
static int launch_t(const GemmArgs& a, hipStream_t s) {
  if constexpr (kTallOn<BKC, NRB, WT> && !TALL) {
    if (a.E <= kSmallLastE) return launch_t<BKC, NRB, WT, true, DB, SWI>(a, s);
  }
  auto kern = grouped_gemm_bf16_kernel<BKC, NRB, WT, TALL, DB, SWI>;
  const size_t lds = lds_bytes(a.E, WT);
  static std::mutex mu;
  static std::unordered_map<int64_t, int> grid_cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail("grouped_gemm: hipGetDevice failed");
  int grid = 0;
  {
    std::lock_guard<std::mutex> g(mu);
    const int64_t key = ((int64_t)dev << 32) | (int64_t)lds;
    auto it = grid_cache.find(key);
    if (it != grid_cache.end()) {
      grid = it->second;
    } else {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail("grouped_gemm: cannot grant %zu bytes of LDS", lds);
      int cus = 0, per_cu = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return fail("grouped_gemm: cannot read the compute unit count");
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kern, kThreads, lds) != hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      grid = (cus * per_cu + kXcds - 1) / kXcds * kXcds;
      grid_cache[key] = grid;
    }
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, s, a);
  if constexpr (DB) {
    if (int rc = launch_status("grouped_gemm")) return rc;
    hipLaunchKernelGGL(db_finish_kernel, dim3((unsigned)((a.K + 255) / 256), (unsigned)a.E), dim3(256), 0, s, a.dbw,
                       a.offsets, a.rows, a.E, a.K, TALL ? XR : 0, a.scaling, a.dbo, a.dbo_se, a.dbo_sk, a.dbo_sr);
    return launch_status("grouped_gemm/adapter gradient");
  }
  return launch_status("grouped_gemm");
}

template <bool BKC, int WT>
static int launch_r(const GemmArgs& a, hipStream_t s) {
  if (a.swi != 0) {  // the fused SwiGLU: forward stacks (bf16, fp8, NF4 either way), rank 16 or no adapters
    if constexpr (kSwiOn && WT != kWFp8K) {
      if (a.rank == 0) return launch_t<BKC, 0, WT, false, false, true>(a, s);
      if (a.rank == 16) return launch_t<BKC, 1, WT, false, false, true>(a, s);
    }
    return fail("grouped_gemm_swiglu: the fused SwiGLU takes bf16, fp8 or NF4 stacks with adapters of rank 16 or none");
  }
  switch (a.rank / 16) {
    case 0: return launch_t<BKC, 0, WT>(a, s);
    case 1: return launch_t<BKC, 1, WT>(a, s);
    case 2: return launch_t<BKC, 2, WT>(a, s);
    case 3: return launch_t<BKC, 3, WT>(a, s);
    default: return launch_t<BKC, 4, WT>(a, s);
  }
}

}  // namespace dma

int launch_grouped_gemm_bf16(const GemmArgs& a, bool k_contiguous, hipStream_t s) {
  if (a.scale_kind == MLORA_SCALE_ROW && a.scale_se == 0) return fail("grouped_gemm: per-row scale without a stride");
  if (a.dbl != nullptr) {  // with the fused adapter gradient: rank 16, at most kDbMaxE experts (checked at the ABI)
    if (a.rank != 16 || a.E > dma::kDbMaxE) return fail("grouped_gemm: the fused adapter gradient needs rank 16 and <= %d experts", dma::kDbMaxE);
    return k_contiguous ? dma::launch_t<true, 1, dma::kWBf16, false, true>(a, s)
                        : dma::launch_t<false, 1, dma::kWBf16, false, true>(a, s);
  }
  return k_contiguous ? dma::launch_r<true, dma::kWBf16>(a, s) : dma::launch_r<false, dma::kWBf16>(a, s);
}

int64_t grouped_gemm_db_slots(int64_t rows, int E) { return E + rows / dma::BM + 1; }
int grouped_gemm_db_max_experts() { return dma::kDbMaxE; }
bool grouped_gemm_swiglu_fits() { return dma::kSwiOn; }

bool grouped_gemm_dma_takes(const GemmArgs& a, int w_dtype, bool k_contiguous, bool scale_on_k) {
  // fp8 and NF4 stacks: k contiguous (each row copied as stored), rows of whole 16-byte chunks, a
  // stack scale per expert or per output row (a scale along k stays with the register-staged kernel)
  if (!k_contiguous) return false;
  if (w_dtype == MLORA_DT_FP8_E4M3)
    return a.w_sn % 16 == 0 && a.w_se % 16 == 0 && ((uintptr_t)a.w & 15u) == 0 &&
           (!scale_on_k || (a.scale_kind == MLORA_SCALE_ROW && a.scale_se % 4 == 0 && ((uintptr_t)a.scale & 15u) == 0));
  if (scale_on_k) return false;
  if (w_dtype == MLORA_DT_NF4 || w_dtype == MLORA_DT_NF4_KT)  // rows of whole 64-code blocks, 16-byte aligned packing
    return a.w_sn % 64 == 0 && a.w_se % 64 == 0 && ((uintptr_t)a.w & 15u) == 0 &&
           (w_dtype == MLORA_DT_NF4 || a.N % 64 == 0);
  return false;
}

int launch_grouped_gemm_dma_q(const GemmArgs& a, int w_dtype, bool scale_on_k, hipStream_t s) {
  if (a.scale_kind == MLORA_SCALE_ROW && a.scale_se == 0) return fail("grouped_gemm: per-row scale without a stride");
  if (w_dtype == MLORA_DT_FP8_E4M3 && scale_on_k) return dma::launch_r<true, dma::kWFp8K>(a, s);
  if (w_dtype == MLORA_DT_FP8_E4M3) return dma::launch_r<true, dma::kWFp8>(a, s);
  if (w_dtype == MLORA_DT_NF4) return dma::launch_r<true, dma::kWNf4>(a, s);
  if (w_dtype == MLORA_DT_NF4_KT) return dma::launch_r<true, dma::kWNf4T>(a, s);
  return fail("grouped_gemm: stack dtype %d has no DMA-fed product", w_dtype);
}

}  // namespace mlora
