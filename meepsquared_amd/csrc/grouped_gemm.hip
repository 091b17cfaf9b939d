// The grouped product of the experts with the rank-r LoRA fused in, for gfx950 (CDNA4) MFMA.
//
//   out_e = c · x_e W_e + scaling · bf16(x_e A_e) B_e + bias_e         for every expert e
//
// x's rows are sorted by expert; offsets[e] is the end of expert e's rows.  Each expert's rows are
// cut into BM-row tiles (no tile spans two experts) and a work item is one (tile, BN-column block).
// The kernel is persistent: the grid is a fixed number of workgroups per compute unit and each
// workgroup derives the tile map itself, from offsets, in LDS (no tile arrays, no host round
// trip).  Items are split into 8 contiguous ranges, one per XCD (the hardware deals workgroup b to
// XCD b % 8), so that the workgroups running together on one XCD work on neighbouring tiles of
// the same expert and share its weight tiles and x tiles in that XCD's L2.
//
// Main loop: BK-deep stages double-buffered in LDS.  x tiles (BM x BK) and weight tiles (BN x BK)
// are held in LDS as [row][k] bf16 with k contiguous, whatever the stack's layout:
//   * a stack whose k axis is contiguous is copied 8 k-values at a time;
//   * a stack whose n axis is contiguous (the input-gradient pass of an (E, out, in) stack) is
//     loaded as 4(k) x 8(n) blocks and transposed in registers (v_perm_b32) on the way to LDS;
//   * fp8 e4m3 and NF4 stacks are decoded to bf16 in registers between the global load and the
//     LDS store, with a per-output-row scale folded in when it runs along k.
// Global loads go through buffer resources (32-bit offsets; reads past a resource's end return
// zero), which bounds every tile at the end of x and of each expert's weights.
// Each of the 4 waves owns a 64 x 64 corner of the 128 x 128 tile: 2 x 2 v_mfma_f32_32x32x16_bf16
// accumulators.  The LoRA's x·A_e (BM x R, R a multiple of 16) is accumulated in the same loop
// from the same LDS x tile with v_mfma_f32_16x16x32_bf16, each wave taking 32 of the rows, so x is
// read from HBM once for both products.  The epilogue rounds x·A_e to bf16 (as the reference
// does), optionally stores it ("low", kept for the backward pass), and adds scaling · low · B_e
// with one more MFMA of depth R, then the scale and the bias.
//
// Reference behaviour: src/meepsquared/_grouped.py:120-221 (_grouped_gemm_kernel), :313-345 (_launch).
#include <mutex>
#include <unordered_map>

#include "gemm_common.hpp"

namespace mlora {

// Tile shape: a workgroup computes BM x BN of the output with WAVES_M x WAVES_N waves; OCC is the
// number of waves per SIMD the register budget is sized for.  (Compile-time; the defaults are the
// shape measured fastest on the config-1 products.)
#ifndef MLORA_BM
#define MLORA_BM 256
#endif
#ifndef MLORA_BN
#define MLORA_BN 256
#endif
#ifndef MLORA_WAVES_M
#define MLORA_WAVES_M 2
#endif
#ifndef MLORA_WAVES_N
#define MLORA_WAVES_N 2
#endif
#ifndef MLORA_OCC
#define MLORA_OCC 1
#endif
constexpr int BM = MLORA_BM, BN = MLORA_BN, BK = 64;
constexpr int WAVES_M = MLORA_WAVES_M, WAVES_N = MLORA_WAVES_N;
constexpr int kThreads = 64 * WAVES_M * WAVES_N;
constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;  // each wave's share of the tile
constexpr int FM = WTM / 32, FN = WTN / 32;            // its 32 x 32 MFMA blocks
static_assert(FM >= 1 && FN >= 1 && (2 * FM) % WAVES_N == 0, "tile shape");
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// 8 fp8 (element 0 in the lowest byte) -> 8 bf16, each times s (exact when s == 1)
__device__ __forceinline__ u32x4 fp8x8_to_bf16(u32x2 v, float s) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = v[i >> 1] >> (16 * (i & 1));
    r[i] = pack_bf16x2(fp8_e4m3_to_f32(d & 0xFFu) * s, fp8_e4m3_to_f32((d >> 8) & 0xFFu) * s);
  }
  return r;
}
__device__ __forceinline__ u32x4 fp8x8_to_bf16_scaled(u32x2 v, const float* s) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = v[i >> 1] >> (16 * (i & 1));
    r[i] = pack_bf16x2(fp8_e4m3_to_f32(d & 0xFFu) * s[2 * i], fp8_e4m3_to_f32((d >> 8) & 0xFFu) * s[2 * i + 1]);
  }
  return r;
}
// 8 NF4 codes in 4 bytes (byte j: element 2j in the high nibble, 2j+1 in the low) -> 8 bf16 · absmax
__device__ __forceinline__ u32x4 nf4x8_to_bf16(uint32_t v, float absmax, const float* code) {
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t byte = (v >> (8 * j)) & 0xFFu;
    r[j] = pack_bf16x2(code[byte >> 4] * absmax, code[byte & 0xFu] * absmax);
  }
  return r;
}
// a block's absmax: code2[q] * absmax2 + offset, rounded after the product and after the sum (no fma)
__device__ __forceinline__ float nf4_block_absmax(const GemmArgs& p, int64_t block) {
#pragma clang fp contract(off)
  return p.nf4_code2[p.nf4_q[block]] * p.nf4_absmax2[block >> 8] + p.nf4_offset[0];
}

// Byte offset of a stack element (NF4: two per byte).
template <int WDT>
__device__ __forceinline__ uint32_t w_bytes(int64_t el) {
  if constexpr (WDT == W_BF16) return (uint32_t)(el * 2);
  else if constexpr (WDT == W_FP8) return (uint32_t)el;
  else return (uint32_t)(el >> 1);
}

// LDS tiles are [row][k] with rows of BK = 64 bf16 (128 bytes) and no padding; the 16-byte chunk c of
// row r sits in slot c ^ ((r >> 1) & 7).  An MFMA operand read serves 16 lanes on 16 consecutive rows
// at one chunk per cycle: two rows share each 256-byte bank line, and the XOR gives the 16 reads 16
// distinct 16-byte bank groups; the stage writes (8 lanes per row) stay conflict-free as well.
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 1) & 7)) << 3); }

// One BK-deep stage: the global loads land in registers (issued a stage ahead) and are decoded
// into LDS after the current stage's MFMAs.
template <int WDT, bool BKC, bool SCALE_K, int NRB>
struct Stage {
  static constexpr int kXChunks = BM * BK / 8;                                // 16-byte chunks of x per stage
  static constexpr int kXPer = (kXChunks + kThreads - 1) / kThreads;
  static constexpr int kWUnits = BKC ? BN * BK / 8 : (BK / 4) * (BN / 8);       // W chunks, or 4(k) x 8(n) blocks
  static constexpr int kWPer = (kWUnits + kThreads - 1) / kThreads;
  static constexpr int kWVec = BKC ? kWPer : kWPer * 4;                         // W vectors per thread
  static constexpr int kAChunks = NRB * 16 * BK / 8;                                      // A^T chunks per stage
  static constexpr int kAPer = (kAChunks + kThreads - 1) / kThreads;
  u32x4 x[kXPer];
  u32x4 w16[kWVec];
  u32x2 w8[kWVec];
  uint32_t w4[kWVec];
  float ws[BKC && SCALE_K ? kWVec * 8 : kWVec];
  u32x4 a[kAPer > 0 ? kAPer : 1];

  __device__ __forceinline__ void load(const GemmArgs& p, rsrc_t rx, rsrc_t rw, rsrc_t ra, int e, int n0, int k0,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int c = tid + i * kThreads;
      const int rr = c >> 3, k = k0 + (c & 7) * 8;
      if (c < kXChunks) x[i] = ld128(rx, k < p.K ? (uint32_t)((rr * p.ldx + k) * 2) : kOob);
    }
    if constexpr (BKC) {
#pragma unroll
      for (int i = 0; i < kWPer; ++i) {
        const int c = tid + i * kThreads;
        const int n = n0 + (c >> 3), k = k0 + (c & 7) * 8;
        const bool ok = c < kWUnits && n < p.N && k < p.K;
        const int64_t el = (int64_t)n * p.w_sn + k;
        const uint32_t off = ok ? w_bytes<WDT>(el) : kOob;
        if constexpr (WDT == W_BF16) {
          w16[i] = ld128(rw, off);
        } else if constexpr (WDT == W_FP8) {
          w8[i] = ld64(rw, off);
          if constexpr (SCALE_K) {
#pragma unroll
            for (int q = 0; q < 8; ++q) ws[i * 8 + q] = ok ? p.scale[(int64_t)e * p.scale_se + k + q] : 0.f;
          }
        } else {
          w4[i] = ld32(rw, off);
          ws[i] = ok ? nf4_block_absmax(p, ((int64_t)e * p.w_se + el) >> 6) : 0.f;
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < kWPer; ++b) {
        const int blk = tid + b * kThreads;
        const int kb = blk & 15, n = n0 + (blk >> 4) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int k = k0 + kb * 4 + q;
          const bool ok = blk < kWUnits && n < p.N && k < p.K;
          const int64_t el = (int64_t)k * p.w_sk + n;
          const uint32_t off = ok ? w_bytes<WDT>(el) : kOob;
          const int v = b * 4 + q;
          if constexpr (WDT == W_BF16) {
            w16[v] = ld128(rw, off);
          } else if constexpr (WDT == W_FP8) {
            w8[v] = ld64(rw, off);
            if constexpr (SCALE_K) ws[v] = ok ? p.scale[(int64_t)e * p.scale_se + k] : 0.f;
          } else {
            w4[v] = ld32(rw, off);
            ws[v] = ok ? nf4_block_absmax(p, ((int64_t)e * p.w_se + el) >> 6) : 0.f;
          }
        }
      }
    }
    if constexpr (NRB > 0) {
#pragma unroll
      for (int i = 0; i < kAPer; ++i) {
        const int c = tid + i * kThreads;
        const int r = c >> 3, k = k0 + (c & 7) * 8;
        if (c < kAChunks) a[i] = ld128(ra, k < p.K ? (uint32_t)((r * p.at_sr + k) * 2) : kOob);
      }
    }
  }

  __device__ __forceinline__ void store(bf16* As, bf16* Bs, bf16* Aa, const float* code, int tid) const {
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
      const int c = tid + i * kThreads;
      if (c < kXChunks) *(u32x4*)(As + swz(c >> 3, c & 7)) = x[i];
    }
    if constexpr (BKC) {
#pragma unroll
      for (int i = 0; i < kWPer; ++i) {
        const int c = tid + i * kThreads;
        if (c >= kWUnits) continue;
        u32x4 v;
        if constexpr (WDT == W_BF16) v = w16[i];
        else if constexpr (WDT == W_FP8) v = SCALE_K ? fp8x8_to_bf16_scaled(w8[i], ws + i * 8) : fp8x8_to_bf16(w8[i], 1.0f);
        else v = nf4x8_to_bf16(w4[i], ws[i], code);
        *(u32x4*)(Bs + swz(c >> 3, c & 7)) = v;
      }
    } else {
#pragma unroll
      for (int b = 0; b < kWPer; ++b) {
        const int blk = tid + b * kThreads;
        if (blk >= kWUnits) continue;
        const int kb = blk & 15, nb8 = blk >> 4;
        u32x4 row[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int v = b * 4 + q;
          if constexpr (WDT == W_BF16) row[q] = w16[v];
          else if constexpr (WDT == W_FP8) row[q] = fp8x8_to_bf16(w8[v], SCALE_K ? ws[v] : 1.0f);
          else row[q] = nf4x8_to_bf16(w4[v], ws[v], code);
        }
        // transpose 4 (k) x 8 (n) into 8 rows (n) of 4 k: 8 bytes at k = kb*4, in chunk kb/2
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          u32x2 ev, od;
          ev[0] = lo_pair(row[0][m], row[1][m]);
          ev[1] = lo_pair(row[2][m], row[3][m]);
          od[0] = hi_pair(row[0][m], row[1][m]);
          od[1] = hi_pair(row[2][m], row[3][m]);
          const int n_ev = nb8 * 8 + 2 * m, n_od = n_ev + 1;
          *(u32x2*)(Bs + swz(n_ev, kb >> 1) + (kb & 1) * 4) = ev;
          *(u32x2*)(Bs + swz(n_od, kb >> 1) + (kb & 1) * 4) = od;
        }
      }
    }
    if constexpr (NRB > 0) {
#pragma unroll
      for (int i = 0; i < kAPer; ++i) {
        const int c = tid + i * kThreads;
        if (c < kAChunks) *(u32x4*)(Aa + swz(c >> 3, c & 7)) = a[i];
      }
    }
  }
};

constexpr int kLS = 2 * FM / WAVES_N;  // 16-row halves of x·A_e per wave

// The K loop of one work item for a wave with AM live row blocks (of FM): every MFMA of the loop
// is unconditional, so the compiler can interleave operand reads, MFMAs and the next stage's loads.
template <int AM, int WDT, bool BKC, bool SCALE_K, int NRB>
__device__ __forceinline__ void kloop(const GemmArgs& p, Stage<WDT, BKC, SCALE_K, NRB>& st, rsrc_t rx, rsrc_t rw,
                                      rsrc_t ra, int e, int n0, int nk, bf16* As, bf16* Bs, bf16* Aa,
                                      const float* code, int tid, int lane, int wm, int wn, f32x16 (&acc)[FM][FN],
                                      f32x4 (&lacc)[kLS][NRB > 0 ? NRB : 1]) {
  constexpr int RP = NRB * 16;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) st.load(p, rx, rw, ra, e, n0, (kt + 1) * BK, tid);
    const bf16* as = As + buf * BM * BK;
    const bf16* bs = Bs + buf * BN * BK;
    if constexpr (AM > 0) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8 af[AM], bfr[FN];
        const int ch = kk * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < AM; ++i) af[i] = *(const bf16x8*)(as + swz((i * WAVES_M + wm) * 32 + (lane & 31), ch));
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[j] = *(const bf16x8*)(bs + swz((j * WAVES_N + wn) * 32 + (lane & 31), ch));
#pragma unroll
        for (int i = 0; i < AM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
      }
      if constexpr (NRB > 0) {
        const bf16* aa = Aa + buf * RP * BK;
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
          const int ch = kk * 4 + (lane >> 4);
          bf16x8 af[NRB];
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb) af[rb] = *(const bf16x8*)(aa + swz(rb * 16 + (lane & 15), ch));
#pragma unroll
          for (int q = 0; q < kLS; ++q) {
            const int sh = wn + WAVES_N * q;  // this wave's 16-row half: block sh / 2, half sh % 2
            if ((sh >> 1) < AM) {  // wn is wave-uniform: a scalar branch around whole MFMA groups
              const int rbase = ((sh >> 1) * WAVES_M + wm) * 32 + (sh & 1) * 16;
              const bf16x8 xf = *(const bf16x8*)(as + swz(rbase + (lane & 15), ch));
#pragma unroll
              for (int rb = 0; rb < NRB; ++rb)
                lacc[q][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, af[rb], lacc[q][rb], 0, 0, 0);
            }
          }
        }
      }
    }
    if (kt + 1 < nk) st.store(As + (buf ^ 1) * BM * BK, Bs + (buf ^ 1) * BN * BK, Aa + (buf ^ 1) * RP * BK, code, tid);
    __syncthreads();
  }
}

// NRB = rank / 16 (0: no adapters).  Wave (wm, wn) owns the 32-row blocks i*WAVES_M + wm and the
// 32-column blocks j*WAVES_N + wn of the tile (interleaved, so a tile cut short by the end of an
// expert's rows still spreads its rows over every wave); blocks past the expert's last row or
// past N are skipped, MFMAs included.
template <int WDT, bool BKC, bool SCALE_K, int NRB>
__global__ __launch_bounds__(kThreads, MLORA_OCC) void grouped_gemm_kernel(GemmArgs p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int RP = NRB * 16;
  constexpr int LP = RP + 8;  // pitch of the epilogue's low and B^T tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int E = p.E;

  bf16* As = (bf16*)smem;                    // [2][BM][BK] swizzled
  bf16* Bs = As + 2 * BM * BK;               // [2][BN][BK] swizzled
  bf16* Aa = Bs + 2 * BN * BK;               // [2][RP][BK] swizzled
  int* starts = (int*)(Aa + 2 * RP * BK);    // E + 1
  int* tstart = starts + (E + 1);            // E + 1
  float* code = (float*)(tstart + (E + 1));  // 16 (NF4 code book)
  bf16* Ls = As;                             // epilogue: [BM][LP], aliasing the x stages
  bf16* Lb = Bs;                             // epilogue: [BN][LP], aliasing the W stages

  // ---- the tile map, from offsets ----
  // row starts clamped into [0, rows]: offsets past the end of x (a caller's mistake) cannot send a
  // tile outside x or out
  for (int e = tid; e <= E; e += kThreads) {
    const int64_t o = e == 0 ? 0 : (int64_t)p.offsets[e - 1];
    starts[e] = (int)(o < 0 ? 0 : (o > p.rows ? p.rows : o));
  }
  if constexpr (WDT == W_NF4) {
    if (tid < 16) code[tid] = p.nf4_code[tid];
  }
  __syncthreads();
  for (int e = tid; e < E; e += kThreads) {
    const int c = max(starts[e + 1] - starts[e], 0);
    tstart[e] = (c + BM - 1) / BM;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of tstart[0..E), 64 at a time
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
  const int nb = (p.N + BN - 1) / BN;
  const int64_t total = (int64_t)__builtin_amdgcn_readfirstlane(tstart[E]) * nb;
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds, per_xcd = gridDim.x / kXcds;
  const int64_t chunk = (total + kXcds - 1) / kXcds;
  const int64_t beg = xcd * chunk, end = min(beg + chunk, total);
  const int nk = (p.K + BK - 1) / BK;

  for (int64_t item = beg + slot; item < end; item += per_xcd) {
    const int t = (int)(item / nb), nblk = (int)(item - (int64_t)t * nb);
    int lo = 0, hi = E - 1;  // the expert e with tstart[e] <= t < tstart[e+1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tstart[mid] <= t) lo = mid; else hi = mid - 1;
    }
    // values read from LDS are per-lane to the compiler: make the tile's scalars wave-uniform (SGPRs)
    const int e = __builtin_amdgcn_readfirstlane(lo);
    const int e_start = __builtin_amdgcn_readfirstlane(starts[e]);
    const int e_end = __builtin_amdgcn_readfirstlane(starts[e + 1]);
    const int e_t0 = __builtin_amdgcn_readfirstlane(tstart[e]);
    const int64_t row0 = (int64_t)e_start + (int64_t)(t - e_t0) * BM;
    const int mrows = (int)min((int64_t)BM, (int64_t)e_end - row0);
    const int n0 = nblk * BN;
    const int ncols = min(BN, p.N - n0);
    // this wave's live blocks: a prefix of its interleaved row and column blocks
    const int mb = (mrows + 31) >> 5, nbk = (ncols + 31) >> 5;
    const int am = min(FM, max(0, (mb - wm + WAVES_M - 1) / WAVES_M));
    const int an = min(FN, max(0, (nbk - wn + WAVES_N - 1) / WAVES_N));

    // resources: the tile's own rows of x (rows past the expert read as zero); W, A^T of expert e
    const rsrc_t rx = make_rsrc(p.x + row0 * p.ldx, (int64_t)mrows * p.ldx * 2);
    const int64_t we = (int64_t)e * p.w_se;
    const rsrc_t rw = WDT == W_BF16 ? make_rsrc(p.w + we * 2, p.w_se * 2)
                    : WDT == W_FP8  ? make_rsrc(p.w + we, p.w_se)
                                    : make_rsrc(p.w + (we >> 1), p.w_se >> 1);
    rsrc_t ra = rx;
    if constexpr (NRB > 0) ra = make_rsrc(p.at + (int64_t)e * p.at_se, (int64_t)RP * p.at_sr * 2);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
    // x·A_e: the 16-row halves s = 0 .. 2*FM-1 of this wave-row's blocks (block s/2, half s%2) are
    // shared among its WAVES_N waves: this wave takes s = wn + WAVES_N*q
    f32x4 lacc[kLS][NRB > 0 ? NRB : 1];
#pragma unroll
    for (int q = 0; q < kLS; ++q)
#pragma unroll
      for (int j = 0; j < (NRB > 0 ? NRB : 1); ++j) lacc[q][j] = f32x4{};

    Stage<WDT, BKC, SCALE_K, NRB> st;
    __syncthreads();  // the previous item's epilogue is done with the LDS
    st.load(p, rx, rw, ra, e, n0, 0, tid);
    st.store(As, Bs, Aa, code, tid);
    __syncthreads();

    switch (am) {  // the K loop, specialised on this wave's live row blocks: no branches inside
      case FM: kloop<FM, WDT, BKC, SCALE_K, NRB>(p, st, rx, rw, ra, e, n0, nk, As, Bs, Aa, code, tid, lane, wm, wn, acc, lacc); break;
#if MLORA_BM / MLORA_WAVES_M / 32 >= 4
      case 3: kloop<3, WDT, BKC, SCALE_K, NRB>(p, st, rx, rw, ra, e, n0, nk, As, Bs, Aa, code, tid, lane, wm, wn, acc, lacc); break;
#endif
#if MLORA_BM / MLORA_WAVES_M / 32 >= 3
      case 2: kloop<2, WDT, BKC, SCALE_K, NRB>(p, st, rx, rw, ra, e, n0, nk, As, Bs, Aa, code, tid, lane, wm, wn, acc, lacc); break;
#endif
#if MLORA_BM / MLORA_WAVES_M / 32 >= 2
      case 1: kloop<1, WDT, BKC, SCALE_K, NRB>(p, st, rx, rw, ra, e, n0, nk, As, Bs, Aa, code, tid, lane, wm, wn, acc, lacc); break;
#endif
      default: kloop<0, WDT, BKC, SCALE_K, NRB>(p, st, rx, rw, ra, e, n0, nk, As, Bs, Aa, code, tid, lane, wm, wn, acc, lacc); break;
    }

    // ---- epilogue ----
    // acc[i][j] holds out^T of the 32 x 32 block (i, j): lane l has the tile row (i*WAVES_M + wm)*32 + l%32
    // and, for value v, the column (j*WAVES_N + wn)*32 + 8*(v/4) + 4*(l/32) + v%4: four runs of four.
    const int col_l = 4 * (lane >> 5);
    f32x4 cs[FN][4];  // the base product's scale per column
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (p.scale_kind == MLORA_SCALE_EXPERT) {
          const float c = p.scale[e];
          cs[j][g] = f32x4{c, c, c, c};
        } else if (p.scale_kind == MLORA_SCALE_ROW && !SCALE_K) {
          const int n = n0 + (j * WAVES_N + wn) * 32 + 8 * g + col_l;
          cs[j][g] = n < p.N ? *(const f32x4*)(p.scale + (int64_t)e * p.scale_se + n) : f32x4{};
        } else {
          cs[j][g] = f32x4{1.f, 1.f, 1.f, 1.f};
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
      // B_e^T rows n0 .. n0+BN: Lb[n][r]
      const rsrc_t rbt = make_rsrc(p.bt + (int64_t)e * p.bt_se, (int64_t)p.N * p.bt_sn * 2);
      for (int c = tid; c < BN * RP / 8; c += kThreads) {
        const int nn = c / (RP / 8), rc = (c - nn * (RP / 8)) * 8;
        const int n = n0 + nn;
        *(u32x4*)(Lb + nn * LP + rc) = ld128(rbt, n < p.N ? (uint32_t)((n * p.bt_sn + rc) * 2) : kOob);
      }
      __syncthreads();
      if (p.low != nullptr && nblk == 0) {  // bf16(x·A_e) of the tile's rows, 16 bytes at a time
        for (int c = tid; c < BM * RP / 8; c += kThreads) {
          const int m = c / (RP / 8), rc = (c - m * (RP / 8)) * 8;
          if (m < mrows) *(u32x4*)(p.low + (row0 + m) * p.ldl + rc) = *(const u32x4*)(Ls + m * LP + rc);
        }
      }
    }
    // Block by block: out = c · acc + s · bf16(x·A_e)·B_e (one MFMA chain of depth R into a
    // temporary) + bias, stored 8 bytes (four consecutive columns of one row) per lane and group.
    const bool lora_on = NRB > 0 && p.scaling != 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = (i * WAVES_M + wm) * 32 + (lane & 31);
      if (i >= am) continue;
      bf16* orow = p.out + (row0 + row) * p.ldo;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if (j >= an) continue;
        f32x16 t = f32x16{};
        if constexpr (NRB > 0) {
          if (lora_on) {
#pragma unroll
            for (int rk = 0; rk < NRB; ++rk) {
              const bf16x8 lf = *(const bf16x8*)(Ls + ((i * WAVES_M + wm) * 32 + (lane & 31)) * LP + rk * 16 + (lane >> 5) * 8);
              const bf16x8 bfr = *(const bf16x8*)(Lb + ((j * WAVES_N + wn) * 32 + (lane & 31)) * LP + rk * 16 + (lane >> 5) * 8);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr, lf, t, 0, 0, 0);
            }
          }
        }
        if (row >= mrows) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + (j * WAVES_N + wn) * 32 + 8 * g + col_l;
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

// ---- launch ----
static size_t lds_bytes(int rp, int E) {
  return (size_t)2 * (BM + BN + rp) * BK * sizeof(bf16) + (size_t)(2 * (E + 1) + 16) * sizeof(int);
}
static_assert(BM * (kMaxRank + 8) <= 2 * BM * BK && BN * (kMaxRank + 8) <= 2 * BN * BK,
              "the epilogue's low and B^T tiles must fit in the stage buffers they alias");

template <int WDT, bool BKC, bool SCALE_K, int NRB>
static int launch_t(const GemmArgs& a, hipStream_t s) {
  auto kern = grouped_gemm_kernel<WDT, BKC, SCALE_K, NRB>;
  const size_t lds = lds_bytes(NRB * 16, a.E);
  static std::mutex mu;
  static std::unordered_map<int64_t, int> grid_cache;  // (device, lds) -> grid
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
  return launch_status("grouped_gemm");
}

template <int WDT, bool BKC, bool SCALE_K>
static int launch_r(const GemmArgs& a, hipStream_t s) {
  switch (a.rank / 16) {
    case 0: return launch_t<WDT, BKC, SCALE_K, 0>(a, s);
    case 1: return launch_t<WDT, BKC, SCALE_K, 1>(a, s);
    case 2: return launch_t<WDT, BKC, SCALE_K, 2>(a, s);
    case 3: return launch_t<WDT, BKC, SCALE_K, 3>(a, s);
    default: return launch_t<WDT, BKC, SCALE_K, 4>(a, s);
  }
}

}  // namespace mlora

using namespace mlora;

static bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

// The fused adapter gradient's arguments (mlora_grouped_gemm_db)
struct DbIn {
  const void* l;
  int64_t ldl;
  void* out;
  int64_t o_se, o_sk, o_sr;
  void* workspace;
  size_t workspace_bytes;
};

// The fused SwiGLU's output (mlora_grouped_gemm_gather_swiglu)
struct SwiOut {
  void* act;
  int64_t lda;
};

static int grouped_gemm_impl(const DbIn* db, const SwiOut* so, const void* x, int64_t ldx, const int64_t* gather, int gk, int64_t xrows,
                             const void* row_scale, int row_scale_dt, int64_t rows, int K, int N, const void* w,
                             int w_dtype,
                                  int64_t w_se, int64_t w_sk, int64_t w_sn, const float* scale, int scale_kind,
                                  int64_t scale_se, int scale_on_k, const uint8_t* nf4_absmax_q,
                                  const float* nf4_absmax2, const float* nf4_code2, const float* nf4_offset,
                                  const float* nf4_code, const void* at, int64_t at_se, int64_t at_sr,
                                  const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                                  const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                                  const int32_t* offsets, int E, void* stream) {
  clear_error();
  if (rows < 0) return fail("grouped_gemm: rows=%lld is negative", (long long)rows);
  if (gather != nullptr) {
    if (gk < 1) return fail("grouped_gemm_gather: k=%d must be >= 1", gk);
    if (rows > (int64_t)0xFFFFFFFFu) return fail("grouped_gemm_gather: rows=%lld must be below 2^32", (long long)rows);
    if (xrows < 0 || xrows * ldx * 2 > 0x7FFFFFF0) return fail("grouped_gemm_gather: x (%lld rows) exceeds 2 GiB", (long long)xrows);
  }
  if (row_scale != nullptr) {
    if (gather == nullptr) return fail("grouped_gemm: a row scale is indexed through gather");
    if (row_scale_dt != MLORA_DT_BF16 && row_scale_dt != MLORA_DT_F32)
      return fail("grouped_gemm_gather: row scale dtype %d is not bf16/f32", row_scale_dt);
  }
  if (E < 1 || E > 4096) return fail("grouped_gemm: E=%d outside [1, 4096]", E);
  if (K < 8 || K % 8) return fail("grouped_gemm: K=%d must be a positive multiple of 8", K);
  if (N < 8 || N % 8) return fail("grouped_gemm: N=%d must be a positive multiple of 8", N);
  if (ldx < K || ldx % 8 || !aligned(x, 16))
    return fail("grouped_gemm: x needs a 16-byte aligned base and a row stride (%lld) that is a multiple of 8 and >= K",
                (long long)ldx);
  if (ldo < N || ldo % 8 || !aligned(out, 16))
    return fail("grouped_gemm: out needs a 16-byte aligned base and a row stride (%lld) that is a multiple of 8 and >= N",
                (long long)ldo);
  if ((int64_t)BM * ldx * 2 > 0x7FFFFFF0) return fail("grouped_gemm: row stride %lld too large", (long long)ldx);
  if ((int64_t)BM * ldo * 2 > 0x7FFFFFF0) return fail("grouped_gemm: out row stride %lld too large", (long long)ldo);
  const bool bkc = w_sk == 1;
  if (!bkc && w_sn != 1)
    return fail("grouped_gemm: the stack needs a unit stride along k or n (w_sk=%lld, w_sn=%lld)", (long long)w_sk,
                (long long)w_sn);
  const int64_t other = bkc ? w_sn : w_sk;
  const int64_t esize = w_dtype == MLORA_DT_BF16 ? 2 : 1;
  if (w_se * esize > 0x7FFFFFF0) return fail("grouped_gemm: one expert's weights exceed 2 GiB");
  if (w_dtype == MLORA_DT_BF16) {
    if (other % 8 || w_se % 8 || !aligned(w, 16)) return fail("grouped_gemm: a bf16 stack needs 16-byte aligned rows");
  } else if (w_dtype == MLORA_DT_FP8_E4M3) {
    if (other % 8 || w_se % 8 || !aligned(w, 8)) return fail("grouped_gemm: an fp8 stack needs 8-byte aligned rows");
  } else if (w_dtype == MLORA_DT_NF4_KT) {
    if (w_sk != 1 || other % 64 || w_se % 64 || N % 64 || !aligned(w, 16))
      return fail("grouped_gemm: NF4 codes along k need k contiguous, rows of a multiple of 64 values and N %% 64 == 0");
    if (!nf4_absmax2 || !nf4_code) return fail("grouped_gemm: NF4 codes along k need their absmax table and code");
  } else if (w_dtype == MLORA_DT_NF4) {
    if (other % 64 || w_se % 64 || !aligned(w, 4))
      return fail("grouped_gemm: an NF4 stack needs rows of a multiple of 64 values");
    if (!nf4_absmax_q || !nf4_absmax2 || !nf4_code2 || !nf4_offset || !nf4_code)
      return fail("grouped_gemm: an NF4 stack needs its absmax_q, absmax2, code2, offset and code");
  } else {
    return fail("grouped_gemm: stack dtype %d is not bf16, fp8 e4m3 or NF4", w_dtype);
  }
  if (scale_kind < 0 || scale_kind > 2) return fail("grouped_gemm: scale_kind %d unknown", scale_kind);
  if (scale_kind != MLORA_SCALE_NONE && scale == nullptr)
    return fail("grouped_gemm: scale_kind %d without a scale", scale_kind);
  const bool scale_k = scale_kind == MLORA_SCALE_ROW && scale_on_k;
  if (scale_k && w_dtype != MLORA_DT_FP8_E4M3) return fail("grouped_gemm: a per-row scale along k is for fp8 stacks");
  const bool lora = at != nullptr;
  if (lora) {
    if (bt == nullptr) return fail("grouped_gemm: adapter A without B");
    if (rank < 16 || rank > kMaxRank || rank % 16)
      return fail("grouped_gemm: rank=%d must be 16, 32, 48 or 64 (pad with zeros)", rank);
    if (at_sr < K || at_sr % 8 || at_se % 8 || !aligned(at, 16))
      return fail("grouped_gemm: A^T needs 16-byte aligned rows of >= K values");
    if (bt_sn < rank || bt_sn % 8 || bt_se % 8 || !aligned(bt, 16))
      return fail("grouped_gemm: B^T needs 16-byte aligned rows of >= rank values");
    if (low != nullptr && (ldl < rank || ldl % 8 || !aligned(low, 16)))
      return fail("grouped_gemm: low needs 16-byte aligned rows of >= rank values");
  }
  if (db != nullptr) {
    if (w_dtype != MLORA_DT_BF16) return fail("grouped_gemm_db: the fused adapter gradient takes a bf16 stack");
    if (!lora || rank != 16) return fail("grouped_gemm_db: the fused adapter gradient needs the adapters at rank 16");
    if (E > grouped_gemm_db_max_experts()) return fail("grouped_gemm_db: E=%d above %d", E, grouped_gemm_db_max_experts());
    if (db->l == nullptr || db->out == nullptr) return fail("grouped_gemm_db: l and the gradient are required");
    if (db->ldl < 16 || db->ldl % 8 || !aligned(db->l, 16)) return fail("grouped_gemm_db: l needs 16-byte aligned rows of >= 16 values");
    const size_t need = mlora_grouped_gemm_db_workspace_bytes(rows, K, E);
    if (db->workspace == nullptr || db->workspace_bytes < need || !aligned(db->workspace, 16))
      return fail("grouped_gemm_db: workspace of %zu bytes, %zu needed (16-byte aligned)", db->workspace_bytes, need);
  }
  if (so != nullptr) {
    if (db != nullptr) return fail("grouped_gemm_swiglu: no fused adapter gradient with the fused SwiGLU");
    if (!grouped_gemm_swiglu_fits()) return fail("grouped_gemm_swiglu: this build's tile shape does not pair gate and up columns");
    if (N % 256) return fail("grouped_gemm_swiglu: N=%d (gate and up) must be a multiple of 256", N);
    if (so->act == nullptr || so->lda < N / 2 || so->lda % 8 || !aligned(so->act, 16))
      return fail("grouped_gemm_swiglu: act needs a 16-byte aligned base and a row stride (%lld) that is a multiple of 8 "
                  "and >= N/2", (long long)so->lda);
    if ((int64_t)BM * so->lda * 2 > 0x7FFFFFF0) return fail("grouped_gemm_swiglu: act row stride %lld too large", (long long)so->lda);
  }
  if (rows == 0 && db == nullptr) return 0;  // (with the fused gradient, the launch writes its zeros)

  GemmArgs g{};
  g.x = (const bf16*)x; g.ldx = ldx;
  g.gather = gather; g.gk = gk; g.xrows = xrows;
  g.row_scale = row_scale; g.row_scale_dt = row_scale_dt;
  g.w = (const uint8_t*)w; g.w_se = w_se; g.w_sk = w_sk; g.w_sn = w_sn;
  g.scale = scale; g.scale_se = scale_se; g.scale_kind = scale_kind;
  g.nf4_q = nf4_absmax_q; g.nf4_absmax2 = nf4_absmax2; g.nf4_code2 = nf4_code2; g.nf4_offset = nf4_offset;
  g.nf4_code = nf4_code;
  g.at = (const bf16*)at; g.at_se = at_se; g.at_sr = at_sr;
  g.bt = (const bf16*)bt; g.bt_se = bt_se; g.bt_sn = bt_sn;
  g.rank = lora ? rank : 0;
  g.scaling = scaling;
  g.bias = (const bf16*)bias; g.bias_se = bias_se;
  g.out = (bf16*)out; g.ldo = ldo;
  g.low = lora ? (bf16*)low : nullptr; g.ldl = ldl;
  g.offsets = offsets; g.rows = rows; g.E = E; g.K = K; g.N = N;
  if (db != nullptr) {
    g.dbl = (const bf16*)db->l; g.dbl_ld = db->ldl;
    g.dbw = (float*)db->workspace;
    g.dbo = (bf16*)db->out; g.dbo_se = db->o_se; g.dbo_sk = db->o_sk; g.dbo_sr = db->o_sr;
  }
  if (so != nullptr) {
    g.act = (bf16*)so->act; g.lda = so->lda; g.swi = N / 2;
    if (w_dtype != MLORA_DT_BF16 && !grouped_gemm_dma_takes(g, w_dtype, bkc, scale_k))
      return fail("grouped_gemm_swiglu: the fused SwiGLU needs a stack the DMA-fed product takes (k contiguous, "
                  "16-byte aligned rows; NF4: rows of whole 64-code blocks)");
  }
  hipStream_t s = as_stream(stream);
  // gathered rows are read by the DMA-fed product only (every stack type it takes)
  const char* no_gather = "grouped_gemm_gather: gathered rows need a stack the DMA-fed product takes (k contiguous, "
                          "16-byte aligned rows; NF4: rows of whole 64-code blocks)";
  switch (w_dtype) {
    case MLORA_DT_BF16: return launch_grouped_gemm_bf16(g, bkc, s);
    case MLORA_DT_FP8_E4M3:
      if (grouped_gemm_dma_takes(g, w_dtype, bkc, scale_k)) return launch_grouped_gemm_dma_q(g, w_dtype, scale_k, s);
      if (gather != nullptr) return fail("%s", no_gather);
      if (scale_k) return bkc ? launch_r<W_FP8, true, true>(g, s) : launch_r<W_FP8, false, true>(g, s);
      return bkc ? launch_r<W_FP8, true, false>(g, s) : launch_r<W_FP8, false, false>(g, s);
    case MLORA_DT_NF4_KT:
      if (grouped_gemm_dma_takes(g, w_dtype, bkc, false)) return launch_grouped_gemm_dma_q(g, w_dtype, false, s);
      return fail("grouped_gemm: NF4 codes along k need a 16-byte aligned stack");
    default:
      if (grouped_gemm_dma_takes(g, w_dtype, bkc, false)) return launch_grouped_gemm_dma_q(g, w_dtype, false, s);
      if (gather != nullptr) return fail("%s", no_gather);
      return bkc ? launch_r<W_NF4, true, false>(g, s) : launch_r<W_NF4, false, false>(g, s);
  }
}

extern "C" int mlora_grouped_gemm(const void* x, int64_t ldx, int64_t rows, int K, int N, const void* w, int w_dtype,
                                  int64_t w_se, int64_t w_sk, int64_t w_sn, const float* scale, int scale_kind,
                                  int64_t scale_se, int scale_on_k, const uint8_t* nf4_absmax_q,
                                  const float* nf4_absmax2, const float* nf4_code2, const float* nf4_offset,
                                  const float* nf4_code, const void* at, int64_t at_se, int64_t at_sr,
                                  const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                                  const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                                  const int32_t* offsets, int E, void* stream) {
  return grouped_gemm_impl(nullptr, nullptr, x, ldx, nullptr, 1, rows, nullptr, 0, rows, K, N, w, w_dtype, w_se, w_sk, w_sn, scale,
                           scale_kind,
                           scale_se, scale_on_k, nf4_absmax_q, nf4_absmax2, nf4_code2, nf4_offset, nf4_code, at, at_se,
                           at_sr, bt, bt_se, bt_sn, rank, scaling, bias, bias_se, out, ldo, low, ldl, offsets, E, stream);
}

extern "C" int mlora_grouped_gemm_gather(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                         const void* row_scale, int row_scale_dtype, int64_t rows, int K, int N, const void* w, int w_dtype, int64_t w_se,
                                         int64_t w_sk, int64_t w_sn, const float* scale, int scale_kind,
                                         int64_t scale_se, const void* at, int64_t at_se, int64_t at_sr,
                                         const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                                         const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low,
                                         int64_t ldl, const int32_t* offsets, int E, void* stream) {
  if (gather == nullptr) {
    clear_error();
    return fail("grouped_gemm_gather: gather is NULL");
  }
  return grouped_gemm_impl(nullptr, nullptr, x, ldx, gather, k, x_rows, row_scale, row_scale_dtype, rows, K, N, w, w_dtype, w_se, w_sk,
                           w_sn, scale, scale_kind,
                           scale_se, 0, nullptr, nullptr, nullptr, nullptr, nullptr, at, at_se, at_sr, bt, bt_se, bt_sn,
                           rank, scaling, bias, bias_se, out, ldo, low, ldl, offsets, E, stream);
}

extern "C" int mlora_grouped_gemm_gather_q(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                           const void* row_scale, int row_scale_dtype, int64_t rows, int K, int N,
                                           const void* w, int w_dtype, int64_t w_se, int64_t w_sk, int64_t w_sn,
                                           const float* scale, int scale_kind, int64_t scale_se, int scale_on_k,
                                           const uint8_t* nf4_absmax_q, const float* nf4_absmax2,
                                           const float* nf4_code2, const float* nf4_offset, const float* nf4_code,
                                           const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                                           int64_t bt_sn, int rank, float scaling, const void* bias, int64_t bias_se,
                                           void* out, int64_t ldo, void* low, int64_t ldl, const int32_t* offsets, int E,
                                           void* stream) {
  if (gather == nullptr) {
    clear_error();
    return fail("grouped_gemm_gather_q: gather is NULL");
  }
  return grouped_gemm_impl(nullptr, nullptr, x, ldx, gather, k, x_rows, row_scale, row_scale_dtype, rows, K, N, w, w_dtype,
                           w_se, w_sk, w_sn, scale, scale_kind, scale_se, scale_on_k, nf4_absmax_q, nf4_absmax2,
                           nf4_code2, nf4_offset, nf4_code, at, at_se, at_sr, bt, bt_se, bt_sn, rank, scaling, bias,
                           bias_se, out, ldo, low, ldl, offsets, E, stream);
}

extern "C" int mlora_grouped_gemm_gather_swiglu(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                                 int64_t rows, int K, int N, const void* w, int w_dtype, int64_t w_se,
                                                 int64_t w_sk, int64_t w_sn, const float* scale, int scale_kind,
                                                 int64_t scale_se, const uint8_t* nf4_absmax_q,
                                                 const float* nf4_absmax2, const float* nf4_code2,
                                                 const float* nf4_offset, const float* nf4_code, const void* at,
                                                 int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                                                 int64_t bt_sn, int rank, float scaling, const void* bias,
                                                 int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                                                 void* act, int64_t lda, const int32_t* offsets, int E, void* stream) {
  if (gather == nullptr) {
    clear_error();
    return fail("grouped_gemm_gather_swiglu: gather is NULL");
  }
  const SwiOut so{act, lda};
  return grouped_gemm_impl(nullptr, &so, x, ldx, gather, k, x_rows, nullptr, 0, rows, K, N, w, w_dtype, w_se, w_sk,
                           w_sn, scale, scale_kind, scale_se, 0, nf4_absmax_q, nf4_absmax2, nf4_code2, nf4_offset,
                           nf4_code, at, at_se, at_sr, bt, bt_se, bt_sn, rank, scaling, bias, bias_se, out, ldo, low,
                           ldl, offsets, E, stream);
}

extern "C" size_t mlora_grouped_gemm_db_workspace_bytes(int64_t rows, int K, int E) {
  if (rows < 0 || K < 1 || E < 1) return 0;
  return (size_t)grouped_gemm_db_slots(rows, E) * 16 * (size_t)K * sizeof(float);
}

extern "C" int mlora_grouped_gemm_db(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                     const void* row_scale, int row_scale_dtype, int64_t rows, int K, int N,
                                     const void* w, int64_t w_se, int64_t w_sk, int64_t w_sn, const float* scale,
                                     int scale_kind, int64_t scale_se, const void* at, int64_t at_se, int64_t at_sr,
                                     const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                                     const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                                     const void* db_l, int64_t db_ldl, void* db_out, int64_t db_o_se, int64_t db_o_sk,
                                     int64_t db_o_sr, void* workspace, size_t workspace_bytes,
                                     const int32_t* offsets, int E, void* stream) {
  const DbIn db{db_l, db_ldl, db_out, db_o_se, db_o_sk, db_o_sr,
                workspace, workspace_bytes};
  if (gather == nullptr) {
    if (row_scale != nullptr) {
      clear_error();
      return fail("grouped_gemm_db: a row scale is indexed through gather");
    }
    x_rows = rows;
  }
  return grouped_gemm_impl(&db, nullptr, x, ldx, gather, k, x_rows, row_scale, row_scale_dtype, rows, K, N, w, MLORA_DT_BF16,
                           w_se, w_sk, w_sn, scale, scale_kind, scale_se, 0, nullptr, nullptr, nullptr, nullptr,
                           nullptr, at, at_se, at_sr, bt, bt_se, bt_sn, rank, scaling, bias, bias_se, out, ldo, low,
                           ldl, offsets, E, stream);
}
