// The layer's data movement and elementwise steps around the grouped products: the gather of the
// tokens' rows into expert order, the SwiGLU gate, and the weighted combine back to tokens, with
// their gradients.  All of them are bound by HBM bandwidth: rows move as 16-byte vectors, every
// sum runs in fp32 in a fixed order (no atomics), so results are the same every run.
//
// Reference behaviour (paths into thinkube/meepsquared; TF: = transformers):
//   gather   src/meepsquared/_moe.py:80,85-87  selected = h[perm // k], sentinel rows zeroed
//   SwiGLU   TF:integrations/moe.py:509-520     gate, up = chunk(2); silu(gate) * up
//   combine  src/meepsquared/_moe.py:123-126   (out * w)[inverse].view(T, k, H).sum(1)
//   weights  src/meepsquared/_moe.py:123         each routed row's weight, applied to the adapters' rows
//            (l[r] weighted as the combine weights the gradient rows of the down product)
#include <algorithm>

#include "common.hpp"

namespace mlora {

// ---- gather: one 16-byte vector per thread, grid-stride over (row, vector) ----
__global__ __launch_bounds__(256) void gather_rows_kernel(const u32x4* __restrict__ h, int64_t ldh_v, int64_t Hv,
                                                          const int64_t* __restrict__ perm, int64_t S, int k,
                                                          const int32_t* __restrict__ offsets, int E,
                                                          u32x4* __restrict__ out) {
  const int64_t valid = offsets[E - 1];
  const int64_t total = S * Hv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = i / Hv, c = i - p * Hv;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (p < valid) v = h[(perm[p] / k) * ldh_v + c];
    out[i] = v;
  }
}

// ---- the gather's gradient: per token, the sum of its k rows ----
// Rows summed or weighted per token over its k slots: with k known at compile time (KT > 0) the slot
// loop is unrolled, so every slot's index and row loads are in flight together.
template <int KT, typename F>
__device__ __forceinline__ void for_slots(int k, F&& f) {
  if constexpr (KT > 0) {
#pragma unroll
    for (int j = 0; j < KT; ++j) f(j);
  } else {
    for (int j = 0; j < k; ++j) f(j);
  }
}

// One token per workgroup: the token's k row indices are workgroup-uniform (scalar loads), its
// threads stride over the row's 16-byte vectors.
template <int KT>
__global__ __launch_bounds__(256) void gather_rows_backward_kernel(const u32x4* __restrict__ dsel, int64_t Hv,
                                                                   const int64_t* __restrict__ inv, int64_t T, int k,
                                                                   const int32_t* __restrict__ offsets, int E,
                                                                   u32x4* __restrict__ dh) {
  if constexpr (KT > 0) k = KT;
  const int64_t valid = offsets[E - 1];
  const int64_t t = blockIdx.x;
  for (int64_t c = threadIdx.x; c < Hv; c += blockDim.x) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (KT > 0) {  // every slot's row loaded before any is added (a sentinel's reads row 0, unused)
      u32x4 v[KT];
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const int64_t p = inv[t * KT + j];
        v[j] = dsel[(p < valid ? p : 0) * Hv + c];
      }
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        float f[8];
        unpack8(v[j], f);
        const bool ok = inv[t * KT + j] < valid;
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] += ok ? f[q] : 0.f;
      }
    } else {
      for (int j = 0; j < k; ++j) {
        const int64_t p = inv[t * k + j];
        if (p < valid) {
          float f[8];
          unpack8(dsel[p * Hv + c], f);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[q] += f[q];
        }
      }
    }
    dh[t * Hv + c] = pack8(acc);
  }
}

// ---- SwiGLU ----
__global__ __launch_bounds__(256) void swiglu_kernel(const u32x4* __restrict__ gu, int64_t S, int64_t Iv,
                                                     u32x4* __restrict__ act) {
  const int64_t total = S * Iv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / Iv, c = i - r * Iv;
    float g[8], u[8], o[8];
    unpack8(gu[r * 2 * Iv + c], g);
    unpack8(gu[r * 2 * Iv + Iv + c], u);
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = g[q] * sigmoidf_(g[q]) * u[q];
    act[i] = pack8(o);
  }
}

__global__ __launch_bounds__(256) void swiglu_backward_kernel(const u32x4* __restrict__ gu,
                                                              const u32x4* __restrict__ dact, int64_t S, int64_t Iv,
                                                              u32x4* __restrict__ dgu) {
  const int64_t total = S * Iv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / Iv, c = i - r * Iv;
    float g[8], u[8], d[8], dg[8], du[8];
    unpack8(gu[r * 2 * Iv + c], g);
    unpack8(gu[r * 2 * Iv + Iv + c], u);
    unpack8(dact[i], d);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float sg = sigmoidf_(g[q]);
      const float silu = g[q] * sg;
      du[q] = d[q] * silu;
      dg[q] = d[q] * u[q] * sg * (1.0f + g[q] * (1.0f - sg));
    }
    dgu[r * 2 * Iv + c] = pack8(dg);
    dgu[r * 2 * Iv + Iv + c] = pack8(du);
  }
}

// The SwiGLU backward fed by the down product's input gradient g taken WITHOUT the combine weights,
// with the combine weights' gradient formed on the way.  Row p of the expert order carries the
// weight w[perm[p]]: dact = w · g, and the weight's gradient <dout[t], y[p]>, with y[p] = act[p]·W_e
// + scaling · bf16(act[p]·A_e)·B_e (no bias), equals <g[p], act[p]> (g[p] = dout[t]·(W_e^T +
// scaling · B_e^T A_e^T) is the gradient of that inner product with respect to act[p]); act is
// recomputed from gu exactly as the forward rounds it, so neither y nor act is read.
// A block takes `rows` rows (8, fewer for wide rows: their parts fit 32 KB of LDS); its threads stride
// over the rows' 16-byte vectors (consecutive threads, consecutive vectors), each vector's part of the
// dot product goes to LDS, and one wave per row sums a row's parts in a fixed order.  Rows from
// offsets[E-1] on (the sentinels') get zero gradients.
constexpr int kSwRows = 8;
constexpr int kSwUnroll = 4;  // vectors per thread loaded together

template <typename TW>
__global__ __launch_bounds__(256) void swiglu_backward_weighted_kernel(
    const u32x4* __restrict__ gu, const u32x4* __restrict__ g, int64_t S, int64_t Iv, const TW* __restrict__ w,
    const int64_t* __restrict__ perm, const int32_t* __restrict__ offsets, int E, u32x4* __restrict__ dgu,
    TW* __restrict__ dw, int rows) {
  extern __shared__ float sw_part[];  // rows * Iv vector parts, then the rows' weights
  float* wrow = sw_part + rows * Iv;
  const int64_t r0 = (int64_t)blockIdx.x * rows;
  const int nrows = (int)min((int64_t)rows, S - r0);
  const int64_t valid = offsets[E - 1];
  const int tid = threadIdx.x;
  if (tid < nrows) wrow[tid] = r0 + tid < valid ? load_w(w, perm[r0 + tid]) : 0.f;
  __syncthreads();
  const int n = nrows * (int)Iv;
  for (int i0 = tid; i0 < n; i0 += 256 * kSwUnroll) {  // every load of the kSwUnroll vectors in flight at once
    u32x4 vg[kSwUnroll], vu[kSwUnroll], vd[kSwUnroll];
#pragma unroll
    for (int h = 0; h < kSwUnroll; ++h) {
      const int i = i0 + 256 * h;
      if (i < n) {
        const int rr = i / (int)Iv;
        const int64_t p = r0 + rr, c = i - rr * Iv;
        vg[h] = gu[p * 2 * Iv + c];
        vu[h] = gu[p * 2 * Iv + Iv + c];
        vd[h] = g[p * Iv + c];
      }
    }
#pragma unroll
    for (int h = 0; h < kSwUnroll; ++h) {
      const int i = i0 + 256 * h;
      if (i >= n) continue;
      const int rr = i / (int)Iv;
      const int64_t p = r0 + rr, c = i - rr * Iv;
      float gg[8], u[8], d[8], dg[8], du[8];
      unpack8(vg[h], gg);
      unpack8(vu[h], u);
      unpack8(vd[h], d);
      const bool live = p < valid;
      float act[8];
      const float dot = swiglu_grad8(gg, u, d, wrow[rr], live, dg, du, act);
      dgu[p * 2 * Iv + c] = pack8(dg);
      dgu[p * 2 * Iv + Iv + c] = pack8(du);
      sw_part[i] = dot;
    }
  }
  __syncthreads();
  const int lane = tid & 63;
  for (int rr = tid >> 6; rr < nrows; rr += 4) {
    float dot = 0.f;
    for (int c = lane; c < Iv; c += 64) dot += sw_part[rr * Iv + c];
    dot = wave_sum(dot);
    const int64_t p = r0 + rr;
    if (lane == 0) dw[perm[p]] = (TW)(p < valid ? dot : 0.f);
  }
}

// ---- combine: per token, sum over its k rows of bf16(y * w) ----
template <int KT, typename TW>
__global__ __launch_bounds__(256) void combine_kernel(const u32x4* __restrict__ y, int64_t Hv,
                                                      const TW* __restrict__ w, const int64_t* __restrict__ inv,
                                                      int64_t T, int k, const int32_t* __restrict__ offsets, int E,
                                                      u32x4* __restrict__ out) {
  constexpr bool kBf16Weights = sizeof(TW) == 2;
  if constexpr (KT > 0) k = KT;
  const int64_t valid = offsets[E - 1];
  const int64_t t = blockIdx.x;  // one token per workgroup (row indices and weights workgroup-uniform)
  for (int64_t c = threadIdx.x; c < Hv; c += blockDim.x) {
    const int64_t i = t * Hv + c;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add = [&](const u32x4& v, float wt) {
      float f[8];
      unpack8(v, f);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        // with bf16 weights the reference's product is a bf16 tensor; with fp32 weights it is fp32
        const float prod = f[q] * wt;
        acc[q] += kBf16Weights ? round_bf16(prod) : prod;
      }
    };
    if constexpr (KT > 0) {  // every slot's row and weight loaded before any is added (a sentinel reads row 0)
      u32x4 v[KT];
      float wt[KT];
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const int64_t p = inv[t * KT + j];
        v[j] = y[(p < valid ? p : 0) * Hv + c];
        wt[j] = load_w(w, t * KT + j);
      }
#pragma unroll
      for (int j = 0; j < KT; ++j)
        if (inv[t * KT + j] < valid) add(v[j], wt[j]);
    } else {
      for (int j = 0; j < k; ++j) {
        const int64_t p = inv[t * k + j];
        if (p < valid) add(y[p * Hv + c], load_w(w, t * k + j));
      }
    }
    out[i] = pack8(acc);
  }
}

// ---- the combine's gradients: one block per token ----
template <typename TW>
__global__ __launch_bounds__(256) void combine_backward_kernel(const u32x4* __restrict__ dout,
                                                               const u32x4* __restrict__ y, int64_t Hv,
                                                               const TW* __restrict__ w,
                                                               const int64_t* __restrict__ inv, int64_t T, int k,
                                                               const int32_t* __restrict__ offsets, int E,
                                                               u32x4* __restrict__ dy, TW* __restrict__ dw) {
  __shared__ float part[4];
  const int64_t valid = offsets[E - 1];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int j = 0; j < k; ++j) {
    const int64_t p = inv[t * k + j];
    const bool sentinel = p >= valid;
    const float wt = load_w(w, t * k + j);
    float dot = 0.f;
    for (int64_t c = threadIdx.x; c < Hv; c += blockDim.x) {
      float d[8], f[8], o[8];
      unpack8(dout[t * Hv + c], d);
      if (sentinel) {
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] = 0.f;
      } else {
        unpack8(y[p * Hv + c], f);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          o[q] = d[q] * wt;
          dot += d[q] * f[q];
        }
      }
      if (dy != nullptr) dy[p * Hv + c] = pack8(o);
    }
    dot = wave_sum(dot);
    if (lane == 0) part[wv] = dot;
    __syncthreads();
    if (threadIdx.x == 0) {
      const float s = sentinel ? 0.f : ((part[0] + part[1]) + (part[2] + part[3]));
      dw[t * k + j] = (TW)s;
    }
    __syncthreads();
  }
}

// The combine weights' gradient alone (the down product then reads the output gradient through the
// permutation, so no weighted copy dy is written): one wave per (token, slot), dw = <dout[t], y[p]>,
// fp32 lane sums then a wave sum; no barrier.
template <typename TW>
__global__ __launch_bounds__(256) void combine_dw_kernel(const u32x4* __restrict__ dout, const u32x4* __restrict__ y,
                                                         int64_t Hv, const int64_t* __restrict__ inv, int64_t T, int k,
                                                         const int32_t* __restrict__ offsets, int E,
                                                         TW* __restrict__ dw) {
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= T * k) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const int64_t t = idx / k, p = inv[idx];
  float dot = 0.f;
  if (p < offsets[E - 1]) {
    for (int64_t c = lane; c < Hv; c += 64) {
      float d[8], f[8];
      unpack8(dout[t * Hv + c], d);
      unpack8(y[p * Hv + c], f);
#pragma unroll
      for (int q = 0; q < 8; ++q) dot += d[q] * f[q];
    }
  }
  dot = wave_sum(dot);
  if (lane == 0) dw[idx] = (TW)dot;
}

static unsigned grid_for(int64_t total) {
  int64_t g = (total + 255) / 256;
  if (g > 256 * 64) g = 256 * 64;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_gather_rows(const void* h, int64_t ldh, int64_t H, const int64_t* perm, int64_t S, int k,
                                 const int32_t* offsets, int E, void* out, void* stream) {
  clear_error();
  if (H % 8 || ldh % 8) return fail("gather_rows: H=%lld and ldh=%lld must be multiples of 8", (long long)H, (long long)ldh);
  if (k < 1 || E < 1) return fail("gather_rows: k=%d, E=%d must be >= 1", k, E);
  if (S == 0) return 0;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(grid_for(S * (H / 8))), dim3(256), 0, as_stream(stream),
                     (const u32x4*)h, ldh / 8, H / 8, perm, S, k, offsets, E, (u32x4*)out);
  return launch_status("gather_rows");
}

extern "C" int mlora_gather_rows_backward(const void* dsel, int64_t H, const int64_t* inv, int64_t T, int k,
                                          const int32_t* offsets, int E, void* dh, void* stream) {
  clear_error();
  if (H % 8) return fail("gather_rows_backward: H=%lld must be a multiple of 8", (long long)H);
  if (k < 1 || E < 1) return fail("gather_rows_backward: k=%d, E=%d must be >= 1", k, E);
  if (T == 0) return 0;
  if (T > 0x7FFFFFFF) return fail("gather_rows_backward: T=%lld too large", (long long)T);
  const dim3 g((unsigned)T), b((unsigned)std::min<int64_t>(256, (H / 8 + 63) / 64 * 64));
#define MLORA_GRB(KT)                                                                                      \
  hipLaunchKernelGGL(gather_rows_backward_kernel<KT>, g, b, 0, as_stream(stream), (const u32x4*)dsel, H / 8, inv, T, \
                     k, offsets, E, (u32x4*)dh)
  switch (k) {
    case 1: MLORA_GRB(1); break;
    case 2: MLORA_GRB(2); break;
    case 4: MLORA_GRB(4); break;
    case 6: MLORA_GRB(6); break;
    case 8: MLORA_GRB(8); break;
    default: MLORA_GRB(0); break;
  }
#undef MLORA_GRB
  return launch_status("gather_rows_backward");
}

// ---- row weights: out[r, :] = bf16(w[index[r]] · l[r, :]), one 16-byte vector per thread ----
template <typename TW>
__global__ __launch_bounds__(256) void scale_rows_kernel(const u32x4* __restrict__ l, int64_t ldl_v, int64_t Rv,
                                                         const TW* __restrict__ w, const int64_t* __restrict__ index,
                                                         int64_t rows, u32x4* __restrict__ out, int64_t ldo_v) {
  const int64_t n = rows * Rv;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / Rv, v = i - r * Rv;
    const float s = load_w(w, index[r]);
    float f[8];
    unpack8(l[r * ldl_v + v], f);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] *= s;
    out[r * ldo_v + v] = pack8(f);
  }
}

extern "C" int mlora_scale_rows(const void* l, int64_t ldl, int64_t rows, int64_t R, const void* w, int w_dtype,
                                const int64_t* index, void* out, int64_t ldo, void* stream) {
  clear_error();
  if (R % 8 || ldl % 8 || ldo % 8 || ldl < R || ldo < R || ((uintptr_t)l & 15u) || ((uintptr_t)out & 15u))
    return fail("scale_rows: R (%lld) and the row strides must be multiples of 8, the bases 16-byte aligned", (long long)R);
  if (w_dtype != MLORA_DT_BF16 && w_dtype != MLORA_DT_F32) return fail("scale_rows: w_dtype %d is not bf16/f32", w_dtype);
  if (rows == 0) return 0;
  const dim3 grid(grid_for(rows * (R / 8)));
  if (w_dtype == MLORA_DT_F32)
    hipLaunchKernelGGL(scale_rows_kernel<float>, grid, dim3(256), 0, as_stream(stream), (const u32x4*)l, ldl / 8, R / 8,
                       (const float*)w, index, rows, (u32x4*)out, ldo / 8);
  else
    hipLaunchKernelGGL(scale_rows_kernel<bf16>, grid, dim3(256), 0, as_stream(stream), (const u32x4*)l, ldl / 8, R / 8,
                       (const bf16*)w, index, rows, (u32x4*)out, ldo / 8);
  return launch_status("scale_rows");
}

extern "C" int mlora_swiglu(const void* gu, int64_t S, int64_t I, void* act, void* stream) {
  clear_error();
  if (I % 8) return fail("swiglu: I=%lld must be a multiple of 8", (long long)I);
  if (S == 0) return 0;
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(S * (I / 8))), dim3(256), 0, as_stream(stream), (const u32x4*)gu,
                     S, I / 8, (u32x4*)act);
  return launch_status("swiglu");
}

extern "C" int mlora_swiglu_backward(const void* gu, const void* dact, int64_t S, int64_t I, void* dgu, void* stream) {
  clear_error();
  if (I % 8) return fail("swiglu_backward: I=%lld must be a multiple of 8", (long long)I);
  if (S == 0) return 0;
  hipLaunchKernelGGL(swiglu_backward_kernel, dim3(grid_for(S * (I / 8))), dim3(256), 0, as_stream(stream),
                     (const u32x4*)gu, (const u32x4*)dact, S, I / 8, (u32x4*)dgu);
  return launch_status("swiglu_backward");
}

extern "C" int mlora_swiglu_backward_weighted(const void* gu, const void* g, int64_t S, int64_t I, const void* w,
                                              int w_dtype, const int64_t* perm, const int32_t* offsets, int E,
                                              void* dgu, void* dw, void* stream) {
  clear_error();
  if (I % 8) return fail("swiglu_backward_weighted: I=%lld must be a multiple of 8", (long long)I);
  if (E < 1) return fail("swiglu_backward_weighted: E=%d must be >= 1", E);
  if (S == 0) return 0;
  const int64_t Iv = I / 8;
  if (Iv > 8192) return fail("swiglu_backward_weighted: I=%lld above 65536", (long long)I);
  const int rows = (int)std::max<int64_t>(1, std::min<int64_t>(kSwRows, 8192 / Iv));
  if ((S + rows - 1) / rows > 0x7FFFFFFF) return fail("swiglu_backward_weighted: S=%lld too large", (long long)S);
  const dim3 grid((unsigned)((S + rows - 1) / rows)), block(256);
  const size_t sh = (size_t)(rows * Iv + rows) * sizeof(float);
  if (w_dtype == MLORA_DT_F32)
    hipLaunchKernelGGL(swiglu_backward_weighted_kernel<float>, grid, block, sh, as_stream(stream), (const u32x4*)gu,
                       (const u32x4*)g, S, Iv, (const float*)w, perm, offsets, E, (u32x4*)dgu, (float*)dw, rows);
  else if (w_dtype == MLORA_DT_BF16)
    hipLaunchKernelGGL(swiglu_backward_weighted_kernel<bf16>, grid, block, sh, as_stream(stream), (const u32x4*)gu,
                       (const u32x4*)g, S, Iv, (const bf16*)w, perm, offsets, E, (u32x4*)dgu, (bf16*)dw, rows);
  else
    return fail("swiglu_backward_weighted: weight dtype %d is not bf16/f32", w_dtype);
  return launch_status("swiglu_backward_weighted");
}

extern "C" int mlora_combine(const void* y, int64_t H, const void* w, int w_dtype, const int64_t* inv, int64_t T,
                             int k, const int32_t* offsets, int E, void* out, void* stream) {
  clear_error();
  if (H % 8) return fail("combine: H=%lld must be a multiple of 8", (long long)H);
  if (k < 1 || E < 1) return fail("combine: k=%d, E=%d must be >= 1", k, E);
  if (T == 0) return 0;
  if (T > 0x7FFFFFFF) return fail("combine: T=%lld too large", (long long)T);
  const dim3 g((unsigned)T), b((unsigned)std::min<int64_t>(256, (H / 8 + 63) / 64 * 64));
  if (w_dtype != MLORA_DT_F32 && w_dtype != MLORA_DT_BF16) return fail("combine: weight dtype %d is not bf16/f32", w_dtype);
#define MLORA_CMB(KT)                                                                                          \
  if (w_dtype == MLORA_DT_F32)                                                                                 \
    hipLaunchKernelGGL((combine_kernel<KT, float>), g, b, 0, as_stream(stream), (const u32x4*)y, H / 8,         \
                       (const float*)w, inv, T, k, offsets, E, (u32x4*)out);                                   \
  else                                                                                                         \
    hipLaunchKernelGGL((combine_kernel<KT, bf16>), g, b, 0, as_stream(stream), (const u32x4*)y, H / 8,          \
                       (const bf16*)w, inv, T, k, offsets, E, (u32x4*)out)
  switch (k) {
    case 1: MLORA_CMB(1); break;
    case 2: MLORA_CMB(2); break;
    case 4: MLORA_CMB(4); break;
    case 6: MLORA_CMB(6); break;
    case 8: MLORA_CMB(8); break;
    default: MLORA_CMB(0); break;
  }
#undef MLORA_CMB
  return launch_status("combine");
}

extern "C" int mlora_combine_backward(const void* dout, const void* y, int64_t H, const void* w, int w_dtype,
                                      const int64_t* inv, int64_t T, int k, const int32_t* offsets, int E, void* dy,
                                      void* dw, void* stream) {
  clear_error();
  if (H % 8) return fail("combine_backward: H=%lld must be a multiple of 8", (long long)H);
  if (k < 1 || E < 1) return fail("combine_backward: k=%d, E=%d must be >= 1", k, E);
  if (T == 0) return 0;
  if (T > 0x7FFFFFFF) return fail("combine_backward: T=%lld too large", (long long)T);
  if (dy == nullptr) {
    const int64_t blocks = (T * k + 3) / 4;
    if (blocks > 0x7FFFFFFF) return fail("combine_backward: T*k=%lld too large", (long long)(T * k));
    if (w_dtype == MLORA_DT_F32)
      hipLaunchKernelGGL(combine_dw_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                         (const u32x4*)dout, (const u32x4*)y, H / 8, inv, T, k, offsets, E, (float*)dw);
    else if (w_dtype == MLORA_DT_BF16)
      hipLaunchKernelGGL(combine_dw_kernel<bf16>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                         (const u32x4*)dout, (const u32x4*)y, H / 8, inv, T, k, offsets, E, (bf16*)dw);
    else
      return fail("combine_backward: weight dtype %d is not bf16/f32", w_dtype);
    return launch_status("combine_backward");
  }
  const dim3 g((unsigned)T), b(256);
  if (w_dtype == MLORA_DT_F32)
    hipLaunchKernelGGL(combine_backward_kernel<float>, g, b, 0, as_stream(stream), (const u32x4*)dout,
                       (const u32x4*)y, H / 8, (const float*)w, inv, T, k, offsets, E, (u32x4*)dy, (float*)dw);
  else if (w_dtype == MLORA_DT_BF16)
    hipLaunchKernelGGL(combine_backward_kernel<bf16>, g, b, 0, as_stream(stream), (const u32x4*)dout,
                       (const u32x4*)y, H / 8, (const bf16*)w, inv, T, k, offsets, E, (u32x4*)dy, (bf16*)dw);
  else
    return fail("combine_backward: weight dtype %d is not bf16/f32", w_dtype);
  return launch_status("combine_backward");
}

// ---- adapter layouts ----
// dst[e][b][a] = src[e*s_e + a*s_a + b*s_b]: a batched transpose into a contiguous (E, B, A) bf16
// tensor, through a 64 x 64 LDS tile (reads along b, writes along a).  Used for the adapters'
// roles in the input-gradient product (src/meepsquared/_grouped.py:304-310 addresses the same
// factors by strides; the kernel here takes them k-contiguous).
namespace mlora {

template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ src, int64_t A, int64_t B,
                                                        int64_t s_e, int64_t s_a, int64_t s_b, T* __restrict__ dst) {
  __shared__ T tile[64][66];
  const int64_t e = blockIdx.z, a0 = (int64_t)blockIdx.y * 64, b0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  const T* s = src + e * s_e;
#pragma unroll 4
  for (int i = ty; i < 64; i += 4) {
    const int64_t a = a0 + i, b = b0 + tx;
    if (a < A && b < B) tile[i][tx] = s[a * s_a + b * s_b];
  }
  __syncthreads();
  T* d = dst + e * A * B;
#pragma unroll 4
  for (int j = ty; j < 64; j += 4) {
    const int64_t b = b0 + j, a = a0 + tx;
    if (a < A && b < B) d[b * A + a] = tile[tx][j];
  }
}

// The same for a narrow side (the adapters' rank, 16 or 32): a TA x TB tile of 4096 values, so that
// every thread has work and each side's accesses run along its contiguous axis.
template <typename T, int TA, int TB>
__global__ __launch_bounds__(256) void transpose_narrow_kernel(const T* __restrict__ src, int64_t A, int64_t B,
                                                               int64_t s_e, int64_t s_a, int64_t s_b,
                                                               T* __restrict__ dst) {
  static_assert(TA * TB == 4096, "one tile of 4096 values");
  __shared__ T tile[TA][TB + 2];
  const int64_t e = blockIdx.z, a0 = (int64_t)blockIdx.y * TA, b0 = (int64_t)blockIdx.x * TB;
  const T* s = src + e * s_e;
#pragma unroll 4
  for (int idx = threadIdx.x; idx < TA * TB; idx += 256) {
    const int i = idx / TB, j = idx % TB;
    const int64_t a = a0 + i, b = b0 + j;
    if (a < A && b < B) tile[i][j] = s[a * s_a + b * s_b];
  }
  __syncthreads();
  T* d = dst + e * A * B;
#pragma unroll 4
  for (int idx = threadIdx.x; idx < TA * TB; idx += 256) {
    const int j = idx / TA, i = idx % TA;
    const int64_t a = a0 + i, b = b0 + j;
    if (a < A && b < B) d[b * A + a] = tile[i][j];
  }
}

// The narrow-side transpose with 16-byte accesses on both sides (bf16, both sizes multiples of 8,
// the source contiguous along b): rows of the source are read as vectors into a TA x TB tile,
// columns of the tile are gathered eight at a time and written as vectors along a.
template <int TA, int TB>
__global__ __launch_bounds__(256) void transpose_vec_kernel(const bf16* __restrict__ src, int64_t A, int64_t B,
                                                            int64_t s_e, int64_t s_a, bf16* __restrict__ dst) {
  static_assert(TA * TB == 4096 && TA % 8 == 0 && TB % 8 == 0, "a tile of 4096 values in vectors of 8");
  __shared__ __attribute__((aligned(16))) bf16 tile[TA][TB + 8];
  constexpr int NV = TA * TB / 8;
  const int64_t e = blockIdx.z, a0 = (int64_t)blockIdx.y * TA, b0 = (int64_t)blockIdx.x * TB;
  const bf16* s = src + e * s_e;
#pragma unroll
  for (int v = threadIdx.x; v < NV; v += 256) {
    const int i = v / (TB / 8), j = (v % (TB / 8)) * 8;
    const int64_t a = a0 + i, b = b0 + j;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (a < A && b < B) val = *(const u32x4*)(s + a * s_a + b);
    *(u32x4*)&tile[i][j] = val;
  }
  __syncthreads();
  bf16* d = dst + e * A * B;
#pragma unroll
  for (int v = threadIdx.x; v < NV; v += 256) {
    const int j = v / (TA / 8), i = (v % (TA / 8)) * 8;  // column j, rows i .. i + 7
    const int64_t a = a0 + i, b = b0 + j;
    if (a < A && b < B) {
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = (uint32_t)__builtin_bit_cast(uint16_t, tile[i + 2 * q][j]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, tile[i + 2 * q + 1][j]) << 16);
      *(u32x4*)(d + b * A + a) = o;
    }
  }
}

// The narrow-side transpose without LDS: each thread moves one 8 x 16 block (NB: 8 rows of the
// source by 16 of its narrow columns; else 16 narrow rows by 8 columns) through registers, reading
// 16-byte vectors along the source's rows and writing 16-byte vectors along the destination's, the
// pairs of bf16 regrouped by byte permutes.  Consecutive threads take consecutive blocks along the
// wide side, so both sides' accesses are contiguous across a wave.
__device__ __forceinline__ uint32_t lo_halves(uint32_t x0, uint32_t x1) { return __builtin_amdgcn_perm(x1, x0, 0x05040100u); }
__device__ __forceinline__ uint32_t hi_halves(uint32_t x0, uint32_t x1) { return __builtin_amdgcn_perm(x1, x0, 0x07060302u); }

template <bool NB>  // NB: the source's columns (B) are the narrow side; item t of the transpose
__device__ __forceinline__ void transpose_reg_item(const bf16* __restrict__ src, int64_t A, int64_t B, int64_t s_e,
                                                   int64_t s_a, bf16* __restrict__ dst, int64_t t) {
  if constexpr (NB) {  // rows a0 .. a0+7, columns b0 .. b0+15 -> dst rows b0 .. b0+15, columns a0 .. a0+7
    const int64_t na = A / 8, nb = B / 16;
    const int64_t a0 = (t % na) * 8, rest = t / na, b0 = (rest % nb) * 16, e = rest / nb;
    const bf16* s = src + e * s_e + a0 * s_a + b0;
    u32x4 r[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r[i][0] = *(const u32x4*)(s + i * s_a);
      r[i][1] = *(const u32x4*)(s + i * s_a + 8);
    }
    bf16* d = dst + e * A * B + b0 * A + a0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t x0 = r[2 * q][j >> 3][(j & 7) >> 1], x1 = r[2 * q + 1][j >> 3][(j & 7) >> 1];
        o[q] = (j & 1) ? hi_halves(x0, x1) : lo_halves(x0, x1);
      }
      *(u32x4*)(d + j * A) = o;
    }
  } else {  // rows a0 .. a0+15, columns b0 .. b0+7 -> dst rows b0 .. b0+7, columns a0 .. a0+15
    const int64_t nbk = B / 8, na = A / 16;
    const int64_t b0 = (t % nbk) * 8, rest = t / nbk, a0 = (rest % na) * 16, e = rest / na;
    const bf16* s = src + e * s_e + a0 * s_a + b0;
    u32x4 r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = *(const u32x4*)(s + i * s_a);
    bf16* d = dst + e * A * B + b0 * A + a0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t x0 = r[8 * h + 2 * q][j >> 1], x1 = r[8 * h + 2 * q + 1][j >> 1];
          o[q] = (j & 1) ? hi_halves(x0, x1) : lo_halves(x0, x1);
        }
        *(u32x4*)(d + j * A + 8 * h) = o;
      }
    }
  }
}

template <bool NB>
__global__ __launch_bounds__(64) void transpose_reg_kernel(const bf16* __restrict__ src, int64_t A, int64_t B,
                                                           int64_t s_e, int64_t s_a, bf16* __restrict__ dst,
                                                           int64_t items) {
  const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (t < items) transpose_reg_item<NB>(src, A, B, s_e, s_a, dst, t);
}

// One projection's adapters swapped for the input-gradient product: bt (E, N, R) -> at_out (E, R, N) (the
// narrow side the source's columns) over the job's first nb1 blocks, at (E, R, K) -> bt_out (E, K, R) over
// the rest of its nb blocks.
struct SwapJob {
  const bf16* bt;
  int64_t N, R, bt_se, bt_sn;
  bf16* at_out;
  int64_t items1, nb1;
  const bf16* at;
  int64_t K, at_se, at_sr;
  bf16* bt_out;
  int64_t items2, nb;
};
struct SwapJobs {
  SwapJob j[2];  // the second one's blocks follow the first's (nb = 0: none)
};

__device__ __forceinline__ void swap_block(const SwapJob& p, int64_t b) {
  if (b < p.nb1) {
    const int64_t t = b * 64 + threadIdx.x;
    if (t < p.items1) transpose_reg_item<true>(p.bt, p.N, p.R, p.bt_se, p.bt_sn, p.at_out, t);
  } else {
    const int64_t t = (b - p.nb1) * 64 + threadIdx.x;
    if (t < p.items2) transpose_reg_item<false>(p.at, p.R, p.K, p.at_se, p.at_sr, p.bt_out, t);
  }
}

// The adapters' transposes for the input-gradient products of one or two projections in one launch.
__global__ __launch_bounds__(64) void transpose_pair_kernel(SwapJobs jobs) {
  const int64_t b = blockIdx.x;
  if (b < jobs.j[0].nb) swap_block(jobs.j[0], b);
  else swap_block(jobs.j[1], b - jobs.j[0].nb);
}

template <bool NB>
static int launch_transpose_reg(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a,
                                void* dst, void* stream) {
  const int64_t items = E * (A / (NB ? 8 : 16)) * (B / (NB ? 16 : 8));
  const int64_t blocks = (items + 63) / 64;
  if (blocks > 0x7FFFFFFF) return fail("transpose: (E=%lld, A=%lld, B=%lld) exceeds the grid", (long long)E,
                                       (long long)A, (long long)B);
  hipLaunchKernelGGL((transpose_reg_kernel<NB>), dim3((unsigned)blocks), dim3(64), 0, as_stream(stream),
                     (const bf16*)src, A, B, s_e, s_a, (bf16*)dst, items);
  return launch_status("transpose");
}

template <int TA, int TB>
static int launch_transpose_vec(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a,
                                void* dst, void* stream) {
  if (E > 65535 || (A + TA - 1) / TA > 65535 || (B + TB - 1) / TB > 0x7FFFFFFF)
    return fail("transpose: (E=%lld, A=%lld, B=%lld) exceeds the grid", (long long)E, (long long)A, (long long)B);
  const dim3 grid((unsigned)((B + TB - 1) / TB), (unsigned)((A + TA - 1) / TA), (unsigned)E);
  hipLaunchKernelGGL((transpose_vec_kernel<TA, TB>), grid, dim3(256), 0, as_stream(stream), (const bf16*)src, A, B,
                     s_e, s_a, (bf16*)dst);
  return launch_status("transpose");
}

template <typename T, int TA, int TB>
static int launch_transpose(const char* what, const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e,
                            int64_t s_a, int64_t s_b, void* dst, void* stream) {
  if (E > 65535 || (A + TA - 1) / TA > 65535 || (B + TB - 1) / TB > 0x7FFFFFFF)
    return fail("%s: (E=%lld, A=%lld, B=%lld) exceeds the grid", what, (long long)E, (long long)A, (long long)B);
  const dim3 grid((unsigned)((B + TB - 1) / TB), (unsigned)((A + TA - 1) / TA), (unsigned)E);
  if constexpr (TA == 64 && TB == 64)
    hipLaunchKernelGGL(transpose_kernel<T>, grid, dim3(256), 0, as_stream(stream), (const T*)src, A, B, s_e, s_a, s_b,
                       (T*)dst);
  else
    hipLaunchKernelGGL((transpose_narrow_kernel<T, TA, TB>), grid, dim3(256), 0, as_stream(stream), (const T*)src, A,
                       B, s_e, s_a, s_b, (T*)dst);
  return launch_status(what);
}

}  // namespace mlora

extern "C" int mlora_transpose(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a,
                               int64_t s_b, void* dst, void* stream) {
  clear_error();
  if (E < 0 || A < 0 || B < 0) return fail("transpose: negative size");
  if (E == 0 || A == 0 || B == 0) return 0;
  const bool vec = s_b == 1 && A % 8 == 0 && B % 8 == 0 && s_a % 8 == 0 && s_e % 8 == 0 && ((uintptr_t)src & 15u) == 0 &&
                   ((uintptr_t)dst & 15u) == 0;
  // a narrow side of 16 or 32 (the adapters' rank) with a wide side past it: blocks through registers
  if (vec && B % 16 == 0 && B <= 32 && A > B) return launch_transpose_reg<true>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec && A % 16 == 0 && A <= 32 && B > A) return launch_transpose_reg<false>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec && A <= 16 && B > 16) return launch_transpose_vec<16, 256>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec && B <= 16 && A > 16) return launch_transpose_vec<256, 16>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec && A <= 32 && B > 32) return launch_transpose_vec<32, 128>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec && B <= 32 && A > 32) return launch_transpose_vec<128, 32>(src, E, A, B, s_e, s_a, dst, stream);
  if (vec) return launch_transpose_vec<64, 64>(src, E, A, B, s_e, s_a, dst, stream);
  if (A <= 16 && B > 16) return launch_transpose<bf16, 16, 256>("transpose", src, E, A, B, s_e, s_a, s_b, dst, stream);
  if (B <= 16 && A > 16) return launch_transpose<bf16, 256, 16>("transpose", src, E, A, B, s_e, s_a, s_b, dst, stream);
  if (A <= 32 && B > 32) return launch_transpose<bf16, 32, 128>("transpose", src, E, A, B, s_e, s_a, s_b, dst, stream);
  if (B <= 32 && A > 32) return launch_transpose<bf16, 128, 32>("transpose", src, E, A, B, s_e, s_a, s_b, dst, stream);
  return launch_transpose<bf16, 64, 64>("transpose", src, E, A, B, s_e, s_a, s_b, dst, stream);
}

extern "C" int mlora_transpose_u8(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a,
                                  int64_t s_b, void* dst, void* stream) {
  clear_error();
  if (E < 0 || A < 0 || B < 0) return fail("transpose_u8: negative size");
  if (E == 0 || A == 0 || B == 0) return 0;
  if (E > 65535 || (A + 63) / 64 > 65535 || (B + 63) / 64 > 0x7FFFFFFF)
    return fail("transpose_u8: (E=%lld, A=%lld, B=%lld) exceeds the grid", (long long)E, (long long)A, (long long)B);
  hipLaunchKernelGGL(transpose_kernel<uint8_t>, dim3((unsigned)((B + 63) / 64), (unsigned)((A + 63) / 64), (unsigned)E),
                     dim3(256), 0, as_stream(stream), (const uint8_t*)src, A, B, s_e, s_a, s_b, (uint8_t*)dst);
  return launch_status("transpose_u8");
}

// Fills one projection's swap job; nonzero (the error recorded) when its shapes or strides do not fit.
static int swap_job(const char* what, const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                    int64_t bt_sn, int64_t E, int64_t R, int64_t K, int64_t N, void* at_out, void* bt_out,
                    SwapJob& j) {
  if (E < 1 || (R != 16 && R != 32) || K <= R || N <= R || K % 8 || N % 8)
    return fail("%s: E=%lld, R=%lld, K=%lld, N=%lld: needs R 16 or 32 and K, N multiples of 8 above R", what,
                (long long)E, (long long)R, (long long)K, (long long)N);
  if (at_sr < K || at_sr % 8 || at_se % 8 || bt_sn < R || bt_sn % 8 || bt_se % 8 ||
      (((uintptr_t)at | (uintptr_t)bt | (uintptr_t)at_out | (uintptr_t)bt_out) & 15u))
    return fail("%s: the factors need 16-byte aligned rows and strides that are multiples of 8", what);
  j.bt = (const bf16*)bt;
  j.N = N;
  j.R = R;
  j.bt_se = bt_se;
  j.bt_sn = bt_sn;
  j.at_out = (bf16*)at_out;
  j.items1 = E * (N / 8) * (R / 16);
  j.nb1 = (j.items1 + 63) / 64;
  j.at = (const bf16*)at;
  j.K = K;
  j.at_se = at_se;
  j.at_sr = at_sr;
  j.bt_out = (bf16*)bt_out;
  j.items2 = E * (R / 16) * (K / 8);
  j.nb = j.nb1 + (j.items2 + 63) / 64;
  return 0;
}

static int launch_swap(const char* what, SwapJobs& jobs, void* stream) {
  const int64_t blocks = jobs.j[0].nb + jobs.j[1].nb;
  if (blocks > 0x7FFFFFFF) return fail("%s: the adapters exceed the grid", what);
  hipLaunchKernelGGL(transpose_pair_kernel, dim3((unsigned)blocks), dim3(64), 0, as_stream(stream), jobs);
  return launch_status(what);
}

extern "C" int mlora_swap_adapters(const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                                   int64_t bt_sn, int64_t E, int64_t R, int64_t K, int64_t N, void* at_out,
                                   void* bt_out, void* stream) {
  clear_error();
  SwapJobs jobs = {};
  if (int rc = swap_job("swap_adapters", at, at_se, at_sr, bt, bt_se, bt_sn, E, R, K, N, at_out, bt_out, jobs.j[0]))
    return rc;
  return launch_swap("swap_adapters", jobs, stream);
}

extern "C" int mlora_swap_adapters_two(const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                                       int64_t bt_sn, int64_t E, int64_t R, int64_t K, int64_t N, void* at_out,
                                       void* bt_out, const void* at2, int64_t at2_se, int64_t at2_sr, const void* bt2,
                                       int64_t bt2_se, int64_t bt2_sn, int64_t E2, int64_t R2, int64_t K2,
                                       int64_t N2, void* at2_out, void* bt2_out, void* stream) {
  clear_error();
  SwapJobs jobs = {};
  if (int rc = swap_job("swap_adapters_two", at, at_se, at_sr, bt, bt_se, bt_sn, E, R, K, N, at_out, bt_out,
                        jobs.j[0]))
    return rc;
  if (int rc = swap_job("swap_adapters_two (second)", at2, at2_se, at2_sr, bt2, bt2_se, bt2_sn, E2, R2, K2, N2,
                        at2_out, bt2_out, jobs.j[1]))
    return rc;
  return launch_swap("swap_adapters_two", jobs, stream);
}
