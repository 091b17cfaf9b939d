// Frozen expert stacks in fp8 e4m3 (one fp32 scale per expert or per output row) and in NF4 with
// double quantisation.  These run once, when a stack is converted; the grouped product decodes
// the result in its main loop.  All reductions (amax, mean) have a fixed order or are
// order-independent (max), so a conversion gives the same bytes every run.
//
// Reference behaviour (paths into thinkube/meepsquared):
//   fp8  src/meepsquared/_fp8.py:40 (E4M3_MAX), :122-134 (quantize_stack/dequantize_stack: scale =
//        max(amax, 1e-12) / 448 per expert, q = e4m3(w / scale)) — extended to per-row scales.
//   NF4  src/meepsquared/_vendor/axolotl/quantize.py:52-101,202-235 (the NF4 double-quant fields:
//        packed codes, absmax per 64, its 8-bit code with a second absmax per 256 and an offset).
#include <type_traits>

#include "common.hpp"

// Bit-exact definitions: no multiply-add contraction anywhere in this file.
#pragma clang fp contract(off)

namespace mlora {

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ldf<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldf<bf16>(const bf16* p, int64_t i) { return (float)p[i]; }
template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v) { p[i] = (T)v; }

__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, sh[i]);
  __syncthreads();
  return m;
}

// ---- fp8: amax per group ----
// groups laid out as contiguous runs of `len` values (per expert: R*C; per row: C)
template <typename T>
__global__ __launch_bounds__(256) void amax_runs_kernel(const T* __restrict__ x, int64_t len, float* __restrict__ scale) {
  __shared__ float sh[4];
  const int64_t g = blockIdx.x;
  float m = 0.f;
  for (int64_t i = threadIdx.x; i < len; i += blockDim.x) m = fmaxf(m, fabsf(ldf(x, g * len + i)));
  m = block_max(m, sh);
  if (threadIdx.x == 0) scale[g] = fmaxf(m, 1e-12f) / 448.0f;
}

// per column (e, c) over R rows: one thread per column
template <typename T>
__global__ __launch_bounds__(256) void amax_cols_kernel(const T* __restrict__ x, int64_t E, int64_t R, int64_t C,
                                                        float* __restrict__ scale) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E * C) return;
  const int64_t e = i / C, c = i - e * C;
  float m = 0.f;
  for (int64_t r = 0; r < R; ++r) m = fmaxf(m, fabsf(ldf(x, (e * R + r) * C + c)));
  scale[i] = fmaxf(m, 1e-12f) / 448.0f;
}

// the scale index of flat element i
__device__ __forceinline__ int64_t scale_index(int64_t i, int group, int rows_on_last, int64_t R, int64_t C) {
  if (group == MLORA_SCALE_EXPERT) return i / (R * C);
  if (!rows_on_last) return i / C;
  const int64_t e = i / (R * C);
  return e * C + (i % C);
}

template <typename T>
__global__ __launch_bounds__(256) void fp8_quant_kernel(const T* __restrict__ x, int64_t n, int group, int rows_on_last,
                                                        int64_t R, int64_t C, const float* __restrict__ scale,
                                                        uint8_t* __restrict__ q) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    q[i] = (uint8_t)f32_to_e4m3(ldf(x, i) / scale[scale_index(i, group, rows_on_last, R, C)]);
}

template <typename T>
__global__ __launch_bounds__(256) void fp8_dequant_kernel(const uint8_t* __restrict__ q, int64_t n, int group,
                                                          int rows_on_last, int64_t R, int64_t C,
                                                          const float* __restrict__ scale, T* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    stf(y, i, fp8_e4m3_to_f32(q[i]) * scale[scale_index(i, group, rows_on_last, R, C)]);
}

// ---- NF4 ----
// absmax of each 64-value block: one thread per block
template <typename T>
__global__ __launch_bounds__(256) void nf4_absmax_kernel(const T* __restrict__ x, int64_t nblocks, float* __restrict__ absmax) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float m = 0.f;
  for (int i = 0; i < 64; ++i) m = fmaxf(m, fabsf(ldf(x, b * 64 + i)));
  absmax[b] = m;
}

// offset = mean of the absmaxes: one block, each thread a strided fp64 partial sum, then a fixed tree
__global__ __launch_bounds__(1024) void nf4_mean_kernel(const float* __restrict__ absmax, int64_t nblocks,
                                                        float* __restrict__ offset) {
  __shared__ double sh[1024];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < nblocks; i += blockDim.x) s += (double)absmax[i];
  sh[threadIdx.x] = s;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) offset[0] = (float)(sh[0] / (double)nblocks);
}

// nearest entry of a code book (ties to the lower index)
__device__ __forceinline__ int nearest(float v, const float* code, int n) {
  int best = 0;
  float bd = fabsf(v - code[0]);
  for (int i = 1; i < n; ++i) {
    const float d = fabsf(v - code[i]);
    if (d < bd) {
      bd = d;
      best = i;
    }
  }
  return best;
}

// second level: per 256 absmaxes, absmax2 = max |absmax - offset|, q = nearest code2 entry of the ratio
__global__ __launch_bounds__(256) void nf4_double_quant_kernel(const float* __restrict__ absmax, int64_t nblocks,
                                                               const float* __restrict__ offset,
                                                               const float* __restrict__ code2,
                                                               uint8_t* __restrict__ absmax_q,
                                                               float* __restrict__ absmax2) {
  __shared__ float sh[4];
  __shared__ float c2[256];
  c2[threadIdx.x] = code2[threadIdx.x];
  const int64_t g = blockIdx.x;
  const int64_t i = g * 256 + threadIdx.x;
  const float off = offset[0];
  const float v = i < nblocks ? absmax[i] - off : 0.f;
  const float m = block_max(fabsf(v), sh);
  if (threadIdx.x == 0) absmax2[g] = m;
  if (i < nblocks) absmax_q[i] = (uint8_t)nearest(m > 0.f ? v / m : 0.f, c2, 256);
}

// codes: one thread per 8 values (4 bytes), relative to the block's own absmax
template <typename T>
__global__ __launch_bounds__(256) void nf4_codes_kernel(const T* __restrict__ x, int64_t n,
                                                        const float* __restrict__ absmax,
                                                        const float* __restrict__ code, uint8_t* __restrict__ packed) {
  __shared__ float c[16];
  if (threadIdx.x < 16) c[threadIdx.x] = code[threadIdx.x];
  __syncthreads();
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8-value group
  if (j * 8 >= n) return;
  const float a = absmax[(j * 8) >> 6];
  const float inv = a > 0.f ? 1.0f / a : 0.f;
  uint32_t word = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int hi = nearest(ldf(x, j * 8 + 2 * p) * inv, c, 16);
    const int lo = nearest(ldf(x, j * 8 + 2 * p + 1) * inv, c, 16);
    word |= (uint32_t)((hi << 4) | lo) << (8 * p);
  }
  *(uint32_t*)(packed + j * 4) = word;
}

template <typename T>
__global__ __launch_bounds__(256) void nf4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                          const uint8_t* __restrict__ absmax_q,
                                                          const float* __restrict__ absmax2,
                                                          const float* __restrict__ offset,
                                                          const float* __restrict__ code,
                                                          const float* __restrict__ code2, int64_t n,
                                                          T* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i >> 6;
    const float a = code2[absmax_q[b]] * absmax2[b >> 8] + offset[0];  // two roundings (contraction is off)
    const uint32_t byte = packed[i >> 1];
    const uint32_t nib = (i & 1) ? (byte & 0xFu) : (byte >> 4);
    stf(y, i, code[nib] * a);
  }
}

// The NF4 stack read the other way: from a contiguous stack (E, R, C) (blocks of 64 along C), the codes
// of its transpose (E, C, R) packed two per byte along R (first in the high nibble), and every block's
// decoded absmax laid out as (E, C / 64, R): for the input-gradient product, which reads the stack with
// R as its k.  The values are unchanged: element (e, c, r) decodes as code[nibble] · absmax[e, c/64, r],
// the same two roundings as nf4_dequant_kernel.
__global__ __launch_bounds__(256) void nf4_transpose_codes_kernel(const uint8_t* __restrict__ packed, int64_t E,
                                                                  int64_t R, int64_t C, uint8_t* __restrict__ out) {
  const int64_t n = E * C * (R / 2);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rp = i % (R / 2), ec = i / (R / 2), c = ec % C, e = ec / C;
    uint32_t nib[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int64_t el = (e * R + 2 * rp + q) * C + c;
      const uint32_t byte = packed[el >> 1];
      nib[q] = (el & 1) ? (byte & 0xFu) : (byte >> 4);
    }
    out[i] = (uint8_t)((nib[0] << 4) | nib[1]);
  }
}

__global__ __launch_bounds__(256) void nf4_transpose_absmax_kernel(const uint8_t* __restrict__ absmax_q,
                                                                   const float* __restrict__ absmax2,
                                                                   const float* __restrict__ offset,
                                                                   const float* __restrict__ code2, int64_t E,
                                                                   int64_t R, int64_t C, float* __restrict__ out) {
  const int64_t cb = C / 64, n = E * cb * R;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i % R, ecb = i / R, b = ecb % cb, e = ecb / cb;
    const int64_t blk = (e * R + r) * cb + b;
    out[i] = code2[absmax_q[blk]] * absmax2[blk >> 8] + offset[0];  // two roundings (contraction is off)
  }
}

static unsigned grid_of(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_fp8_quantize(const void* x, int x_dtype, int64_t E, int64_t R, int64_t C, int group,
                                  int rows_on_last, uint8_t* q, float* scale, void* stream) {
  clear_error();
  if (E < 1 || R < 1 || C < 1) return fail("fp8_quantize: empty stack (%lld, %lld, %lld)", (long long)E, (long long)R, (long long)C);
  if (group != MLORA_SCALE_EXPERT && group != MLORA_SCALE_ROW) return fail("fp8_quantize: group %d unknown", group);
  if (x_dtype != MLORA_DT_BF16 && x_dtype != MLORA_DT_F32) return fail("fp8_quantize: dtype %d is not bf16/f32", x_dtype);
  hipStream_t s = as_stream(stream);
  const int64_t n = E * R * C;
  auto run = [&](auto* xp) {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
    if (group == MLORA_SCALE_EXPERT)
      hipLaunchKernelGGL(amax_runs_kernel<T>, dim3((unsigned)E), dim3(256), 0, s, xp, R * C, scale);
    else if (!rows_on_last)
      hipLaunchKernelGGL(amax_runs_kernel<T>, dim3((unsigned)(E * R)), dim3(256), 0, s, xp, C, scale);
    else
      hipLaunchKernelGGL(amax_cols_kernel<T>, dim3(grid_of(E * C)), dim3(256), 0, s, xp, E, R, C, scale);
    hipLaunchKernelGGL(fp8_quant_kernel<T>, dim3(grid_of(n)), dim3(256), 0, s, xp, n, group, rows_on_last, R, C, scale, q);
  };
  if (x_dtype == MLORA_DT_F32) run((const float*)x); else run((const bf16*)x);
  return launch_status("fp8_quantize");
}

extern "C" int mlora_fp8_dequantize(const uint8_t* q, const float* scale, int64_t E, int64_t R, int64_t C, int group,
                                    int rows_on_last, void* y, int y_dtype, void* stream) {
  clear_error();
  if (E < 1 || R < 1 || C < 1) return fail("fp8_dequantize: empty stack");
  if (group != MLORA_SCALE_EXPERT && group != MLORA_SCALE_ROW) return fail("fp8_dequantize: group %d unknown", group);
  const int64_t n = E * R * C;
  hipStream_t s = as_stream(stream);
  if (y_dtype == MLORA_DT_F32)
    hipLaunchKernelGGL(fp8_dequant_kernel<float>, dim3(grid_of(n)), dim3(256), 0, s, q, n, group, rows_on_last, R, C, scale, (float*)y);
  else if (y_dtype == MLORA_DT_BF16)
    hipLaunchKernelGGL(fp8_dequant_kernel<bf16>, dim3(grid_of(n)), dim3(256), 0, s, q, n, group, rows_on_last, R, C, scale, (bf16*)y);
  else
    return fail("fp8_dequantize: dtype %d is not bf16/f32", y_dtype);
  return launch_status("fp8_dequantize");
}

extern "C" size_t mlora_nf4_workspace_bytes(int64_t n) { return (size_t)((n + 63) / 64) * sizeof(float); }

extern "C" int mlora_nf4_quantize(const void* x, int x_dtype, int64_t n, const float* code, const float* code2,
                                  uint8_t* packed, uint8_t* absmax_q, float* absmax2, float* offset, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  clear_error();
  if (n < 64 || n % 64) return fail("nf4_quantize: n=%lld must be a positive multiple of 64", (long long)n);
  if (x_dtype != MLORA_DT_BF16 && x_dtype != MLORA_DT_F32) return fail("nf4_quantize: dtype %d is not bf16/f32", x_dtype);
  if (workspace == nullptr || workspace_bytes < mlora_nf4_workspace_bytes(n))
    return fail("nf4_quantize: workspace of %zu bytes, %zu needed", workspace_bytes, mlora_nf4_workspace_bytes(n));
  const int64_t nblocks = n / 64;
  float* absmax = (float*)workspace;
  hipStream_t s = as_stream(stream);
  auto run = [&](auto* xp) {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
    hipLaunchKernelGGL(nf4_absmax_kernel<T>, dim3(grid_of(nblocks)), dim3(256), 0, s, xp, nblocks, absmax);
    hipLaunchKernelGGL(nf4_mean_kernel, dim3(1), dim3(1024), 0, s, absmax, nblocks, offset);
    hipLaunchKernelGGL(nf4_double_quant_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, absmax,
                       nblocks, offset, code2, absmax_q, absmax2);
    hipLaunchKernelGGL(nf4_codes_kernel<T>, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, s, xp, n, absmax, code, packed);
  };
  if (x_dtype == MLORA_DT_F32) run((const float*)x); else run((const bf16*)x);
  return launch_status("nf4_quantize");
}

extern "C" int mlora_nf4_dequantize(const uint8_t* packed, const uint8_t* absmax_q, const float* absmax2,
                                    const float* offset, const float* code, const float* code2, int64_t n, void* y,
                                    int y_dtype, void* stream) {
  clear_error();
  if (n < 64 || n % 64) return fail("nf4_dequantize: n=%lld must be a positive multiple of 64", (long long)n);
  hipStream_t s = as_stream(stream);
  if (y_dtype == MLORA_DT_F32)
    hipLaunchKernelGGL(nf4_dequant_kernel<float>, dim3(grid_of(n)), dim3(256), 0, s, packed, absmax_q, absmax2, offset, code, code2, n, (float*)y);
  else if (y_dtype == MLORA_DT_BF16)
    hipLaunchKernelGGL(nf4_dequant_kernel<bf16>, dim3(grid_of(n)), dim3(256), 0, s, packed, absmax_q, absmax2, offset, code, code2, n, (bf16*)y);
  else
    return fail("nf4_dequantize: dtype %d is not bf16/f32", y_dtype);
  return launch_status("nf4_dequantize");
}

extern "C" int mlora_nf4_transpose(const uint8_t* packed, const uint8_t* absmax_q, const float* absmax2,
                                   const float* offset, const float* code2, int64_t E, int64_t R, int64_t C,
                                   uint8_t* out_packed, float* out_absmax, void* stream) {
  clear_error();
  if (E < 1 || R < 2 || R % 2 || C < 64 || C % 64)
    return fail("nf4_transpose: (E=%lld, R=%lld, C=%lld) needs R even and C a multiple of 64", (long long)E,
                (long long)R, (long long)C);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(nf4_transpose_codes_kernel, dim3(grid_of(E * C * (R / 2))), dim3(256), 0, s, packed, E, R, C,
                     out_packed);
  hipLaunchKernelGGL(nf4_transpose_absmax_kernel, dim3(grid_of(E * (C / 64) * R)), dim3(256), 0, s, absmax_q, absmax2,
                     offset, code2, E, R, C, out_absmax);
  return launch_status("nf4_transpose");
}
