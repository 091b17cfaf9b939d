// Shared definitions of the gfx950 kernels: vector types, conversions, wave primitives, errors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/mlora.h"

namespace mlora {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---- error reporting (per host thread), defined in api.hip ----
int fail(const char* fmt, ...);
void clear_error();
// status of the last launch on the calling thread; 0 or a failure recorded with the kernel's name
int launch_status(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- conversions ----
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// two bf16 packed in a dword (element 0 in the low half) from two floats, rounded to nearest even
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16 a = (bf16)lo, b = (bf16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ float round_bf16(float v) { return (float)(bf16)v; }

// OCP e4m3fn byte to fp32: exact (every e4m3 value is a bf16/fp32 value).  0x7f/0xff (NaN) are not
// produced by the quantisers here and decode as 480.
__device__ __forceinline__ float fp8_e4m3_to_f32(uint32_t byte) {
  uint32_t s = (byte & 0x80u) << 24;
  uint32_t e = (byte >> 3) & 0xFu;
  uint32_t m = byte & 0x7u;
  float normal = __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
  float sub = __uint_as_float(s | __float_as_uint((float)m * 0.001953125f));  // m * 2^-9
  return e ? normal : sub;
}

// fp32 -> OCP e4m3fn with round-to-nearest-even.  Magnitudes from 464 up (and NaN) give NaN
// (0x7F | sign), as torch's float8_e4m3fn conversion does; 448 < |v| < 464 round to 448.
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  uint32_t b = __float_as_uint(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  b &= 0x7FFFFFFFu;
  if (b >= 0x43E80000u) return sign | 0x7Fu;  // >= 464 or NaN
  if (b < 0x3C800000u) {                       // below 2^-6: subnormal range, units of 2^-9
    // add 2^-9 * 2^23 style bias: rounding of the integer count of 2^-9 steps, ties to even
    const float steps = __uint_as_float(b) * 512.0f;  // exact (power-of-two scaling)
    const float r = __builtin_rintf(steps);           // nearest, ties to even
    return sign | (uint32_t)r;                        // r <= 8 -> 8 is the smallest normal 0x08
  }
  // normal: keep 3 mantissa bits, round to nearest even on the dropped 20 bits
  const uint32_t lsb = (b >> 20) & 1u;
  b += 0x7FFFFu + lsb;
  const uint32_t exp = (b >> 23) - 120u;  // rebias 127 -> 7
  return sign | (exp << 3) | ((b >> 20) & 7u);
}

// eight bf16 (one 16-byte vector) <-> eight floats
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(v[i] & 0xFFFFu);
    f[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

// a routing weight (bf16 or fp32) as fp32
template <typename TW>
__device__ __forceinline__ float load_w(const TW* w, int64_t i);
template <>
__device__ __forceinline__ float load_w<float>(const float* w, int64_t i) { return w[i]; }
template <>
__device__ __forceinline__ float load_w<bf16>(const bf16* w, int64_t i) { return (float)w[i]; }

// ---- SwiGLU (TF integrations/moe.py:509-520: act = silu(gate) * up) ----
// sigmoid(g) = 1 / (1 + e^-g) from the hardware's base-2 exponential and reciprocal (v_exp_f32, v_rcp_f32,
// each within about 1 ulp of fp32): a few ulp of fp32 in all, far below the bf16 rounding every caller
// applies to its results.  e^-g overflowing to +inf gives 0 (silu(g) = -0 for very negative g), as the
// libm form does.
__device__ __forceinline__ float sigmoidf_(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// SwiGLU's backward over eight columns of one row: gate gg, up u, the incoming gradient d taken with the
// row's weight wt (dact = wt * d), zeros where !live.  act receives the forward's act values (bf16(silu *
// up), as the forward kernel rounds them); returns sum_q d[q] * act[q] in column order.
__device__ __forceinline__ float swiglu_grad8(const float* gg, const float* u, const float* d, float wt, bool live,
                                              float* dg, float* du, float* act) {
  float dot = 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float sg = sigmoidf_(gg[q]);
    const float silu = gg[q] * sg;
    act[q] = round_bf16(silu * u[q]);
    dot += d[q] * act[q];
    const float dd = wt * d[q];
    du[q] = live ? dd * silu : 0.f;
    dg[q] = live ? dd * u[q] * sg * (1.0f + gg[q] * (1.0f - sg)) : 0.f;
  }
  return dot;
}

// ---- wave primitives (wave64) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = __shfl_xor((unsigned long long)v, o, kWave);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace mlora
