// Shared device helpers for the dsv41 sparse-attention path on CDNA4 (gfx950).
//
// Storage formats (the same bits the reference stores, see include/dsv41_hip.h for the interface):
//   bf16   : uint16_t raw bits, round-to-nearest-even conversion from fp32
//   e4m3   : OCP float8_e4m3fn (bias 7, max 448, subnormal ulp 2^-9), the operand format of gfx950 fp8 MFMA
// Rounding helpers reproduce the reference's fake-quant closed forms exactly (dsv41/fused.py:10-43).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsv41_hip.h"

#define DSV41_DEV __device__ __forceinline__

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(8))) int i32x8_t;

static constexpr float kLog2e = 1.4426950408889634f;

DSV41_DEV float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

DSV41_DEV uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

DSV41_DEV float round_bf16(float f) { return bf2f(f2bf(f)); }

// ceil(log2(a)) for a > 0, exact from the bit pattern (normal a).
DSV41_DEV int ceil_log2_f(float a) {
  const int bits = __float_as_int(a);
  const int e = ((bits >> 23) & 0xff) - 127;
  return e + ((bits & 0x7fffff) != 0 ? 1 : 0);
}

DSV41_DEV float pow2i(int e) { return __int_as_float((e + 127) << 23); }

// Nearest e4m3fn value (ties to even) of v with |v| <= 448, as fp32.
DSV41_DEV float round_e4m3(float v) {
  const float a = fabsf(v);
  int e = ((__float_as_int(a) >> 23) & 0xff) - 127;
  e = e < -6 ? -6 : e;
  const float ulp = pow2i(e - 3);
  float r = rintf(a * pow2i(3 - e)) * ulp;  // scaling by a power of two is exact
  r = fminf(r, 448.0f);
  return v < 0.0f ? -r : r;
}

// Nearest E2M1 value {0,.5,1,1.5,2,3,4,6} (ties to even) of v with |v| <= 6.
DSV41_DEV float round_e2m1(float v) {
  const float a = fabsf(v);
  float r = a < 2.0f ? rintf(a * 2.0f) * 0.5f : (a < 4.0f ? rintf(a) : rintf(a * 0.5f) * 2.0f);
  r = fminf(r, 6.0f);
  return v < 0.0f ? -r : r;
}

// Encode an fp32 value that is already on the e4m3 grid (|v| <= 448) as the e4m3fn byte.
DSV41_DEV uint32_t e4m3_bits(float v) {
  const uint32_t s = v < 0.0f ? 0x80u : 0u;
  const float a = fabsf(v);
  if (a == 0.0f) return s;
  const int e = ((__float_as_int(a) >> 23) & 0xff) - 127;
  if (e < -6) {  // subnormal: a = m * 2^-9
    return s | (uint32_t)(int)(a * 512.0f);
  }
  const uint32_t m = (uint32_t)((__float_as_int(a) >> 20) & 7);
  return s | ((uint32_t)(e + 7) << 3) | m;
}

DSV41_DEV float e4m3_value(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  const float a = e == 0 ? (float)m * 0.001953125f : pow2i((int)e - 7) * (1.0f + (float)m * 0.125f);
  return (b & 0x80u) ? -a : a;
}

// Order-preserving uint32 key of an fp32 score: larger float -> larger key, -0.0 folded onto +0.0.
DSV41_DEV uint32_t score_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <typename T>
DSV41_DEV T wave_shfl_xor(T v, int m) {
  return __shfl_xor(v, m, 64);
}

DSV41_DEV bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16x16x32 bf16 MFMA: D[16x16] += A[16x32] * B[32x16].  Output layout: lane l holds column (l & 15),
// rows 4*(l >> 4) + i.  Operand k-ordering is symmetric between A and B.
DSV41_DEV f32x4_t mfma_bf16_16x16x32(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 16x16x128 fp8(e4m3) x fp8(e4m3) MFMA with unit block scales (E8M0 127 = 2^0).
DSV41_DEV f32x4_t mfma_fp8_16x16x128(i32x8_t a, i32x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Phase timestamps for development builds (-DDSV41_TIMING): thread 0 of block (0,0,0) records wall_clock64() (a
// constant-rate clock) into g_dsv41_ts[i].  Compiled out otherwise.
#ifdef DSV41_TIMING
__device__ long long g_dsv41_ts[64];
#define DSV41_TS(i)                                                                                       \
  do {                                                                                                    \
    if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) g_dsv41_ts[i] = wall_clock64(); \
  } while (0)
// Per-workgroup start / end stamps (first 4096 workgroups of a launch, linear block id).
__device__ long long g_dsv41_wg[4096][2];
#define DSV41_WG_TS(k)                                                                                     \
  do {                                                                                                     \
    const int _b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);                         \
    if (threadIdx.x == 0 && _b < 4096) g_dsv41_wg[_b][k] = wall_clock64();                                 \
  } while (0)
#else
#define DSV41_TS(i) \
  do {              \
  } while (0)
#define DSV41_WG_TS(k) \
  do {                 \
  } while (0)
#endif

#define DSV41_CHECK_LAUNCH()                          \
  do {                                                \
    hipError_t _e = hipGetLastError();                \
    if (_e != hipSuccess) return (int)_e;             \
  } while (0)
