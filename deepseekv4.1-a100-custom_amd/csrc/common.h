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

// max(x, 0) for finite x in one v_med3_f32 (fmaxf adds a canonicalisation of its MFMA-produced operand).
DSV41_DEV float relu(float x) { return __builtin_amdgcn_fmed3f(x, 0.0f, 3.402823466e38f); }

// Sum / max over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48), result in every lane: two VALU row
// swaps (v_permlane32_swap, v_permlane16_swap) instead of LDS-routed shuffles.
DSV41_DEV float row_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// row_sum4 of two values at once: x0's sum in lanes 0-31, x1's in lanes 32-63 (one swap of each kind for both).
DSV41_DEV float row_sum4_pair(float x0, float x1) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // lanes l < 32: x0[l] + x0[l+32]; else x1
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
DSV41_DEV float row_max4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Reductions within 16-lane rows by DPP lane moves (VALU, no LDS round trip): quad xor 1 and 2, then the
// half-row mirror (the other quad of each 8-lane half) and the row mirror (the other half); every lane of the
// group receives the result.
template <int CTRL>
DSV41_DEV float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
DSV41_DEV float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);         // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);         // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);        // row_half_mirror
  return v + dpp_mov<0x140>(v);  // row_mirror
}
// Whole-wave sum, the result in every lane.
DSV41_DEV float wave_sum(float v) { return row_sum4(row16_sum(v)); }
// Maximum over aligned groups of `group` consecutive lanes (a power of two <= 64), the result in every lane.
DSV41_DEV float group_max(float v, int group) {
  if (group >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
  if (group >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
  if (group >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
  if (group >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
  if (group >= 32) {
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
  }
  if (group >= 64) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  }
  return v;
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
// As DSV41_TS, from thread `thr` of block (0,0,0).
#define DSV41_TST(i, thr)                                                                                  \
  do {                                                                                                     \
    if (threadIdx.x == (thr) && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) g_dsv41_ts[i] = wall_clock64(); \
  } while (0)
// Per-workgroup start / end stamps (first 4096 workgroups of a launch, linear block id).
__device__ long long g_dsv41_wg[4096][2];
#define DSV41_WG_TS(k)                                                                                     \
  do {                                                                                                     \
    const int _b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);                         \
    if (threadIdx.x == 0 && _b < 4096) g_dsv41_wg[_b][k] = wall_clock64();                                 \
  } while (0)
// Per-workgroup phase stamps (1-D grids, first 1024 workgroups).
__device__ long long g_dsv41_ph[1024][8];
__device__ long long g_dsv41_ck[1024][8];  // shader clock at the same points
// Extra per-workgroup stamps (32 slots, 1-D grids, first 1024 workgroups).
__device__ long long g_dsv41_px[1024][32];
#define DSV41_PX(k)                                                                       \
  do {                                                                                    \
    if (threadIdx.x == 0 && blockIdx.x < 1024) g_dsv41_px[blockIdx.x][k] = wall_clock64(); \
  } while (0)
#define DSV41_PH(k)                                                  \
  do {                                                               \
    if (threadIdx.x == 0 && blockIdx.x < 1024) {                     \
      g_dsv41_ph[blockIdx.x][k] = wall_clock64();                    \
      g_dsv41_ck[blockIdx.x][k] = clock64();                         \
    }                                                                \
  } while (0)
#else
#define DSV41_PX(k) \
  do {              \
  } while (0)
#define DSV41_PH(k) \
  do {              \
  } while (0)
#define DSV41_TS(i) \
  do {              \
  } while (0)
#define DSV41_TST(i, thr) \
  do {                    \
  } while (0)
#define DSV41_WG_TS(k) \
  do {                 \
  } while (0)
#endif

// Workgroup execution barrier that waits for this wave's LDS operations but not for its outstanding global loads
// (e.g. direct-to-LDS tile loads still in flight, waited for separately with a counted vmcnt).  __syncthreads()
// would wait for every outstanding memory operation.  The memory clobber keeps the compiler from moving memory
// accesses across it.
// s_waitcnt immediate that waits for vmcnt <= n (n < 64) and nothing else.
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }
DSV41_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// As lds_dma16, with the destination given as a wave-uniform LDS byte address (no generic-to-LDS conversion per
// load: the caller computes the workgroup's LDS base once).
DSV41_DEV void lds_dma16_at(const void* src, uint32_t lds_addr) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr);  // (an SGPR operand: uniform values may sit in VGPRs)
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
// As lds_dma16_at, 4 bytes per lane (lane i writes lds_addr + 4 i).
DSV41_DEV void lds_dma4_at(const void* src, uint32_t lds_addr) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
// The LDS-address-space view of a generic pointer to a __shared__ object (its low 32 bits): accesses through it
// are LDS instructions (counted by lgkmcnt alone), not flat ones.
template <class T>
DSV41_DEV __attribute__((address_space(3))) T* lds_ptr(T* p) {
  return (__attribute__((address_space(3))) T*)(uint32_t)(uintptr_t)p;
}
// LDS byte address of a __shared__ object.
DSV41_DEV uint32_t lds_addr_of(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p);
}

// 16-byte direct-to-LDS load: lane i writes lds_dst + 16 i (lds_dst is wave-uniform).  Issued as inline assembly
// so the compiler does not treat later LDS reads as dependent on it (it would wait for every outstanding load
// before them); callers wait for these loads with explicit vmcnt counts.  Compiler-tracked loads are unaffected:
// loads complete in order, so the compiler's own waits only become stricter.
// The LDS address is the low 32 bits of the flat address of an LDS object (the LDS aperture sits in the high
// half), taken without the address-space conversion's null test.
DSV41_DEV void lds_dma16(const void* src, void* lds_dst) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}

// ---- scans
// Inclusive prefix sum over the 64 lanes of a wave with DPP lane moves (no LDS traffic): shifts of 1, 2, 4, 8
// within each row of 16 lanes, then the row totals are carried by row_bcast:15 (into rows 1, 3) and row_bcast:31
// (into rows 2, 3).  Lanes a move does not reach add 0.
DSV41_DEV int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Exclusive prefix sum over the NT threads of a workgroup (tmp: NT/64 ints), with the workgroup total; two barriers.
template <int NT>
DSV41_DEV int block_scan_dpp(int v, int* tmp, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int s = tmp[w];
    before += w < wave ? s : 0;
    all += s;
  }
  *total = all;
  __syncthreads();
  return before + x - v;
}

// Exclusive prefix sums of two values over the NT threads of a workgroup, with both totals; ONE barrier (no
// trailing one): `tmp` (NT/64 int2) must not be written again until a later barrier has passed.
template <int NT>
DSV41_DEV int2 block_scan2_dpp(int v0, int v1, int2* tmp, int2* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x0 = wave_incl_scan(v0), x1 = wave_incl_scan(v1);
  if (lane == 63) tmp[wave] = make_int2(x0, x1);
  __syncthreads();
  int2 before = make_int2(0, 0), all = make_int2(0, 0);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int2 s = tmp[w];
    before.x += w < wave ? s.x : 0;
    before.y += w < wave ? s.y : 0;
    all.x += s.x;
    all.y += s.y;
  }
  *total = all;
  return make_int2(before.x + x0 - v0, before.y + x1 - v1);
}

// ---- workgroup groups that exchange data through one XCD's L2
// The 8 XCDs of an MI355X each have their own L2; a device-scope release/acquire writes back / invalidates a whole
// L2, which costs tens of microseconds when every workgroup of a launch does it.  Workgroups that cooperate are
// therefore placed on one XCD (workgroups of a 1-D grid are dealt to the XCDs round-robin: workgroup b runs on XCD
// b % 8), where the shared L2 makes their stores visible to each other once they have left the CU (the CU caches are
// write-through, and only lines read after the exchange are cached).  Each workgroup checks its hardware XCD id;
// one that finds itself elsewhere publishes with a device-scope fence and flags the group, and a reader that sees
// the flag acquires with a device-scope fence, so a misplaced writer is still read correctly.  A misplaced reader
// cannot see the home members' stores (they stay in the home L2): its caller reports that case as an error.
constexpr int kXcds = 8;
constexpr int kMisplaced = 1 << 16;  // flag added to a group arrival counter by a misplaced workgroup

DSV41_DEV int xcd_id() { return __builtin_amdgcn_s_getreg(0x1814) & 15; }  // hwreg(HW_REG_XCC_ID, 0, 4)

// Arrive at the group counter after this workgroup's stores (call from every thread); returns the previous counter
// value to every thread.  `home` is the XCD the group was placed on.
DSV41_DEV int group_arrive(int* counter, int home, int* s_slot) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have reached the L2
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool away = xcd_id() != home;
    if (away) __threadfence();
    *s_slot = __hip_atomic_fetch_add(counter, away ? 1 + kMisplaced : 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *s_slot;
}

// After the group is complete (`seen` = a counter value that includes every member): make the members' stores
// visible to this workgroup's loads.  Call from every thread; ends with a barrier.
DSV41_DEV void group_acquire(int seen, int home) {
  if (threadIdx.x == 0 && (seen >= kMisplaced || xcd_id() != home)) __threadfence();
  __syncthreads();
}

#define DSV41_CHECK_LAUNCH()                          \
  do {                                                \
    hipError_t _e = hipGetLastError();                \
    if (_e != hipSuccess) return (int)_e;             \
  } while (0)
