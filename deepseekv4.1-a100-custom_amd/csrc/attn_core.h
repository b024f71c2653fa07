// Shared pieces of the sparse attention kernels (attn.hip) and the one-launch decode step (step.hip): the launch
// arguments, bf16 packing, the bf16 16x16x16 MFMA, the LDS transpose read, the zero gather row and the cooperative
// merge of split partials.
#pragma once
#include "common.h"

namespace {

struct AttnArgs {
  const uint16_t* q;  // [R, H, DQK]
  long q_rstride;     // elements between query rows
  int H, R;
  int mode;  // 0: explicit index list over [kv1 | kv2]; 1: ring (kv1, W = n1 rows) then compressed rows kv2[idx]
  const uint16_t* kv1;
  long kv1_sstride;  // elements between slots
  int n1;
  const uint16_t* kv2;
  long kv2_sstride;
  int n2;
  const int* idx;
  long idx_rstride;
  int t;
  int rows_per_slot;  // explicit mode: slot = r / rows_per_slot
  const long* pos;
  const long* seq;
  const long* pmax;
  const long* plim;
  float scale;
  const float* sink;
  int L;      // key positions per query row
  int chunk;  // key positions per split (multiple of 32)
  int nsplit;
  uint16_t* out;  // [R, H, DV] when nsplit == 1
  long out_rstride;
  float* pm;  // [R, H, nsplit]
  float* pl;
  float* pacc;  // [R, H, nsplit, DV]
  int* arrive;  // decode kernel: [R * head groups] split arrival counters (zero between launches), or null
  unsigned long long* coop;  // with arrive, when every workgroup is resident at once: [R * head groups] counters
                             // (launch epoch * 256 + arrivals), every split merges a slice; else null
  int* err;     // with arrive: the workspace error word (set to 1 when a merge stopped waiting for its unit)
  int units;    // with arrive: (row, 16-head group) units, placed upx per XCD (1-D grid of kXcds * upx * nsplit)
  int hg_share; // with coop: the head groups of a (row, split) placed on one XCD instead
  int dec32;    // decode: the 32-head kernel (one gather round trip per split of <= 128 keys), cooperative merge
  int upx;
  const float* cos_t;
  const float* sin_t;
  int rd;
};

// Two floats to packed bf16 (round to nearest even), one v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
DSV41_DEV uint32_t pack_bf16x2(float a, float b) { return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b}); }

typedef __attribute__((ext_vector_type(4))) short s16x4_t;
DSV41_DEV f32x4_t mfma_bf16_16x16x16(uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                   0, 0, 0);
}

// Zero row used as the gather source of invalid key positions (p = 0 then multiplies exact zeros, as the
// reference's masked loads do).
__device__ __align__(16) uint16_t g_zero_row[1024];

// LDS transpose read (gfx950 ds_read_b64_tr_b16): within each group of 16 lanes, output lane i receives element
// (i % 4) of the 4-element (8-byte) reads of input lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12.
DSV41_DEV uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((ext_vector_type(4))) short s4;
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p);
  return __builtin_bit_cast(uint2, v);
}

// Cooperative merge, run by every split workgroup of a unit once all nsplit have published (merge_slice).  The
// partials were written with device-scope stores and are read with device-scope loads (coherent across the XCDs,
// wherever the unit's workgroups ran).  Weights as merge_splits.
// Device-scope (sc1) 16-byte accesses to the split partials of the cooperative merge: one request per 16 bytes, with
// the cache policy of device-scope atomics (coherent across the XCDs).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
constexpr int kCpolDevice = 16;  // sc1
DSV41_DEV __amdgpu_buffer_rsrc_t pacc_rsrc(const float* pacc) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)pacc, 0, 0x7fffffff, 0x00020000);
}

// One (head, 8-column group) element of the merged output.  MS: splits per batch of loads (one batch for up to MS
// splits: one round trip).
template <int DV, int MS>
DSV41_DEV void merge_elem(const AttnArgs& a, int r, int h, int c, long pr) {
  const int ns = a.nsplit, H = a.H;
  const long base = ((long)r * H + h) * ns;
  const __amdgpu_buffer_rsrc_t rs = pacc_rsrc(a.pacc);
  const float sink = a.sink[h];
  float M = -1e30f, den = 0.0f, num[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 1
  for (int s0 = 0; s0 < ns; s0 += MS) {  // (online over batches: the weights are rescaled to the running maximum)
    u32x4_t v[MS];
    float m[MS], l[MS];
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const bool ok = s0 + u < ns;
      const long pi = base + (ok ? s0 + u : 0);
      v[u] = ok ? __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((pi * DV + c) * 2), 0, kCpolDevice)
                : u32x4_t{0, 0, 0, 0};
      m[u] = ok ? __hip_atomic_load(a.pm + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -1e30f;
      l[u] = ok ? __hip_atomic_load(a.pl + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    }
    float Mb = M;
#pragma unroll
    for (int u = 0; u < MS; ++u) Mb = fmaxf(Mb, m[u]);
    const float f = exp2f((M - Mb) * kLog2e);
    den *= f;
#pragma unroll
    for (int q = 0; q < 8; ++q) num[q] *= f;
    M = Mb;
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const float w = s0 + u < ns ? l[u] * exp2f((m[u] - M) * kLog2e) : 0.0f;
      den += w;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t x = v[u][q];
        num[2 * q] += w * __uint_as_float(x << 16);
        num[2 * q + 1] += w * __uint_as_float(x & 0xffff0000u);
      }
    }
  }
  const float inv = 1.0f / (den + exp2f((sink - M) * kLog2e));
  uint32_t pk[4];
#pragma unroll
  for (int q = 0; q < 8; q += 2) {
    float re = round_bf16(num[q] * inv), im = round_bf16(num[q + 1] * inv);
    const int cc = c + q;
    if (a.rd > 0 && cc >= DV - a.rd) {
      const int jj = (cc - (DV - a.rd)) >> 1;
      const float cs = a.cos_t[pr * (a.rd / 2) + jj];
      const float sn = -a.sin_t[pr * (a.rd / 2) + jj];
      const float yr = re * cs - im * sn, yi = re * sn + im * cs;
      re = yr;
      im = yi;
    }
    pk[q / 2] = pack_bf16x2(re, im);
  }
  *(uint4*)(a.out + (long)r * a.out_rstride + (long)h * DV + c) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

// Every split workgroup sp of a unit of NH heads (h0 ..) merges (head, 8-column group) elements
// [sp*E/ns, (sp+1)*E/ns) of the unit's E = NH * DV / 8, one per thread (the host keeps E / ns <= the workgroup).
template <int DV, int NH = 16>
DSV41_DEV void merge_slice(const AttnArgs& a, int r, int h0, long pr, int sp) {
  constexpr int CG = DV / 8, E = NH * CG;
  const int ns = a.nsplit;
  const int e = (int)((long)sp * E / ns) + (int)threadIdx.x;
  if (e >= (int)((long)(sp + 1) * E / ns)) return;
  const int hh = e / CG, c = (e - hh * CG) * 8, h = h0 + hh;
  if (h >= a.H) return;
  if (ns <= 16)
    merge_elem<DV, 16>(a, r, h, c, pr);
  else
    merge_elem<DV, 32>(a, r, h, c, pr);
}

}  // namespace
