// Per-row cache-append numerics shared by the append kernels and the fused decode indexer: [rmsnorm -> bf16] ->
// [rope -> bf16] -> [fake quant] -> stores (+ an e4m3 copy with one power-of-two scale per row), and the e4m3
// preparation of the index queries.  A row operation runs on a whole block of NT threads; element e of a row lives
// in thread e % NT (iteration e / NT), so a quantisation group of 16/32 elements is 16/32 consecutive lanes of one
// wave (shuffle reductions) and a rope pair (2j, 2j+1) is a lane pair (xor 1).
#pragma once
#include "common.h"

namespace {

constexpr int kRowThreads = 256;
constexpr int kRowMaxD = 1024;  // rows up to 1024 elements

// mode 0: fp8 e4m3, pow2 scale (amax >= 1e-4);  1: fp4 e2m1, pow2 scale;  2: fp4 e2m1, e4m3-rounded scale.
DSV41_DEV float fq_scale(float amax, int mode) {
  if (mode == 0) return pow2i(ceil_log2_f(__fdiv_rn(fmaxf(amax, 1e-4f), 448.0f)));
  if (mode == 1) return pow2i(ceil_log2_f(__fdiv_rn(fmaxf(amax, 6.0f * 1.1754944e-38f), 6.0f)));
  return round_e4m3(__fdiv_rn(fmaxf(amax, 6.0f * 0.001953125f), 6.0f));
}

DSV41_DEV float fq_value(float x, float s, int mode) {
  // modes 0 and 1: s is a power of two in [2^-126, 2^126], so x / s is x times the exact reciprocal (both are the
  // correctly rounded x * 2^-e); mode 2 divides
  const float xs = mode == 2 ? __fdiv_rn(x, s) : x * __int_as_float(0x7f000000 - __float_as_int(s));
  if (mode == 0) return round_e4m3(fminf(fmaxf(xs, -448.0f), 448.0f)) * s;
  return round_e2m1(fminf(fmaxf(xs, -6.0f), 6.0f)) * s;
}

// Workgroup barrier; LB: an LDS-only barrier (does not wait for the block's outstanding global loads, e.g. loads
// issued for later work).
template <bool LB>
DSV41_DEV void row_barrier() {
  if constexpr (LB)
    lds_barrier();
  else
    __syncthreads();
}

// Block-wide sum / max of one float per thread (NT threads); red holds >= NT / 64 floats.  NT = 64: one wave's
// (no barrier; red unused), callable by a single wave of a larger block.
template <int NT, bool LB = false>
DSV41_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (NT == 64) return v;
  row_barrier<LB>();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  row_barrier<LB>();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) s += red[w];
  return s;
}

template <int NT, bool LB = false>
DSV41_DEV float block_max(float v, float* red) {
  v = group_max(v, 64);
  if constexpr (NT == 64) return v;
  row_barrier<LB>();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  row_barrier<LB>();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) s = fmaxf(s, red[w]);
  return s;
}

struct RowOp {
  const uint16_t* x;  // input row (bf16), D elements
  int D;
  const uint16_t* norm_w;  // rmsnorm weight (bf16) or null
  float eps;
  const float* cos_t;  // rope tables [pos][rd/2] (rd = 0: no rope)
  const float* sin_t;
  int rd;
  long pos;
  int qmode, group;  // fake quantisation (qmode < 0: none)
  uint16_t* out;     // bf16 destination row or null
  uint16_t* out2;    // second bf16 destination (temporary KV) or null
  uint8_t* k8;       // e4m3 destination row (per-row pow2 scale in *ks) or null
  float* ks;
  uint8_t* k8_lds;   // with k8: the same e4m3 row and scale also to these (shared memory) or null
  float* ks_lds;
};

// The operands of one row operation, loaded ahead of its arithmetic (row_load, then row_compute), for rows of up to
// MAXD elements.  The NT threads doing a row operation are a whole block, or (NT = 64) one wave of a larger block;
// element e lives in thread e % NT of the group.
// (the bf16 operands are held as loaded and converted in row_compute: a conversion next to the load would make the
// compiler wait for it there, before any loads issued after row_load)
template <int NT, int MAXD = kRowMaxD>
struct RowRegs {
  static constexpr int IT = MAXD / NT;
  uint32_t vb[IT], wb[IT];
  float cs[IT], sn[IT];
};

// Stand-ins read by row_load in place of a missing norm weight (bf16 1.0) or rope table.
__device__ uint16_t g_row_one_bf16 = 0x3f80u;
__device__ float g_row_zero_f32 = 0.0f;

// Every operand load is unconditional (absent operands read a stand-in, columns are clamped): a load under a
// condition would make the compiler wait for it where the branches merge, before any load issued after row_load.
template <int NT, int MAXD = kRowMaxD>
DSV41_DEV void row_load(const RowOp& o, RowRegs<NT, MAXD>& g) {
  const int t = threadIdx.x & (NT - 1);
  const int p = o.pos < 0 ? 0 : (int)o.pos;
  const bool nw = o.norm_w != nullptr, rp = o.rd > 0;
  const uint16_t* const wp = nw ? o.norm_w : &g_row_one_bf16;
  const float* const cp = rp ? o.cos_t : &g_row_zero_f32;
  const float* const sp = rp ? o.sin_t : &g_row_zero_f32;
#pragma unroll
  for (int u = 0; u < RowRegs<NT, MAXD>::IT; ++u) {
    const int e = t + u * NT;
    const int ec = e < o.D ? e : 0;
    g.vb[u] = o.x[ec];  // (elements e >= D are zeroed in row_compute)
    g.wb[u] = wp[nw ? ec : 0];
    // (elements outside the rope columns never use cs / sn)
    const bool rope = e < o.D && e >= o.D - o.rd;
    const long j = rp && rope ? (long)p * (o.rd / 2) + ((ec - (o.D - o.rd)) >> 1) : 0;
    g.cs[u] = cp[j];
    g.sn[u] = sp[j];
  }
}

// Every thread of the group (the block, or the one wave when NT = 64) must call it.  LB: LDS-only barriers inside.
template <int NT, bool LB = false, int MAXD = kRowMaxD>
DSV41_DEV void row_compute(const RowOp& o, RowRegs<NT, MAXD>& g, float* red) {
  constexpr int IT = RowRegs<NT, MAXD>::IT;
  const int t = threadIdx.x & (NT - 1);
  float v[IT];
#pragma unroll
  for (int u = 0; u < IT; ++u) v[u] = t + u * NT < o.D ? bf2f((uint16_t)g.vb[u]) : 0.0f;
  if (o.norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < IT; ++u) ss += v[u] * v[u];
    ss = block_sum<NT, LB>(ss, red);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)o.D) + o.eps));
#pragma unroll
    for (int u = 0; u < IT; ++u) v[u] = round_bf16(v[u] * inv * bf2f((uint16_t)g.wb[u]));
  }
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    if (u * NT >= o.D) break;
    if (o.rd > 0) {
      const float partner = dpp_mov<0xB1>(v[u]);  // lane ^ 1
      const int e = t + u * NT;
      if (e >= o.D - o.rd && e < o.D)
        v[u] = (e & 1) ? round_bf16(partner * g.sn[u] + v[u] * g.cs[u]) : round_bf16(v[u] * g.cs[u] - partner * g.sn[u]);
    }
    if (o.qmode >= 0) {
      const float a = group_max(fabsf(v[u]), o.group);
      v[u] = fq_value(v[u], fq_scale(a, o.qmode), o.qmode);
    }
    const int e = t + u * NT;
    if (e < o.D) {
      const uint16_t b = f2bf(v[u]);
      if (o.out) o.out[e] = b;
      if (o.out2) o.out2[e] = b;
    }
  }
  if (o.k8) {  // e4m3 copy of the stored bf16 values with one power-of-two scale per row
    float a = 0.0f;
#pragma unroll
    for (int u = 0; u < IT; ++u) a = fmaxf(a, fabsf(round_bf16(v[u])));
    a = block_max<NT, LB>(a, red);
    int ex = ceil_log2_f(__fdiv_rn(fmaxf(a, 1e-30f), 448.0f));
    ex = ex < -126 ? -126 : ex;
#pragma unroll
    for (int u = 0; u < IT; ++u) {
      const int e = t + u * NT;
      if (e < o.D) {
        const uint8_t b = (uint8_t)e4m3_bits(round_e4m3(fminf(fmaxf(round_bf16(v[u]) * pow2i(-ex), -448.0f), 448.0f)));
        o.k8[e] = b;
        if (o.k8_lds) lds_ptr(o.k8_lds)[e] = b;
      }
    }
    if (t == 0) {
      *o.ks = pow2i(ex);
      if (o.ks_lds) *lds_ptr(o.ks_lds) = pow2i(ex);
    }
  }
}

template <int NT = kRowThreads>
DSV41_DEV void row_op(const RowOp& o, float* red) {
  RowRegs<NT> g;
  row_load<NT>(o, g);
  row_compute<NT>(o, g, red);
}

// Index-query preparation for the fp8 score MFMA: per head h (<= 64 heads, 128 wide) a power-of-two scale
// 2^e = 2^ceil(log2(amax / 448)), q8[h] = e4m3(q[h] / 2^e) and wf[h] = w[h] * 2^e (the scale folds into the head
// weight because relu(s * x) = s * relu(x) for s > 0).  Exact for the reference's FP4-grid queries.
DSV41_DEV void qprep_op(const uint16_t* q, const uint16_t* w_bf16, const float* w_f32, int HI, uint8_t* q8,
                        float* wf) {
  const int t = threadIdx.x, h = t >> 2, part = t & 3;
  const int hc = h < HI ? h : HI - 1;
  const uint4* src = (const uint4*)(q + (long)hc * 128 + part * 32);
  uint4 raw[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) raw[u] = src[u];
  const float wv = w_bf16 ? bf2f(w_bf16[hc]) : w_f32[hc];
  float x[32];
  float amax = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t ww[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[u * 8 + 2 * e] = __uint_as_float(ww[e] << 16);
      x[u * 8 + 2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(x[e]));
  amax = group_max(amax, 4);
  int ex = ceil_log2_f(fmaxf(amax, 1e-30f) * (1.0f / 448.0f));
  ex = ex < -126 ? -126 : ex;
  const float inv = pow2i(-ex);
  uint32_t pk[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    int wd = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * d] * inv, x[4 * d + 1] * inv, 0, false);
    wd = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * d + 2] * inv, x[4 * d + 3] * inv, wd, true);
    pk[d] = (uint32_t)wd;
  }
  if (h < 64) {
    uint4* dst = (uint4*)(q8 + (long)h * 128 + part * 32);
    dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    if (part == 0) wf[h] = h < HI ? wv * pow2i(ex) : 0.0f;
  }
}


// The same preparation by a 512-thread block into shared memory: head h = t / 8, 16 elements per thread (the
// per-head maximum, scale and conversions are those of qprep_op, so the bytes are identical).  Loads and
// arithmetic are separate calls so that the loads can be issued ahead.
struct Qprep512 {
  uint4 raw[2];
  uint32_t wbits;  // the head weight's bf16 bits (converted where used: a conversion here would wait for the load)
};

DSV41_DEV void qprep512_load(const uint16_t* q, const uint16_t* w_bf16, int HI, Qprep512& g) {
  const int t = threadIdx.x, h = t >> 3, part = t & 7;
  const int hc = h < HI ? h : HI - 1;
  const uint4* src = (const uint4*)(q + (long)hc * 128 + part * 16);
  g.raw[0] = src[0];
  g.raw[1] = src[1];
  g.wbits = w_bf16[hc];
}

DSV41_DEV void qprep512_store(const Qprep512& g, int HI, uint8_t* q8, float* wf) {
  const int t = threadIdx.x, h = t >> 3, part = t & 7;
  float x[16];
  float amax = 0.0f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t ww[4] = {g.raw[u].x, g.raw[u].y, g.raw[u].z, g.raw[u].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[u * 8 + 2 * e] = __uint_as_float(ww[e] << 16);
      x[u * 8 + 2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(x[e]));
  amax = group_max(amax, 8);
  int ex = ceil_log2_f(fmaxf(amax, 1e-30f) * (1.0f / 448.0f));
  ex = ex < -126 ? -126 : ex;
  const float inv = pow2i(-ex);
  uint32_t pk[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    int wd = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * d] * inv, x[4 * d + 1] * inv, 0, false);
    wd = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * d + 2] * inv, x[4 * d + 3] * inv, wd, true);
    pk[d] = (uint32_t)wd;
  }
  *(uint4*)(q8 + h * 128 + part * 16) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  if (part == 0) wf[h] = h < HI ? bf2f((uint16_t)g.wbits) * pow2i(ex) : 0.0f;
}

bool row_ok(int D, int group) {
  return D > 0 && D <= kRowMaxD && (group <= 0 || D % group == 0) && D % 2 == 0;
}

}  // namespace
