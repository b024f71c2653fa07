// FP8 block-scaled projections around the attention path (wq_a, wq_b, wkv, wo_a block-diagonal, wo_b; the
// fp8_gemm_tc / fp8_gemv_m1 operators of dsv41/cukern.py:116-200 with the weight format of dsv41/w8.py:19-60):
//   out[m, n] = sum_k x[row(m, n), k] * e4m3(W[n, k]) * 2^(S[n / 32, k / 32] - 127)
// x bf16, fp32 accumulation, bf16 output (optionally fp32 too).  W is stored with the bytes of every 16-k group
// permuted (position p holds k = 16 (p / 16) + kPermK[p % 16]); S is E8M0 per [32 n x 32 k] block.  row(m, n) = m,
// or with group_cols > 0 (block-diagonal o-projection) m * (N / group_cols) + n / group_cols.
//
// A weight stream: every weight byte is read once per 64 output rows.  Workgroup = 4 waves x 16 columns (64
// columns) over a K slice; a lane loads 16 weight bytes (one 16-k group, inside one scale block) per 64-k window and
// converts them to bf16 with the block scale applied by the hardware (v_cvt_scalef32_pk_bf16_fp8: exact, the e4m3
// values times a power of two); the x slice is staged in LDS in the weights' byte order, so a bf16 MFMA (16 rows x
// 16 columns x 32 k) pairs every weight with its x element.  Split K: each slice writes fp32 partials with
// device-scope stores, and the last slice of a column tile to arrive (device-scope counter) sums them in slice order
// (deterministic) and writes the output.
// Few rows over small weights (the decode GEMVs) go to two kernels that need no split exchange: the narrow one
// (16 columns, 16 waves over the whole K) and the vector one (a few columns per workgroup, fp32 VALU dot products);
// the plan picks by rows and columns, from measurements.  All three are deterministic.
#include "common.h"
#include "rowop.h"

namespace {

constexpr int kGemmThreads = 256;             // 4 waves, 16 columns each
constexpr int kGemmCols = 64;                 // columns per workgroup
constexpr int kGemmLdsBf16 = 32 * 1024;       // staged x elements at most (64 KB of dynamic LDS)
constexpr int kPreMaxK = 2 * kGemmThreads * 32;  // prologue rows: two 32-element groups per thread
constexpr int kPermK[16] = {0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15};  // dsv41/w8.py:23

typedef __bf16 bf16x2g_t __attribute__((ext_vector_type(2)));

struct GemmArgs {
  const uint16_t* x;  // bf16 rows, row stride ldx
  long ldx;
  const uint8_t* w8;  // [N, K] e4m3 bits, 16-k groups permuted
  const uint8_t* s8;  // [ceil(N / 32), Kc] E8M0
  int M, N, K, Kc, group_cols;
  int m0;             // first output row of this launch (rows m0 .. m0 + M - 1)
  int splits, kslice; // K slices (kslice: multiple of 64)
  uint16_t* out;      // bf16 [rows, ldo]
  long ldo;
  float* outf;        // optional fp32 copy [rows, ldo]
  float* part;        // [splits, 16 * MT, N] fp32 partials (splits > 1)
  int* cnt;           // [column tiles] arrival counters (zero between launches)
  int pre;            // activation prologue on the one x row: 1 rmsnorm (norm_w, eps) + fp8 fake quant, 2 quant
  const uint16_t* norm_w;
  float eps;
};

DSV41_DEV float e8m0_scale(uint32_t s) { return s ? __uint_as_float(s << 23) : __uint_as_float(0x00400000u); }

// 4 e4m3 bytes -> 4 bf16 (2 words) times the scale.
DSV41_DEV void cvt4(uint32_t w, float sc, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, false));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, true));
}

template <int MT, bool PRE = false>
__global__ void __launch_bounds__(kGemmThreads) fp8_gemm_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint16_t xs[];  // [M rows][kl] in weight byte order (dynamic: M x kslice)
  __shared__ int s_last;
  constexpr int MR = 16 * MT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int ct = blockIdx.x, sp = blockIdx.y;
  const int n0 = ct * kGemmCols;
  const int k0 = sp * a.kslice, k1 = min(a.K, k0 + a.kslice), kl = k1 - k0;  // kl: multiple of 64
  const int xr_off = a.group_cols > 0 ? n0 / a.group_cols : 0;
  const int xr_mul = a.group_cols > 0 ? a.N / a.group_cols : 1;

  // ---- weight stream: lane (l16, g) owns column n0 + 16 wave + l16, bytes 16 g .. 16 g + 15 of every 64-k window;
  // the first windows' loads go out before x is staged (independent round trips overlap)
  const int n = n0 + wave * 16 + l16;
  const int nc = n < a.N ? n : a.N - 1;
  const uint8_t* wrow = a.w8 + (long)nc * a.K + k0 + 16 * g;
  const uint8_t* srow = a.s8 + (long)(nc >> 5) * a.Kc + ((k0 + 16 * g) >> 5);
  const int nw = kl / 64;
  constexpr int U = 4;  // windows per batch; two batches in flight
  uint4 wv[U];
  uint32_t sv[U];
  auto load_batch = [&](int w0, uint4 (&dw)[U], uint32_t (&ds)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + u < nw ? w0 + u : nw - 1;
      dw[u] = *(const uint4*)(wrow + 64 * w);
      ds[u] = srow[2 * w];
    }
  };
  load_batch(0, wv, sv);

  // ---- stage x[rows, k0..k1) into LDS in the weights' byte order (16-byte units: 8 elements = one half group)
  if constexpr (PRE) {  // one row, the prologue applied while staging (the arithmetic of dsv41_norm_quant)
    __shared__ float red[kGemmThreads / 64];
    // 32 x values (raw bf16 pairs) of one group, normalised with its norm weights (mode 1) and fake-quantised, into
    // LDS at dst in the weights' byte order
    auto finish = [&](const uint4 (&rx)[4], const uint4 (&rw)[4], float inv, uint16_t* dst) {
      float v[32];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t xx[4] = {rx[q].x, rx[q].y, rx[q].z, rx[q].w};
        const uint32_t ww[4] = {rw[q].x, rw[q].y, rw[q].z, rw[q].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[8 * q + 2 * e] = __uint_as_float(xx[e] << 16);
          v[8 * q + 2 * e + 1] = __uint_as_float(xx[e] & 0xffff0000u);
          if (a.pre == 1) {
            v[8 * q + 2 * e] = round_bf16(v[8 * q + 2 * e] * inv * __uint_as_float(ww[e] << 16));
            v[8 * q + 2 * e + 1] = round_bf16(v[8 * q + 2 * e + 1] * inv * __uint_as_float(ww[e] & 0xffff0000u));
          }
        }
      }
      float amax = 0.0f;
#pragma unroll
      for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
      const float sc = fq_scale(amax, 0);
      const float rs = __fdiv_rn(1.0f, sc);  // sc is a power of two: x * rs == x / sc exactly
      uint16_t b[32];
#pragma unroll
      for (int e = 0; e < 32; ++e) b[e] = f2bf(round_e4m3(fminf(fmaxf(v[e] * rs, -448.0f), 448.0f)) * sc);
      uint32_t o[16];  // position p of each 16-k group holds k = kPermK[p]
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j2 = 0; j2 < 8; ++j2)
          o[8 * h + j2] = (uint32_t)b[16 * h + kPermK[2 * j2]] | ((uint32_t)b[16 * h + kPermK[2 * j2 + 1]] << 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) *(uint4*)(dst + 8 * q) = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    };
    auto load_grp = [&](int grp, uint4 (&rx)[4], uint4 (&rw)[4]) {  // x and (mode 1) norm weights of a group
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        rx[q] = ((const uint4*)(a.x + 32 * grp))[q];
        rw[q] = a.pre == 1 ? ((const uint4*)(a.norm_w + 32 * grp))[q] : make_uint4(0, 0, 0, 0);
      }
    };
    const int ng = a.K / 32;
    const bool whole = k0 == 0 && kl == a.K;  // the slice is the row: the groups loaded for the norm are staged
    uint4 rx[2][4], rw[2][4];
    float inv = 1.0f;
    if (a.pre == 1 || whole) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int grp = tid + kGemmThreads * q;
        if (grp < ng) load_grp(grp, rx[q], rw[q]);
        else
#pragma unroll
          for (int e = 0; e < 4; ++e) rx[q][e] = rw[q][e] = make_uint4(0, 0, 0, 0);
      }
    }
    if (a.pre == 1) {  // whole-row sum of squares, in the order of the norm_quant kernel
      float ss = 0.0f;
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t xx[4] = {rx[q][u].x, rx[q][u].y, rx[q][u].z, rx[q][u].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(xx[e] << 16), hi = __uint_as_float(xx[e] & 0xffff0000u);
            ss += lo * lo;
            ss += hi * hi;
          }
        }
      ss = block_sum<kGemmThreads>(ss, red);
      inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)a.K) + a.eps));
    }
    if (whole) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int grp = tid + kGemmThreads * q;
        if (grp < ng) finish(rx[q], rw[q], inv, xs + 32 * grp);
      }
    } else {
#pragma unroll 1
      for (int u = tid; u < kl / 32; u += kGemmThreads) {
        uint4 gx[4], gw[4];
        load_grp(k0 / 32 + u, gx, gw);
        finish(gx, gw, inv, xs + 32 * u);
      }
    }
  } else {
    const int units = a.M * (kl / 8);
#pragma unroll 1
    for (int u = tid; u < units; u += kGemmThreads) {
      const int m = u / (kl / 8), p8 = (u - m * (kl / 8)) * 8;  // byte position p8 .. p8 + 7
      const int gm = a.m0 + m;
      uint32_t v[4];
      const uint16_t* xrow = a.x + (long)(gm * xr_mul + xr_off) * a.ldx + k0 + (p8 & ~15);
      const int h = (p8 & 8) ? 8 : 0;  // positions h..h+7 of the group hold k = kPermK[h..h+7]: pairs (2j, 2j+1)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = *(const uint32_t*)(xrow + kPermK[h + 2 * j]);
      *(uint4*)(xs + m * kl + p8) = make_uint4(v[0], v[1], v[2], v[3]);
    }
  }
  __syncthreads();

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int w0 = 0; w0 < nw; w0 += U) {
    uint4 wn[U];
    uint32_t sn[U];
    if (w0 + U < nw) load_batch(w0 + U, wn, sn);  // the next batch in flight while this one is used
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (w0 + u >= nw) break;
      const float sc = e8m0_scale(sv[u]);
      uint32_t b[8];
      cvt4(wv[u].x, sc, b[0], b[1]);
      cvt4(wv[u].y, sc, b[2], b[3]);
      cvt4(wv[u].z, sc, b[4], b[5]);
      cvt4(wv[u].w, sc, b[6], b[7]);
      const uint4 b0 = make_uint4(b[0], b[1], b[2], b[3]), b1 = make_uint4(b[4], b[5], b[6], b[7]);
      const int p = 64 * (w0 + u) + 16 * g;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {  // (rows past M: zero operands, nothing staged)
        const bool rv = 16 * mt + l16 < a.M;
        const uint16_t* xa = xs + (rv ? 16 * mt + l16 : 0) * kl + p;
        const uint4 z = make_uint4(0, 0, 0, 0);
        acc[mt] = mfma_bf16_16x16x32(rv ? *(const uint4*)xa : z, b0, acc[mt]);
        acc[mt] = mfma_bf16_16x16x32(rv ? *(const uint4*)(xa + 8) : z, b1, acc[mt]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      wv[u] = wn[u];
      sv[u] = sn[u];
    }
  }
  // lane (l16, g) holds out[16 mt + 4 g + i][n]
  auto store = [&](int m, float v) {
    if (m < a.M && n < a.N) {
      const long o = (long)(a.m0 + m) * a.ldo + n;
      a.out[o] = f2bf(v);
      if (a.outf) a.outf[o] = v;
    }
  };
  if (a.splits == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) store(16 * mt + 4 * g + i, acc[mt][i]);
    return;
  }
  // ---- split K: partials out with device-scope stores, the last slice of the column tile reduces
  float* pb = a.part + (long)sp * MR * a.N;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n < a.N)
        __hip_atomic_store(pb + (long)(16 * mt + 4 * g + i) * a.N + n, acc[mt][i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(a.cnt + ct, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == a.splits - 1;
    if (s_last) __hip_atomic_store(a.cnt + ct, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  // thread t: column n0 + t % 64, rows t / 64, + 4, ...
  const int cn = n0 + (tid & 63);
  if (cn >= a.N) return;
#pragma unroll 1
  for (int m = tid >> 6; m < min(MR, a.M); m += 4) {
    float v = 0.0f;
#pragma unroll 4
    for (int s = 0; s < a.splits; ++s)
      v += __hip_atomic_load(a.part + ((long)s * MR + m) * a.N + cn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const long o = (long)(a.m0 + m) * a.ldo + cn;
    a.out[o] = f2bf(v);
    if (a.outf) a.outf[o] = v;
  }
}

// Narrow variant for few rows and few columns (the decode GEMVs whose weights are too small to fill the chip with
// 64-column tiles and no split exchange): a workgroup of 16 waves owns 16 columns over the whole K, wave v takes the
// 64-k windows v, v + 16, ...  Lane (l16, g) loads, per window, its 16 weight bytes and the 16 x elements of the same
// 16-k group of row l16 (32 contiguous bytes, put into the weights' byte order in registers), all of a batch in
// flight at once; the waves' partial sums meet in LDS (fixed order: deterministic).  Rows <= 16.
constexpr int kNarrowWaves = 16;
constexpr int kNarrowThreads = 64 * kNarrowWaves;
constexpr int kNarrowU = 6;  // windows per lane per batch (6 x 52 bytes of loads in registers: no spill at 1024 threads)
// Measured against the 64-column split kernel (graph replay, weights past the last-level cache): narrow wins for
// N = 1280 (7.6 vs 9.3 us at K 5120), 2048 and 4096 (8.2 vs 10.0 us at K 4096); it loses below 1024 columns
// (N = 512, K 5120: 7.5 vs 7.2 us; too few workgroups) and from 5120 up (the split kernel's 64-column tiles)
constexpr int kNarrowMinN = 1024, kNarrowMaxN = 4096;

__global__ void __launch_bounds__(kNarrowThreads) fp8_gemv_narrow_kernel(const GemmArgs a) {
  __shared__ f32x4_t red[kNarrowWaves][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int xr_off = a.group_cols > 0 ? n0 / a.group_cols : 0;
  const int xr_mul = a.group_cols > 0 ? a.N / a.group_cols : 1;
  const int n = n0 + l16;
  const int nc = n < a.N ? n : a.N - 1;
  const uint8_t* wrow = a.w8 + (long)nc * a.K + 16 * g;
  const uint8_t* srow = a.s8 + (long)(nc >> 5) * a.Kc + (g >> 1);
  const bool rv = l16 < a.M;
  const uint16_t* xrow = a.x + (long)((a.m0 + (rv ? l16 : 0)) * xr_mul + xr_off) * a.ldx + 16 * g;
  const int nwin = a.K / 64;
  const int mine = nwin > wave ? (nwin - wave + kNarrowWaves - 1) / kNarrowWaves : 0;  // this wave's windows
  uint4 wv[kNarrowU], x0[kNarrowU], x1[kNarrowU];
  uint32_t sv[kNarrowU];
  auto load_batch = [&](int j0) {
#pragma unroll
    for (int u = 0; u < kNarrowU; ++u) {
      const int j = j0 + u < mine ? j0 + u : mine - 1;
      const int w = wave + kNarrowWaves * j;
      wv[u] = *(const uint4*)(wrow + 64 * w);
      sv[u] = srow[2 * w];
      if (rv) {
        x0[u] = *(const uint4*)(xrow + 64 * w);
        x1[u] = *(const uint4*)(xrow + 64 * w + 8);
      }
    }
  };
  if (mine > 0) load_batch(0);
  f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int j0 = 0; j0 < mine; j0 += kNarrowU) {
#pragma unroll
    for (int u = 0; u < kNarrowU; ++u) {
      if (j0 + u >= mine) break;
      const float sc = e8m0_scale(sv[u]);
      uint32_t b[8];
      cvt4(wv[u].x, sc, b[0], b[1]);
      cvt4(wv[u].y, sc, b[2], b[3]);
      cvt4(wv[u].z, sc, b[4], b[5]);
      cvt4(wv[u].w, sc, b[6], b[7]);
      // x element pairs (2i, 2i + 1) of the group: x0 = pairs 0-3, x1 = pairs 4-7; byte order (kPermK) puts
      // pairs 0 4 1 5 in the first half and 2 6 3 7 in the second
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 a0 = rv ? make_uint4(x0[u].x, x1[u].x, x0[u].y, x1[u].y) : z;
      const uint4 a1 = rv ? make_uint4(x0[u].z, x1[u].z, x0[u].w, x1[u].w) : z;
      acc = mfma_bf16_16x16x32(a0, make_uint4(b[0], b[1], b[2], b[3]), acc);
      acc = mfma_bf16_16x16x32(a1, make_uint4(b[4], b[5], b[6], b[7]), acc);
    }
    if (j0 + kNarrowU < mine) load_batch(j0 + kNarrowU);
  }
  red[wave][lane] = acc;  // lane (l16, g): out[4 g + i][n0 + l16]
  __syncthreads();
  if (tid < 256) {
    const int ln = tid & 63, i = tid >> 6;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kNarrowWaves; ++w) v += red[w][ln][i];
    const int m = 4 * (ln >> 4) + i, cn = n0 + (ln & 15);
    if (m < a.M && cn < a.N) {
      const long o = (long)(a.m0 + m) * a.ldo + cn;
      a.out[o] = f2bf(v);
      if (a.outf) a.outf[o] = v;
    }
  }
}

// Vector (no MFMA) variant for up to 4 rows: CPW columns per 256-thread workgroup, 256 / CPW threads per column,
// thread t of a column takes the 16-k groups t, t + 256 / CPW, ... (every load of the thread in flight at once,
// up to kVecG groups per batch): 16 weight bytes decoded to fp32 with the block scale (v_cvt_scalef32_pk_f32_fp8,
// exact) against the group's 16 x elements, then the column's threads reduce (wave shuffles, then LDS; fixed
// order).  Spreads a small weight over every CU: each workgroup streams CPW x K bytes.
constexpr int kVecThreads = 256;
constexpr int kVecG = 4;
constexpr int kVecMaxM = 4;
typedef float f32x2v_t __attribute__((ext_vector_type(2)));

template <int CPW>
__global__ void __launch_bounds__(kVecThreads) fp8_gemv_vec_kernel(const GemmArgs a) {
  constexpr int TPC = kVecThreads / CPW;    // threads per column
  constexpr int WPC = TPC >= 64 ? TPC / 64 : 1;  // waves per column (a wave holds 64 / TPC columns below 64)
  constexpr int SH = TPC >= 64 ? 64 : TPC;  // lanes of one column inside a wave
  __shared__ float red[CPW][WPC][kVecMaxM];
  const int tid = threadIdx.x;
  const int cl = tid / TPC, t = tid - cl * TPC;
  const int n = blockIdx.x * CPW + cl;
  const int nc = n < a.N ? n : a.N - 1;
  const int xr_off = a.group_cols > 0 ? nc / a.group_cols : 0;
  const int xr_mul = a.group_cols > 0 ? a.N / a.group_cols : 1;
  const uint8_t* wrow = a.w8 + (long)nc * a.K;
  const uint8_t* srow = a.s8 + (long)(nc >> 5) * a.Kc;
  const uint16_t* xrow[kVecMaxM];
#pragma unroll
  for (int m = 0; m < kVecMaxM; ++m)
    xrow[m] = a.x + (long)((a.m0 + (m < a.M ? m : 0)) * xr_mul + xr_off) * a.ldx;
  const int ng = a.K / 16;
  const int mine = ng > t ? (ng - t + TPC - 1) / TPC : 0;
  float acc[kVecMaxM] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int j0 = 0; j0 < mine; j0 += kVecG) {
    uint4 wv[kVecG], xv[kVecG][kVecMaxM][2];
    uint32_t sv[kVecG];
#pragma unroll
    for (int u = 0; u < kVecG; ++u) {
      const int j = j0 + u < mine ? j0 + u : mine - 1;
      const int grp = t + TPC * j;
      wv[u] = *(const uint4*)(wrow + 16 * grp);
      sv[u] = srow[grp >> 1];
#pragma unroll
      for (int m = 0; m < kVecMaxM; ++m)
        if (m < a.M) {
          xv[u][m][0] = *(const uint4*)(xrow[m] + 16 * grp);
          xv[u][m][1] = *(const uint4*)(xrow[m] + 16 * grp + 8);
        }
    }
#pragma unroll
    for (int u = 0; u < kVecG; ++u) {
      if (j0 + u >= mine) break;
      const float sc = e8m0_scale(sv[u]);
      // weight word i (bytes 4i .. 4i + 3) holds k = (2i, 2i + 1) and (2i + 8, 2i + 9) of the group
      const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x2v_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[i], sc, false);
        const f32x2v_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[i], sc, true);
#pragma unroll
        for (int m = 0; m < kVecMaxM; ++m) {
          if (m >= a.M) break;
          const uint32_t* xw0 = (const uint32_t*)&xv[u][m][0];
          const uint32_t* xw1 = (const uint32_t*)&xv[u][m][1];
          const uint32_t pl = xw0[i], ph = xw1[i];  // x pairs (2i, 2i + 1) and (2i + 8, 2i + 9)
          acc[m] += lo.x * bf2f((uint16_t)pl) + lo.y * bf2f((uint16_t)(pl >> 16)) + hi.x * bf2f((uint16_t)ph) +
                    hi.y * bf2f((uint16_t)(ph >> 16));
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kVecMaxM; ++m) {
    float v = acc[m];
#pragma unroll
    for (int o = SH / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    acc[m] = v;
  }
  if ((t & (SH - 1)) == 0)
#pragma unroll
    for (int m = 0; m < kVecMaxM; ++m) red[cl][t / SH][m] = acc[m];
  __syncthreads();
  if (t < kVecMaxM && t < a.M && n < a.N) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WPC; ++w) v += red[cl][w][t];
    const long o = (long)(a.m0 + t) * a.ldo + n;
    a.out[o] = f2bf(v);
    if (a.outf) a.outf[o] = v;
  }
}

// Plan: row tiles of up to 64 rows (MT = 1, 2, 4), K slices so that the grid holds >= 512 workgroups when K allows
// (slices >= 256 k) and the staged x fits LDS.
struct GemmPlan {
  int MT, splits, kslice, ctiles;
  bool narrow;  // fp8_gemv_narrow_kernel: 16-column workgroups over the whole K, no split
  int vec_cpw;  // > 0: fp8_gemv_vec_kernel with this many columns per workgroup
};

GemmPlan gemm_plan(int M, int N, int K, bool narrow_ok) {
  GemmPlan p{};
  p.narrow = narrow_ok && M <= 16 && N >= kNarrowMinN && N <= kNarrowMaxN;
  // vector kernel (measured, graph replay, K 5120 / 4096): one row N <= 1024 two columns per workgroup (N = 512:
  // 4.2 us; 64-column split 7.2), <= 2048 four (N = 1280: 6.3 us; narrow 7.6), <= 4096 eight (7.6; narrow 8.3);
  // 2-4 rows N <= 1024 two (N = 512, 4 rows: 5.6 us; split 7.8), beyond that narrow (N = 1280, 4 rows: 8.8; vector 9.6)
  p.vec_cpw = 0;
  if (narrow_ok && M == 1) p.vec_cpw = N <= 1024 ? 2 : N <= 2048 ? 4 : N <= 4096 ? 8 : 0;
  else if (narrow_ok && M <= kVecMaxM && N <= 1024) p.vec_cpw = 2;
  if (p.vec_cpw) {
    p.narrow = false;
    p.MT = 1;
    p.ctiles = (N + p.vec_cpw - 1) / p.vec_cpw;
    p.splits = 1;
    p.kslice = K;
    return p;
  }
  if (p.narrow) {
    p.MT = 1;
    p.ctiles = (N + 15) / 16;
    p.splits = 1;
    p.kslice = K;
    return p;
  }
  const int mrows = M < 64 ? M : 64;
  p.MT = mrows <= 16 ? 1 : mrows <= 32 ? 2 : 4;
  p.ctiles = (N + kGemmCols - 1) / kGemmCols;
  const int kmax = kGemmLdsBf16 / mrows / 64 * 64;  // staged elements per row
  int s = (K + kmax - 1) / kmax;
  while ((long)p.ctiles * s < 512 && K / (2 * s) >= 256) s *= 2;
  int ks = (K + s - 1) / s;
  ks = (ks + 63) / 64 * 64;
  p.kslice = ks;
  p.splits = (K + ks - 1) / ks;
  return p;
}

}  // namespace

extern "C" {

long dsv41_fp8_gemm_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const GemmPlan p = gemm_plan(M, N, K, false);  // the largest need: the narrow kernel uses none
  if (p.splits == 1) return 0;
  return (long)p.ctiles * 4 + 12 + (long)p.splits * 16 * p.MT * N * 4;  // counters, pad, partials
}

int dsv41_fp8_gemm(const void* x, long ldx, const void* w8, const void* s8, int M, int N, int K, int Kc,
                   int group_cols, void* out, long ldo, float* out_f32, void* ws, long ws_bytes, void* stream) {
  if (M <= 0 || N <= 0) return 0;
  if (K <= 0 || K % 64 != 0 || Kc < K / 32 || !x || !w8 || !s8 || !out || ldo < N || ldx < K || ldx % 2 != 0 ||
      ((uintptr_t)x & 3) != 0 || ((uintptr_t)w8 & 15) != 0 ||
      (group_cols > 0 && (group_cols % kGemmCols != 0 || N % group_cols != 0)) || group_cols < 0)
    return (int)hipErrorInvalidValue;
  // the narrow kernel loads x in 16-byte units
  const GemmPlan p = gemm_plan(M, N, K, ((uintptr_t)x & 15) == 0 && ldx % 8 == 0);
  if (p.splits > 1 && (!ws || ws_bytes < dsv41_fp8_gemm_workspace_bytes(M, N, K))) return (int)hipErrorInvalidValue;
  GemmArgs a{};
  a.x = (const uint16_t*)x;
  a.ldx = ldx;
  a.w8 = (const uint8_t*)w8;
  a.s8 = (const uint8_t*)s8;
  a.N = N;
  a.K = K;
  a.Kc = Kc;
  a.group_cols = group_cols;
  a.splits = p.splits;
  a.kslice = p.kslice;
  a.out = (uint16_t*)out;
  a.ldo = ldo;
  a.outf = out_f32;
  if (p.splits > 1) {
    a.cnt = (int*)ws;
    a.part = (float*)((char*)ws + ((long)p.ctiles * 4 + 15) / 16 * 16);
  }
  hipStream_t st = (hipStream_t)stream;
  if (p.vec_cpw) {
    a.m0 = 0;
    a.M = M;
    if (p.vec_cpw == 1) fp8_gemv_vec_kernel<1><<<p.ctiles, kVecThreads, 0, st>>>(a);
    else if (p.vec_cpw == 2) fp8_gemv_vec_kernel<2><<<p.ctiles, kVecThreads, 0, st>>>(a);
    else if (p.vec_cpw == 4) fp8_gemv_vec_kernel<4><<<p.ctiles, kVecThreads, 0, st>>>(a);
    else fp8_gemv_vec_kernel<8><<<p.ctiles, kVecThreads, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  if (p.narrow) {
    a.m0 = 0;
    a.M = M;
    fp8_gemv_narrow_kernel<<<p.ctiles, kNarrowThreads, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  const dim3 grid(p.ctiles, p.splits);
  for (int m0 = 0; m0 < M; m0 += 16 * p.MT) {  // row tiles (more than 64 rows: the weights stream once per 64)
    a.m0 = m0;
    a.M = M - m0 < 16 * p.MT ? M - m0 : 16 * p.MT;
    const size_t lds = (size_t)a.M * p.kslice * 2;
    if (p.MT == 1) fp8_gemm_kernel<1><<<grid, kGemmThreads, lds, st>>>(a);
    else if (p.MT == 2) fp8_gemm_kernel<2><<<grid, kGemmThreads, lds, st>>>(a);
    else fp8_gemm_kernel<4><<<grid, kGemmThreads, lds, st>>>(a);
    DSV41_CHECK_LAUNCH();
  }
  return 0;
}

int dsv41_fp8_gemv_m1_pre(const void* x_raw, const void* norm_w, float eps, int mode, const void* w8, const void* s8,
                          int N, int K, int Kc, void* out, void* ws, long ws_bytes, void* stream) {
  if (N <= 0) return 0;
  if ((mode != 1 && mode != 2) || (mode == 1 && !norm_w) || K <= 0 || K % 64 != 0 || K > kPreMaxK || Kc < K / 32 ||
      !x_raw || !w8 || !s8 || !out || ((uintptr_t)x_raw & 15) != 0 || ((uintptr_t)w8 & 15) != 0 ||
      (mode == 1 && ((uintptr_t)norm_w & 15) != 0))
    return (int)hipErrorInvalidValue;
  const GemmPlan p = gemm_plan(1, N, K, false);  // the 64-column kernel stages x: the prologue runs there
  if (p.splits > 1 && (!ws || ws_bytes < dsv41_fp8_gemm_workspace_bytes(1, N, K))) return (int)hipErrorInvalidValue;
  GemmArgs a{};
  a.x = (const uint16_t*)x_raw;
  a.ldx = K;
  a.w8 = (const uint8_t*)w8;
  a.s8 = (const uint8_t*)s8;
  a.M = 1;
  a.N = N;
  a.K = K;
  a.Kc = Kc;
  a.splits = p.splits;
  a.kslice = p.kslice;
  a.out = (uint16_t*)out;
  a.ldo = N;
  a.pre = mode;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  if (p.splits > 1) {
    a.cnt = (int*)ws;
    a.part = (float*)((char*)ws + ((long)p.ctiles * 4 + 15) / 16 * 16);
  }
  fp8_gemm_kernel<1, true><<<dim3(p.ctiles, p.splits), kGemmThreads, (size_t)p.kslice * 2, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
