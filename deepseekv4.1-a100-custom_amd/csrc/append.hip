// Cache-append kernels of the sparse-attention path and the small per-row numerics they fuse:
//   dsv41_kv_write      SWA ring append (rmsnorm -> bf16 -> rope -> bf16 -> fq8/32 -> ring[seq, pos % W])
//   dsv41_append_rows   compressed-KV / index-key append (optional rmsnorm, rope, fq4 or fq8, optional e4m3 sidecar)
//   dsv41_fake_quant    standalone fake quantisation (fp8 pow2 / fp4 pow2 / fp4 e4m3-scale)
//   dsv41_rope          in-place rotary on the last rd columns (host or device positions)
//   dsv41_rmsnorm       standalone rmsnorm
// One workgroup of 64 lanes (one wave) per row: rows are <= 576 wide, so a wave owns a row and every reduction is
// a cross-lane shuffle; per-32/16 groups map onto lane groups.  These are tiny HBM-bound kernels.
#include "common.h"

namespace {

constexpr int kMaxD = 1024;  // widest row handled (elements); each lane holds kMaxD/64 = 16 values

// Reduction over the 64 lanes of a wave.
DSV41_DEV float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += wave_shfl_xor(v, m);
  return v;
}

// Lane l owns columns [l*per, (l+1)*per) of the row (per = PER, chosen by pick_per); lanes past the row hold zeros.

// Group amax across the lanes sharing a quantisation group of `group` columns (group = 16 or 32, per | group or
// group | per).
DSV41_DEV float group_amax(float local, int per, int group) {
  float a = local;
  if (per < group) {
    const int lanes = group / per;  // 2..32, power of two
    for (int m = 1; m < lanes; m <<= 1) a = fmaxf(a, wave_shfl_xor(a, m));
  }
  return a;
}

// mode 0: fp8 e4m3, pow2 scale (amax >= 1e-4);  1: fp4 e2m1, pow2 scale;  2: fp4 e2m1, e4m3-rounded scale.
DSV41_DEV float fq_scale(float amax, int mode) {
  if (mode == 0) return pow2i(ceil_log2_f(__fdiv_rn(fmaxf(amax, 1e-4f), 448.0f)));
  if (mode == 1) return pow2i(ceil_log2_f(__fdiv_rn(fmaxf(amax, 6.0f * 1.1754944e-38f), 6.0f)));
  return round_e4m3(__fdiv_rn(fmaxf(amax, 6.0f * 0.001953125f), 6.0f));
}

DSV41_DEV float fq_value(float x, float s, int mode) {
  if (mode == 0) return round_e4m3(fminf(fmaxf(__fdiv_rn(x, s), -448.0f), 448.0f)) * s;
  return round_e2m1(fminf(fmaxf(__fdiv_rn(x, s), -6.0f), 6.0f)) * s;
}

// Quantise the lane's `per` contiguous values in place (groups of `group` columns).
template <int PER>
DSV41_DEV void fake_quant_lane(float (&v)[PER], int per, int group, int mode) {
  if (per <= group) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) if (i < per) a = fmaxf(a, fabsf(v[i]));
    a = group_amax(a, per, group);
    const float s = fq_scale(a, mode);
#pragma unroll
    for (int i = 0; i < PER; ++i) if (i < per) v[i] = fq_value(v[i], s, mode);
  } else {  // several groups inside one lane
    for (int g0 = 0; g0 < per; g0 += group) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < PER; ++i) if (i >= g0 && i < g0 + group) a = fmaxf(a, fabsf(v[i]));
      const float s = fq_scale(a, mode);
#pragma unroll
      for (int i = 0; i < PER; ++i) if (i >= g0 && i < g0 + group) v[i] = fq_value(v[i], s, mode);
    }
  }
}

// Rotate the interleaved (re, im) pairs of the last rd columns at position pos; values stay fp32 and are
// rounded to bf16 (the reference stores each rotated component as bf16).  `per` is even, so pairs never straddle
// lanes.
template <int PER>
DSV41_DEV void rope_lane(float (&v)[PER], int lane, int per, int D, int rd, const float* cos_t, const float* sin_t,
                         long pos, bool inverse) {
  const int c0 = lane * per;
#pragma unroll
  for (int i = 0; i < PER; i += 2) {
    const int c = c0 + i;
    if (i < per && c >= D - rd && c < D) {
      const int j = (c - (D - rd)) >> 1;
      const float cs = cos_t[pos * (rd / 2) + j];
      float sn = sin_t[pos * (rd / 2) + j];
      if (inverse) sn = -sn;
      const float xr = v[i], xi = v[i + 1];
      v[i] = round_bf16(xr * cs - xi * sn);
      v[i + 1] = round_bf16(xr * sn + xi * cs);
    }
  }
}

template <int PER>
DSV41_DEV void load_row(float (&v)[PER], const uint16_t* x, int lane, int per, int D) {
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane * per + i;
    v[i] = (i < per && c < D) ? bf2f(x[c]) : 0.0f;
  }
}

template <int PER>
DSV41_DEV void rmsnorm_lane(float (&v)[PER], int lane, int per, int D, const uint16_t* w, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) ss += v[i] * v[i];
  ss = wave_sum(ss);
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)D) + eps));
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane * per + i;
    if (i < per && c < D) v[i] = round_bf16(v[i] * inv * bf2f(w[c]));
  }
}

// ---------------------------------------------------------------------------------------------- kv_write
// Row r: x[r] -> ring[seq[r], pos[r] % W] (and, when tmp != null, tmp[r]).  pos/seq may be null: then
// pos = pos0 + r*pos_stride and seq = r / rows_per_seq.
template <int PER>
__global__ void __launch_bounds__(64) kv_write_kernel(const uint16_t* __restrict__ x, long x_rstride,
                                                      const uint16_t* __restrict__ w, const float* __restrict__ cos_t,
                                                      const float* __restrict__ sin_t, const long* __restrict__ pos,
                                                      const long* __restrict__ seq, long pos0, long pos_stride,
                                                      int rows_per_seq, uint16_t* __restrict__ cache,
                                                      long cache_sstride, int W, uint16_t* __restrict__ tmp, int D,
                                                      int rd, float eps, int commit_from) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int per = PER;
  float v[PER];
  load_row<PER>(v, x + (long)r * x_rstride, lane, per, D);
  rmsnorm_lane<PER>(v, lane, per, D, w, eps);
  long p = pos ? pos[r] : pos0 + (long)r * pos_stride;
  p = p < 0 ? 0 : p;
  rope_lane<PER>(v, lane, per, D, rd, cos_t, sin_t, p, false);
  fake_quant_lane<PER>(v, per, 32, 0);
  uint16_t o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = f2bf(v[i]);
  const long s = seq ? seq[r] : (long)(r / rows_per_seq);
  if (r >= commit_from) {
    uint16_t* dst = cache + s * cache_sstride + (p % W) * (long)D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane * per + i;
      if (i < per && c < D) dst[c] = o[i];
    }
  }
  if (tmp) {
    uint16_t* dst = tmp + (long)r * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane * per + i;
      if (i < per && c < D) dst[c] = o[i];
    }
  }
}

// ---------------------------------------------------------------------------------------------- append_rows
// Row r of x -> [rmsnorm] -> [rope at pos] -> fake quant -> bf16 cache[seq, row]; optional e4m3 sidecar with a
// per-row pow2 scale (k8[seq,row,:], ks[seq,row]).  row[r] < 0 skips the write.
template <int PER>
__global__ void __launch_bounds__(64) append_rows_kernel(
    const uint16_t* __restrict__ x, long x_rstride, const uint16_t* __restrict__ norm_w, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int rd, const long* __restrict__ pos,
    long pos0, long pos_stride, long pos_add, const long* __restrict__ seq, int rows_per_seq,
    const long* __restrict__ row, long row0, uint16_t* __restrict__ cache, long cache_sstride, int qmode, int group,
    uint8_t* __restrict__ k8, long k8_sstride, float* __restrict__ ks, long ks_sstride, int D) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int per = PER;
  float v[PER];
  load_row<PER>(v, x + (long)r * x_rstride, lane, per, D);
  if (norm_w) rmsnorm_lane<PER>(v, lane, per, D, norm_w, eps);
  if (rd > 0) {
    long p = (pos ? pos[r] : pos0 + (long)r * pos_stride) + pos_add;
    p = p < 0 ? 0 : p;
    rope_lane<PER>(v, lane, per, D, rd, cos_t, sin_t, p, false);
  }
  if (qmode >= 0) fake_quant_lane<PER>(v, per, group, qmode);
  const long s = seq ? seq[r] : (long)(r / rows_per_seq);
  const long dr = row ? row[r] : row0 + (r % rows_per_seq);
  if (dr < 0) return;
  if (cache) {
    uint16_t* dst = cache + s * cache_sstride + dr * (long)D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane * per + i;
      if (i < per && c < D) dst[c] = f2bf(v[i]);
    }
  }
  if (k8) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) a = fmaxf(a, fabsf(round_bf16(v[i])));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) a = fmaxf(a, wave_shfl_xor(a, m));
    int e = ceil_log2_f(__fdiv_rn(fmaxf(a, 1e-30f), 448.0f));
    e = e < -126 ? -126 : e;
    const float sc = pow2i(e);
    uint8_t* d8 = k8 + s * k8_sstride + dr * (long)D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane * per + i;
      if (i < per && c < D)
        d8[c] = (uint8_t)e4m3_bits(round_e4m3(fminf(fmaxf(round_bf16(v[i]) * pow2i(-e), -448.0f), 448.0f)));
    }
    if (lane == 0) ks[s * ks_sstride + dr] = sc;
  }
}

// ---------------------------------------------------------------------------------------------- fake quant
template <int PER>
__global__ void __launch_bounds__(64) fake_quant_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                        int D, int group, int mode) {
  const long r = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int per = PER;
  float v[PER];
  load_row<PER>(v, x + r * D, lane, per, D);
  fake_quant_lane<PER>(v, per, group, mode);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane * per + i;
    if (i < per && c < D) y[r * D + c] = f2bf(v[i]);
  }
}

// ---------------------------------------------------------------------------------------------- rope
// Row r of x ([n_rows, D], rows ordered (b, s, h)): position = base(b) + ((r / H) % S) * pos_stride, with
// base(b) = pos[b] + add (device positions) or pos0 (host position).
__global__ void __launch_bounds__(64) rope_kernel(uint16_t* __restrict__ x, const float* __restrict__ cos_t,
                                                  const float* __restrict__ sin_t, const long* __restrict__ pos,
                                                  long pos0, long add, long pos_stride, int H, int S, int D, int rd,
                                                  int inverse) {
  const long r = blockIdx.x;
  const int j = threadIdx.x;
  if (j >= rd / 2) return;
  long p = (pos ? pos[r / ((long)H * S)] + add : pos0) + ((r / H) % S) * pos_stride;
  p = p < 0 ? 0 : p;
  uint16_t* base = x + r * D + (D - rd);
  const float xr = bf2f(base[2 * j]), xi = bf2f(base[2 * j + 1]);
  const float c = cos_t[p * (rd / 2) + j];
  float s = sin_t[p * (rd / 2) + j];
  if (inverse) s = -s;
  base[2 * j] = f2bf(xr * c - xi * s);
  base[2 * j + 1] = f2bf(xr * s + xi * c);
}

template <int PER>
__global__ void __launch_bounds__(64) rmsnorm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     uint16_t* __restrict__ y, int D, float eps) {
  const long r = blockIdx.x;
  const int lane = threadIdx.x;
  constexpr int per = PER;
  float v[PER];
  load_row<PER>(v, x + r * D, lane, per, D);
  rmsnorm_lane<PER>(v, lane, per, D, w, eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane * per + i;
    if (i < per && c < D) y[r * D + c] = f2bf(v[i]);
  }
}

// Columns per lane: the smallest of 2/4/8/16 that covers the row with 64 lanes and divides D, so rope pairs and
// quantisation groups never straddle a lane boundary in an unaligned way.
int pick_per(int D) {
  const int c[4] = {2, 4, 8, 16};
  for (int i = 0; i < 4; ++i)
    if (D % c[i] == 0 && D <= 64 * c[i]) return c[i];
  return 0;
}

}  // namespace

extern "C" {

int dsv41_kv_write(const void* x, long x_rstride, const void* w, const float* cos_t, const float* sin_t,
                   const long* pos, const long* seq, long pos0, long pos_stride, int rows_per_seq, void* cache,
                   long cache_sstride, int W, void* tmp, int n_rows, int D, int rd, float eps, int commit_from,
                   void* stream) {
  if (n_rows <= 0) return 0;
  const int per = pick_per(D);
  if (per == 0 || rd % 2 != 0 || rd > D || W <= 0) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
#define KVW(P)                                                                                                   \
  kv_write_kernel<P><<<n_rows, 64, 0, st>>>((const uint16_t*)x, x_rstride, (const uint16_t*)w, cos_t, sin_t, pos, \
                                             seq, pos0, pos_stride, rows_per_seq, (uint16_t*)cache, cache_sstride, W, \
                                             (uint16_t*)tmp, D, rd, eps, commit_from)
  if (per <= 2) KVW(2);
  else if (per <= 4) KVW(4);
  else if (per <= 8) KVW(8);
  else KVW(16);
#undef KVW
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_append_rows(const void* x, long x_rstride, const void* norm_w, float eps, const float* cos_t,
                      const float* sin_t, int rd, const long* pos, long pos0, long pos_stride, long pos_add,
                      const long* seq, int rows_per_seq, const long* row, long row0, void* cache, long cache_sstride,
                      int qmode, int group, void* k8, long k8_sstride, float* ks, long ks_sstride, int n_rows, int D,
                      void* stream) {
  if (n_rows <= 0) return 0;
  const int per = pick_per(D);
  if (per == 0 || rd % 2 != 0 || rd > D) return (int)hipErrorInvalidValue;
  if (qmode >= 0 && (group != 16 && group != 32)) return (int)hipErrorInvalidValue;
  if (rows_per_seq <= 0) rows_per_seq = 1;
  hipStream_t st = (hipStream_t)stream;
#define APP(P)                                                                                                      \
  append_rows_kernel<P><<<n_rows, 64, 0, st>>>((const uint16_t*)x, x_rstride, (const uint16_t*)norm_w, eps, cos_t, \
                                                sin_t, rd, pos, pos0, pos_stride, pos_add, seq, rows_per_seq, row,    \
                                                row0, (uint16_t*)cache, cache_sstride, qmode, group, (uint8_t*)k8,    \
                                                k8_sstride, ks, ks_sstride, D)
  if (per <= 2) APP(2);
  else if (per <= 4) APP(4);
  else if (per <= 8) APP(8);
  else APP(16);
#undef APP
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_fake_quant(const void* x, void* y, long n_rows, int D, int group, int mode, void* stream) {
  if (n_rows <= 0) return 0;
  const int per = pick_per(D);
  if (per == 0 || (group != 16 && group != 32) || mode < 0 || mode > 2 || D % group != 0)
    return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  if (per <= 2) fake_quant_kernel<2><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (uint16_t*)y, D, group, mode);
  else if (per <= 4) fake_quant_kernel<4><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (uint16_t*)y, D, group, mode);
  else if (per <= 8) fake_quant_kernel<8><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (uint16_t*)y, D, group, mode);
  else fake_quant_kernel<16><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (uint16_t*)y, D, group, mode);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_rope(void* x, const float* cos_t, const float* sin_t, const long* pos, long pos0, long add, long pos_stride,
               long n_rows, int H, int S, int D, int rd, int inverse, void* stream) {
  if (n_rows <= 0) return 0;
  if (rd <= 0 || rd % 2 != 0 || rd > D || rd / 2 > 64 || H <= 0 || S <= 0) return (int)hipErrorInvalidValue;
  rope_kernel<<<n_rows, 64, 0, (hipStream_t)stream>>>((uint16_t*)x, cos_t, sin_t, pos, pos0, add, pos_stride, H, S, D,
                                                      rd, inverse);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_rmsnorm(const void* x, const void* w, void* y, long n_rows, int D, float eps, void* stream) {
  if (n_rows <= 0) return 0;
  const int per = pick_per(D);
  if (per == 0) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  if (per <= 2) rmsnorm_kernel<2><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, D, eps);
  else if (per <= 4) rmsnorm_kernel<4><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, D, eps);
  else if (per <= 8) rmsnorm_kernel<8><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, D, eps);
  else rmsnorm_kernel<16><<<n_rows, 64, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, D, eps);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
