// Cache-append kernels of the sparse-attention path and the small per-row numerics they fuse:
//   dsv41_kv_write        SWA ring append (rmsnorm -> bf16 -> rope -> bf16 -> fq8/32 -> ring[seq, pos % W])
//   dsv41_append_rows     compressed-KV / index-key append (optional rmsnorm, rope, fq4 or fq8, optional e4m3 copy)
//   dsv41_decode_appends  every cache write of a decode step + the e4m3 preparation of the index queries, one launch
//   dsv41_index_qprep     the index-query preparation alone
//   dsv41_fake_quant / dsv41_rope / dsv41_rmsnorm   standalone numerics
//
// One 256-thread block per row operation; element e of a row lives in thread e % 256 (iteration e / 256), so a
// quantisation group of 16/32 elements is 16/32 consecutive lanes of one wave (shuffle reductions) and a rope pair
// (2j, 2j+1) is a lane pair (xor 1).  The code is deliberately small and loop-shaped: these launches sit on the
// decode critical path, where a cold instruction cache costs more than the arithmetic.
#include "rowop.h"

namespace {

// ---------------------------------------------------------------------------------------------- kernels
struct KvWriteArgs {
  const uint16_t* x;
  long x_rstride;
  const uint16_t* w;
  const float* cos_t;
  const float* sin_t;
  const long* pos;
  const long* seq;
  long pos0, pos_stride;
  int rows_per_seq;
  uint16_t* cache;
  long cache_sstride;
  int W;
  uint16_t* tmp;
  int D, rd;
  float eps;
  int commit_from;
  // prefill window (one sequence, positions pos0 + r): the ring's history rows of positions pos0 - hist .. pos0 - 1
  // are copied to hist_tmp[0 .. hist) before the chunk overwrites their slots; blocks n_chunk .. n_chunk + hist - 1
  // copy the history rows whose slot no committed chunk row overwrites
  uint16_t* hist_tmp;
  int hist, n_chunk;
};

// Copy ring row `slot` of sequence s to dst (the whole block, 16-byte units; the row width is a multiple of 8).
DSV41_DEV void copy_ring_row(const KvWriteArgs& a, long s, long slot, uint16_t* dst) {
  const uint4* src = (const uint4*)(a.cache + s * a.cache_sstride + slot * (long)a.D);
  for (int u = threadIdx.x; u < a.D / 8; u += blockDim.x) ((uint4*)dst)[u] = src[u];
}

__global__ void __launch_bounds__(kRowThreads) kv_write_kernel(const KvWriteArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  if (a.hist_tmp && r >= a.n_chunk) {  // history row whose slot is not overwritten by the chunk
    const int h = r - a.n_chunk;
    const long q = a.pos0 - a.hist + h;
    const long r0 = ((q - a.pos0) % a.W + a.W) % a.W;  // chunk row offset that maps to the same slot
    const bool overwritten = r0 < a.n_chunk;  // some committed row r0 + k*W lies in [commit_from, n_chunk)
    if (!overwritten) copy_ring_row(a, 0, q % a.W, a.hist_tmp + (long)h * a.D);
    return;
  }
  long p = a.pos ? a.pos[r] : a.pos0 + (long)(r % a.rows_per_seq) * a.pos_stride;
  p = p < 0 ? 0 : p;
  const long s = a.seq ? a.seq[r] : (long)(r / a.rows_per_seq);
  RowOp o{};
  o.x = a.x + (long)r * a.x_rstride;
  o.D = a.D;
  o.norm_w = a.w;
  o.eps = a.eps;
  o.cos_t = a.cos_t;
  o.sin_t = a.sin_t;
  o.rd = a.rd;
  o.pos = p;
  o.qmode = 0;
  o.group = 32;
  o.out = r >= a.commit_from ? a.cache + s * a.cache_sstride + (p % a.W) * (long)a.D : nullptr;
  o.out2 = a.tmp ? a.tmp + (long)r * a.D : nullptr;
  if (a.hist_tmp && o.out) {  // the slot's previous row (position p - W .. p - 1 congruent to p) leaves first
    const long q_old = a.pos0 - a.W + (p - a.pos0) % a.W;
    const long h = q_old - (a.pos0 - a.hist);
    if (h >= 0 && h < a.hist) copy_ring_row(a, s, p % a.W, a.hist_tmp + h * a.D);
    __syncthreads();  // every thread's reads of the old row are complete before row_op writes the slot
  }
  row_op(o, red);
}

struct AppendArgs {
  const uint16_t* x;
  long x_rstride;
  const uint16_t* norm_w;
  float eps;
  const float* cos_t;
  const float* sin_t;
  int rd;
  const long* pos;
  long pos0, pos_stride, pos_add;
  const long* seq;
  int rows_per_seq;
  const long* row;
  long row0;
  uint16_t* cache;
  long cache_sstride;
  int qmode, group;
  uint8_t* k8;
  long k8_sstride;
  float* ks;
  long ks_sstride;
  int D;
};

__global__ void __launch_bounds__(kRowThreads) append_rows_kernel(const AppendArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const long s = a.seq ? a.seq[r] : (long)(r / a.rows_per_seq);
  const long dr = a.row ? a.row[r] : a.row0 + (r % a.rows_per_seq);
  if (dr < 0) return;  // uniform per block
  RowOp o{};
  o.x = a.x + (long)r * a.x_rstride;
  o.D = a.D;
  o.norm_w = a.norm_w;
  o.eps = a.eps;
  o.cos_t = a.cos_t;
  o.sin_t = a.sin_t;
  o.rd = a.rd;
  o.pos = (a.pos ? a.pos[r] : a.pos0 + (long)(r % a.rows_per_seq) * a.pos_stride) + a.pos_add;
  o.qmode = a.qmode;
  o.group = a.group;
  o.out = a.cache ? a.cache + s * a.cache_sstride + dr * (long)a.D : nullptr;
  o.k8 = a.k8 ? a.k8 + s * a.k8_sstride + dr * (long)a.D : nullptr;
  o.ks = a.ks ? a.ks + s * a.ks_sstride + dr : nullptr;
  row_op(o, red);
}

// Decode step: block (r, op): op 0 the SWA ring row, 1 the compressed-KV row, 2 the index-key row, 3 the index
// query preparation.  Compressed / index-key rows go to compress_len - 1 when (pos + 1) % ratio == 0, else to the
// table's spare last row (dsv41/decode.py:150-164, :176-181, :270-282).
struct DecAppArgs {
  const uint16_t* kv_raw;
  const uint16_t* kv_norm;
  uint16_t* ring;
  long ring_sstride;
  int W, Dw;
  const uint16_t* latent;
  uint16_t* ckv;
  long ckv_sstride;
  int cap;
  const uint16_t* k_raw;
  const uint16_t* k_norm;
  uint16_t* kbf;
  long kbf_sstride;
  uint8_t* k8;
  long k8_sstride;
  float* ks;
  long ks_sstride;
  int kcap, Dk;
  const long* pos;
  const long* seq;
  const long* nw_tab;  // [S] no-write row per sequence, or null (the tables' spare last row)
  int ratio, rd;
  const float* cos_t;
  const float* sin_t;
  float eps;
  const uint16_t* q_idx;  // [B, HI, 128] or null
  const uint16_t* w_idx;  // [B, HI] bf16
  int HI;
  uint8_t* q8;  // [B, 64, 128]
  float* wf;    // [B, 64]
};

__global__ void __launch_bounds__(kRowThreads) decode_appends_kernel(const DecAppArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x, op = blockIdx.y;
  const long p = a.pos[r];
  const long s = a.seq[r];
  if (op == 3) {
    if (a.q_idx)
      qprep_op(a.q_idx + (long)r * a.HI * 128, a.w_idx + (long)r * a.HI, nullptr, a.HI, a.q8 + (long)r * 64 * 128,
               a.wf + (long)r * 64);
    return;
  }
  const bool closes = ((p + 1) % a.ratio) == 0;
  RowOp o{};
  o.cos_t = a.cos_t;
  o.sin_t = a.sin_t;
  o.rd = a.rd;
  o.eps = a.eps;
  if (op == 0) {
    o.x = a.kv_raw + (long)r * a.Dw;
    o.D = a.Dw;
    o.norm_w = a.kv_norm;
    o.pos = p < 0 ? 0 : p;
    o.qmode = 0;
    o.group = 32;
    o.out = a.ring + s * a.ring_sstride + (o.pos % a.W) * (long)a.Dw;
  } else if (op == 1) {
    if (!a.latent || !a.ckv) return;
    const long row = closes ? (p + 1) / a.ratio - 1 : a.nw_tab ? a.nw_tab[s] : a.cap - 1;
    o.x = a.latent + (long)r * a.Dw;
    o.D = a.Dw;
    o.pos = p + 1 - a.ratio;
    o.qmode = 2;
    o.group = 16;
    o.out = a.ckv + s * a.ckv_sstride + row * (long)a.Dw;
  } else {
    if (!a.k_raw || (!a.kbf && !a.k8)) return;
    const long row = closes ? (p + 1) / a.ratio - 1 : a.nw_tab ? a.nw_tab[s] : a.kcap - 1;
    o.x = a.k_raw + (long)r * a.Dk;
    o.D = a.Dk;
    o.norm_w = a.k_norm;
    o.pos = p + 1 - a.ratio;
    o.qmode = 1;
    o.group = 32;
    o.out = a.kbf ? a.kbf + s * a.kbf_sstride + row * (long)a.Dk : nullptr;
    o.k8 = a.k8 ? a.k8 + s * a.k8_sstride + row * (long)a.Dk : nullptr;
    o.ks = a.k8 ? a.ks + s * a.ks_sstride + row : nullptr;
  }
  row_op(o, red);
}

// Index-key table conversion (the reference's bf16 table <-> this build's e4m3 + per-row scale, for cache snapshots
// taken by either, dsv41/engine.py:1072-1230): one wave per 128-wide row, two elements per lane; the encoding is the
// one of the key appends (row_compute's e4m3 copy).
__global__ void __launch_bounds__(256) index_keys_encode_kernel(const uint16_t* kbf, long n_rows, uint8_t* k8,
                                                                float* ks) {
  const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_rows) return;
  const uint32_t w = *(const uint32_t*)(kbf + r * 128 + 2 * lane);
  const float v0 = __uint_as_float(w << 16), v1 = __uint_as_float(w & 0xffff0000u);
  float a = fmaxf(fabsf(v0), fabsf(v1));
  a = group_max(a, 64);
  int ex = ceil_log2_f(__fdiv_rn(fmaxf(a, 1e-30f), 448.0f));
  ex = ex < -126 ? -126 : ex;
  const float inv = pow2i(-ex);
  const uint32_t b0 = e4m3_bits(round_e4m3(fminf(fmaxf(v0 * inv, -448.0f), 448.0f)));
  const uint32_t b1 = e4m3_bits(round_e4m3(fminf(fmaxf(v1 * inv, -448.0f), 448.0f)));
  *(uint16_t*)(k8 + r * 128 + 2 * lane) = (uint16_t)(b0 | b1 << 8);
  if (lane == 0) ks[r] = pow2i(ex);
}

__global__ void __launch_bounds__(256) index_keys_decode_kernel(const uint8_t* k8, const float* ks, long n_rows,
                                                                uint16_t* kbf) {
  const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_rows) return;
  const uint32_t b = *(const uint16_t*)(k8 + r * 128 + 2 * lane);
  const float s = ks[r];
  *(uint32_t*)(kbf + r * 128 + 2 * lane) =
      (uint32_t)f2bf(e4m3_value(b & 0xffu) * s) | (uint32_t)f2bf(e4m3_value(b >> 8) * s) << 16;
}

__global__ void __launch_bounds__(kRowThreads) qprep_kernel(const uint16_t* q, const float* w, int HI, uint8_t* q8,
                                                            float* wf) {
  const int r = blockIdx.x;
  qprep_op(q + (long)r * HI * 128, nullptr, w + (long)r * HI, HI, q8 + (long)r * 64 * 128, wf + (long)r * 64);
}

__global__ void __launch_bounds__(kRowThreads) fake_quant_kernel(const uint16_t* x, uint16_t* y, int D, int group,
                                                                 int mode) {
  __shared__ float red[4];
  RowOp o{};
  o.x = x + (long)blockIdx.x * D;
  o.D = D;
  o.qmode = mode;
  o.group = group;
  o.out = y + (long)blockIdx.x * D;
  row_op(o, red);
}

__global__ void __launch_bounds__(kRowThreads) rmsnorm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* y, int D,
                                                              float eps) {
  __shared__ float red[4];
  RowOp o{};
  o.x = x + (long)blockIdx.x * D;
  o.D = D;
  o.norm_w = w;
  o.eps = eps;
  o.qmode = -1;
  o.out = y + (long)blockIdx.x * D;
  row_op(o, red);
}

// rmsnorm + per-32 fp8 fake quantisation of rows of up to kNqMaxD elements (dsv41/fused2.py:251-272 norm_quant;
// without a weight, the fake quantisation alone: dsv41/fused.py:83-84 fake_quant_fp8 on any row length).  Thread t
// owns the 32-element groups t, t + 256: y = bf16(x * (1 / sqrt(mean(x^2) + eps)) * w), then e4m3 on the group's
// power-of-two scale, bf16 out.  quant = 0: the rmsnorm alone (dsv41_rmsnorm for rows past the row kernels' 1024).
constexpr int kNqMaxD = 2 * kRowThreads * 32;

__global__ void __launch_bounds__(kRowThreads) norm_quant_kernel(const uint16_t* x, const uint16_t* w, float eps,
                                                                 uint16_t* y, int D, int quant) {
  __shared__ float red[kRowThreads / 64];
  const uint16_t* xr = x + (long)blockIdx.x * D;
  uint16_t* yr = y + (long)blockIdx.x * D;
  const int ng = D / 32;
  float v[2][32];
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int grp = threadIdx.x + kRowThreads * q;
    uint4 raw[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) raw[u] = grp < ng ? ((const uint4*)(xr + 32 * grp))[u] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t ww[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[q][8 * u + 2 * e] = __uint_as_float(ww[e] << 16);
        v[q][8 * u + 2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int e = 0; e < 32; ++e) ss += v[q][e] * v[q][e];
  }
  if (w) {
    ss = block_sum<kRowThreads>(ss, red);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)D) + eps));
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int grp = threadIdx.x + kRowThreads * q;
      if (grp >= ng) break;
#pragma unroll
      for (int e = 0; e < 32; ++e) v[q][e] = round_bf16(v[q][e] * inv * bf2f(w[32 * grp + e]));
    }
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int grp = threadIdx.x + kRowThreads * q;
    if (grp >= ng) break;
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[q][e]));
    const float sc = fq_scale(amax, 0);
    uint32_t o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float lo = quant ? fq_value(v[q][2 * e], sc, 0) : v[q][2 * e];
      const float hi = quant ? fq_value(v[q][2 * e + 1], sc, 0) : v[q][2 * e + 1];
      o[e] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      ((uint4*)(yr + 32 * grp))[u] = make_uint4(o[4 * u], o[4 * u + 1], o[4 * u + 2], o[4 * u + 3]);
  }
}

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


}  // namespace

extern "C" {

int dsv41_kv_write(const void* x, long x_rstride, const void* w, const float* cos_t, const float* sin_t,
                   const long* pos, const long* seq, long pos0, long pos_stride, int rows_per_seq, void* cache,
                   long cache_sstride, int W, void* tmp, int n_rows, int D, int rd, float eps, int commit_from,
                   void* stream) {
  if (n_rows <= 0) return 0;
  if (!row_ok(D, 32) || rd % 2 != 0 || rd > D || W <= 0) return (int)hipErrorInvalidValue;
  KvWriteArgs a{(const uint16_t*)x, x_rstride, (const uint16_t*)w, cos_t, sin_t, pos, seq, pos0, pos_stride,
                rows_per_seq > 0 ? rows_per_seq : 1, (uint16_t*)cache, cache_sstride, W, (uint16_t*)tmp, D, rd, eps,
                commit_from, nullptr, 0, n_rows};
  kv_write_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_window_kv(const void* x, long x_rstride, const void* w, const float* cos_t, const float* sin_t,
                    long start_pos, int n_rows, void* ring, int W, void* out, int hist, int D, int rd, float eps,
                    void* stream) {
  if (n_rows <= 0) return 0;
  if (!row_ok(D, 32) || D % 8 != 0 || rd % 2 != 0 || rd > D || W <= 0 || start_pos < 0 || hist < 0 ||
      hist > W - 1 || hist > start_pos)
    return (int)hipErrorInvalidValue;
  uint16_t* o = (uint16_t*)out;
  KvWriteArgs a{(const uint16_t*)x, x_rstride, (const uint16_t*)w, cos_t, sin_t, nullptr, nullptr, start_pos, 1,
                n_rows, (uint16_t*)ring, 0, W, o + (long)hist * D, D, rd, eps, n_rows > W ? n_rows - W : 0,
                hist > 0 ? o : nullptr, hist, n_rows};
  kv_write_kernel<<<n_rows + hist, kRowThreads, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_append_rows(const void* x, long x_rstride, const void* norm_w, float eps, const float* cos_t,
                      const float* sin_t, int rd, const long* pos, long pos0, long pos_stride, long pos_add,
                      const long* seq, int rows_per_seq, const long* row, long row0, void* cache, long cache_sstride,
                      int qmode, int group, void* k8, long k8_sstride, float* ks, long ks_sstride, int n_rows, int D,
                      void* stream) {
  if (n_rows <= 0) return 0;
  if (qmode >= 0 && group != 16 && group != 32) return (int)hipErrorInvalidValue;
  if (!row_ok(D, qmode >= 0 ? group : 0) || rd % 2 != 0 || rd > D) return (int)hipErrorInvalidValue;
  AppendArgs a{(const uint16_t*)x, x_rstride, (const uint16_t*)norm_w, eps, cos_t, sin_t, rd, pos, pos0, pos_stride,
               pos_add, seq, rows_per_seq > 0 ? rows_per_seq : 1, row, row0, (uint16_t*)cache, cache_sstride, qmode,
               group, (uint8_t*)k8, k8_sstride, ks, ks_sstride, D};
  append_rows_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_decode_appends(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                         const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                         const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                         long ks_sstride, int kcap, int Dk, const long* pos, const long* seq,
                         const long* nw_tab, int ratio, const float* cos_t, const float* sin_t, int rd, float eps,
                         const void* q_idx, const void* w_idx, int HI, void* q8, float* wf, int B, void* stream) {
  if (B <= 0) return 0;
  if (!row_ok(Dw, 32) || !row_ok(Dk, 32) || ratio <= 0 || rd % 2 != 0 || rd > Dw || rd > Dk || W <= 0 ||
      cap <= 0 || kcap <= 0 || (q_idx && (!w_idx || !q8 || !wf || HI <= 0 || HI > 64)))
    return (int)hipErrorInvalidValue;
  DecAppArgs a{(const uint16_t*)kv_raw, (const uint16_t*)kv_norm, (uint16_t*)ring, ring_sstride, W, Dw,
               (const uint16_t*)latent, (uint16_t*)ckv, ckv_sstride, cap, (const uint16_t*)k_raw,
               (const uint16_t*)k_norm, (uint16_t*)kbf, kbf_sstride, (uint8_t*)k8, k8_sstride, ks, ks_sstride, kcap,
               Dk, pos, seq, nw_tab, ratio, rd, cos_t, sin_t, eps, (const uint16_t*)q_idx, (const uint16_t*)w_idx,
               HI, (uint8_t*)q8, wf};
  decode_appends_kernel<<<dim3(B, q_idx ? 4 : 3), kRowThreads, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_index_keys_encode(const void* kbf, long n_rows, void* k8, float* ks, void* stream) {
  if (n_rows <= 0) return 0;
  if (!kbf || !k8 || !ks) return (int)hipErrorInvalidValue;
  index_keys_encode_kernel<<<(unsigned)((n_rows + 3) / 4), 256, 0, (hipStream_t)stream>>>((const uint16_t*)kbf, n_rows,
                                                                                          (uint8_t*)k8, ks);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_index_keys_decode(const void* k8, const float* ks, long n_rows, void* kbf, void* stream) {
  if (n_rows <= 0) return 0;
  if (!kbf || !k8 || !ks) return (int)hipErrorInvalidValue;
  index_keys_decode_kernel<<<(unsigned)((n_rows + 3) / 4), 256, 0, (hipStream_t)stream>>>((const uint8_t*)k8, ks,
                                                                                          n_rows, (uint16_t*)kbf);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_index_qprep(const void* q, const float* w, int R, int HI, void* q8, float* wf, void* stream) {
  if (R <= 0) return 0;
  if (HI <= 0 || HI > 64) return (int)hipErrorInvalidValue;
  qprep_kernel<<<R, kRowThreads, 0, (hipStream_t)stream>>>((const uint16_t*)q, w, HI, (uint8_t*)q8, wf);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_fake_quant(const void* x, void* y, long n_rows, int D, int group, int mode, void* stream) {
  if (n_rows <= 0) return 0;
  if ((group != 16 && group != 32) || mode < 0 || mode > 2 || !row_ok(D, group)) return (int)hipErrorInvalidValue;
  fake_quant_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>((const uint16_t*)x, (uint16_t*)y, D, group, mode);
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

int dsv41_norm_quant(const void* x, const void* w, float eps, void* y, long n_rows, int D, void* stream) {
  if (n_rows <= 0) return 0;
  if (D <= 0 || D % 32 != 0 || D > kNqMaxD || ((uintptr_t)x & 15) != 0 || ((uintptr_t)y & 15) != 0)
    return (int)hipErrorInvalidValue;
  norm_quant_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>((const uint16_t*)x, (const uint16_t*)w, eps,
                                                                     (uint16_t*)y, D, 1);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_rmsnorm(const void* x, const void* w, void* y, long n_rows, int D, float eps, void* stream) {
  if (n_rows <= 0) return 0;
  if (D > kRowMaxD && D % 32 == 0 && D <= kNqMaxD && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && w) {
    norm_quant_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>((const uint16_t*)x, (const uint16_t*)w, eps,
                                                                       (uint16_t*)y, D, 0);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  if (!row_ok(D, 0)) return (int)hipErrorInvalidValue;
  rmsnorm_kernel<<<n_rows, kRowThreads, 0, (hipStream_t)stream>>>((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y,
                                                                  D, eps);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
