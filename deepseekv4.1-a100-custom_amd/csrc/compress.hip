// Compressor pooling (dsv41/model.py:577-660, the per-row decode variant dsv41/decode.py:243-265): the softmax-gated
// pooling over `ratio` consecutive positions of the wkv / wgate projection outputs that produces the latent row the
// compressed-KV append stores, followed by rmsnorm.  Per channel d of a group of positions q:
//   pooled[d] = sum_q kv[q, d] * softmax_q(score[q, d]),   latent = rmsnorm(bf16(pooled)) (bf16).
// Every position's raw kv / score also goes to the sequence's ring of the last kRing positions (slot = pos % kRing,
// fp32), from which a group's members that precede the current call are read.
//
// One 256-thread block per output row; element d of a row lives in thread d % 256 (iteration d / 256).
#include "common.h"

namespace {

constexpr int kPoolThreads = 256;
constexpr int kPoolIters = 4;  // rows up to 1024 channels
constexpr int kMaxRatio = 16;

struct PoolArgs {
  const float* kv;     // [rows, D] projection outputs of this call (row stride x_rstride floats)
  const float* score;
  long x_rstride;
  float* ring_kv;      // [S, ring, D] fp32 (slot stride D, sequence stride ring_sstride floats)
  float* ring_sc;
  long ring_sstride;
  int ring;
  const long* pos;     // decode: per-row position and sequence
  const long* seq;
  long pos0;           // prefill: the chunk's first position (sequence 0 of the ring pointers)
  int n_rows;          // rows of kv / score
  int D, ratio;
  const uint16_t* norm_w;
  float eps;
  uint16_t* latent;    // [out rows, D] bf16
  long lat_rstride;
  uint8_t* should;     // decode: per row, (pos + 1) % ratio == 0
  long first_end;      // prefill: the position that closes the first pooled group
};

DSV41_DEV float pool_block_sum(float v, float* red) {
  v = row_sum4(v);
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 1, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Pool the group ending at position `end` of sequence s into latent row `out`; member q is read from this call's
// rows when row_of(q) >= 0, else from the ring.
template <class RowOf>
DSV41_DEV void pool_group(const PoolArgs& a, long s, long end, RowOf row_of, uint16_t* out, float* red) {
  const int t = threadIdx.x;
  float pooled[kPoolIters];
#pragma unroll
  for (int it = 0; it < kPoolIters; ++it) {
    const int d = it * kPoolThreads + t;
    pooled[it] = 0.0f;
    if (d >= a.D) continue;
    float kv[kMaxRatio], sc[kMaxRatio];
    float m = -__builtin_inff();
#pragma unroll 1
    for (int j = 0; j < a.ratio; ++j) {
      const long q = end - a.ratio + 1 + j;
      const long row = row_of(q);
      if (row >= 0) {
        kv[j] = a.kv[row * a.x_rstride + d];
        sc[j] = a.score[row * a.x_rstride + d];
      } else {
        const long slot = ((q % a.ring) + a.ring) % a.ring;
        kv[j] = a.ring_kv[s * a.ring_sstride + slot * a.D + d];
        sc[j] = a.ring_sc[s * a.ring_sstride + slot * a.D + d];
      }
      m = fmaxf(m, sc[j]);
    }
    float num = 0.0f, den = 0.0f;
#pragma unroll 1
    for (int j = 0; j < a.ratio; ++j) {
      const float e = sc[j] == -__builtin_inff() ? 0.0f : expf(sc[j] - m);
      num += e * kv[j];
      den += e;
    }
    pooled[it] = round_bf16(num / den);  // the reference pools in fp32, then casts to the activation dtype
  }
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < kPoolIters; ++it) ss += pooled[it] * pooled[it];
  ss = pool_block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)a.D + a.eps);
#pragma unroll
  for (int it = 0; it < kPoolIters; ++it) {
    const int d = it * kPoolThreads + t;
    if (d < a.D) out[d] = f2bf(pooled[it] * inv * bf2f(a.norm_w[d]));
  }
}

// Decode: this call's kv / score rows into their sequence's ring (before any row pools).
__global__ void __launch_bounds__(kPoolThreads) pool_ring_write_kernel(const PoolArgs a) {
  const int r = blockIdx.x;
  const long p = a.pos[r], s = a.seq[r];
  const long slot = ((p % a.ring) + a.ring) % a.ring;
  for (int d = threadIdx.x; d < a.D; d += kPoolThreads) {
    a.ring_kv[s * a.ring_sstride + slot * a.D + d] = a.kv[(long)r * a.x_rstride + d];
    a.ring_sc[s * a.ring_sstride + slot * a.D + d] = a.score[(long)r * a.x_rstride + d];
  }
}

// Decode: row r pools the group ending at its position from the ring (every member, its own included, is there).
__global__ void __launch_bounds__(kPoolThreads) pool_decode_kernel(const PoolArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const long p = a.pos[r], s = a.seq[r];
  pool_group(a, s, p, [](long) { return -1L; }, a.latent + (long)r * a.lat_rstride, red);
  if (threadIdx.x == 0) a.should[r] = (uint8_t)(((p + 1) % a.ratio) == 0);
}

// Prefill: block g pools the group ending at first_end + g * ratio; members before pos0 come from the ring.
__global__ void __launch_bounds__(kPoolThreads) pool_prefill_kernel(const PoolArgs a) {
  __shared__ float red[4];
  const long end = a.first_end + (long)blockIdx.x * a.ratio;
  const long p0 = a.pos0;
  pool_group(a, 0, end, [p0](long q) { return q >= p0 ? q - p0 : -1L; }, a.latent + (long)blockIdx.x * a.lat_rstride,
             red);
}

// Prefill: the chunk's last min(n_rows, ring) positions into the ring (after the pooling has read it).
__global__ void __launch_bounds__(kPoolThreads) pool_ring_tail_kernel(const PoolArgs a) {
  const int first = a.n_rows > a.ring ? a.n_rows - a.ring : 0;
  const int r = first + blockIdx.x;
  const long q = a.pos0 + r;
  const long slot = q % a.ring;
  for (int d = threadIdx.x; d < a.D; d += kPoolThreads) {
    a.ring_kv[slot * a.D + d] = a.kv[(long)r * a.x_rstride + d];
    a.ring_sc[slot * a.D + d] = a.score[(long)r * a.x_rstride + d];
  }
}

bool pool_ok(int D, int ratio, int ring) {
  return D > 0 && D <= kPoolThreads * kPoolIters && ratio >= 1 && ratio <= kMaxRatio && ring >= ratio;
}

}  // namespace

extern "C" {

int dsv41_compress_pool_decode(const float* kv, const float* score, long x_rstride, float* ring_kv, float* ring_sc,
                               long ring_sstride, int ring, const long* pos, const long* seq, int B, int D, int ratio,
                               const void* norm_w, float eps, void* latent, long lat_rstride, void* should,
                               void* stream) {
  if (B <= 0) return 0;
  if (!pool_ok(D, ratio, ring) || !pos || !seq || !should) return (int)hipErrorInvalidValue;
  PoolArgs a{};
  a.kv = kv;
  a.score = score;
  a.x_rstride = x_rstride;
  a.ring_kv = ring_kv;
  a.ring_sc = ring_sc;
  a.ring_sstride = ring_sstride;
  a.ring = ring;
  a.pos = pos;
  a.seq = seq;
  a.n_rows = B;
  a.D = D;
  a.ratio = ratio;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  a.latent = (uint16_t*)latent;
  a.lat_rstride = lat_rstride;
  a.should = (uint8_t*)should;
  hipStream_t st = (hipStream_t)stream;
  pool_ring_write_kernel<<<B, kPoolThreads, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  pool_decode_kernel<<<B, kPoolThreads, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

int dsv41_compress_pool_prefill(const float* kv, const float* score, long x_rstride, float* ring_kv, float* ring_sc,
                                int ring, long start_pos, int n_rows, int D, int ratio, const void* norm_w, float eps,
                                void* latent, long lat_rstride, int n_groups, void* stream) {
  if (n_rows <= 0) return 0;
  if (!pool_ok(D, ratio, ring) || start_pos < 0) return (int)hipErrorInvalidValue;
  const long first_end = start_pos + (ratio - 1 - start_pos % ratio);
  const long last = start_pos + n_rows - 1;
  const int want = first_end <= last ? (int)((last - first_end) / ratio + 1) : 0;
  if (n_groups != want) return (int)hipErrorInvalidValue;
  PoolArgs a{};
  a.kv = kv;
  a.score = score;
  a.x_rstride = x_rstride;
  a.ring_kv = ring_kv;
  a.ring_sc = ring_sc;
  a.ring = ring;
  a.pos0 = start_pos;
  a.n_rows = n_rows;
  a.D = D;
  a.ratio = ratio;
  a.norm_w = (const uint16_t*)norm_w;
  a.eps = eps;
  a.latent = (uint16_t*)latent;
  a.lat_rstride = lat_rstride;
  a.first_end = first_end;
  hipStream_t st = (hipStream_t)stream;
  if (n_groups > 0) {
    pool_prefill_kernel<<<n_groups, kPoolThreads, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
  }
  pool_ring_tail_kernel<<<n_rows < ring ? n_rows : ring, kPoolThreads, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
