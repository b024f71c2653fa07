// Lightning indexer of the sparse-attention path: scores and top-k selection over the compressed positions.
//
//   dsv41_index_score    score[r, t] = sum_h w[r,h] * relu(q[r,h,:] . k[slot(r), t, :])   (dsv41/fused3.py:20-62)
//                        -inf for t >= cl[r].  Keys are either bf16 rows (the reference's storage, FP4-grid values)
//                        or e4m3 rows with an fp32 per-row scale.  The bf16 query is re-encoded per (row, head) as
//                        e4m3 with a power-of-two scale, folded into the head weight, so the fp8 path runs the
//                        16x16x128 fp8 MFMA; relu(s*x) = s*relu(x) for the positive scales.
//   dsv41_topk_indices   the k largest scores of each row, ascending index order, -1 padding / masking
//                        (dsv41/fused3.py:65-75, dsv41/cuda/topk_select.cu); ties resolved lowest index first.
//
// Score kernel: 4 waves per workgroup, each wave owns 64 consecutive key positions of one query row (4 MFMA
// column tiles of 16 keys); the query fragments live in VGPRs.  MFMA output layout: lane l holds key (l & 15) and
// heads 4*(l >> 4) + i, so the head reduction is 16 in-lane FMAs plus two cross-lane shuffles.
// Keys at positions >= cl are never read: the scan is bounded by the valid count, not the allocated capacity.
#include "common.h"

namespace {

struct ScoreArgs {
  const uint16_t* q;  // [R, HI, 128] bf16
  long q_rstride;
  const float* w;  // [R, HI] fp32
  long w_rstride;
  int HI, R;
  int kfmt;  // 0: bf16 keys; 1: e4m3 keys + fp32 per-row scale
  const void* keys;
  long k_sstride;  // elements (bf16) or bytes (e4m3) between slots
  const float* kscale;
  long ks_sstride;
  const long* seq;  // slot = seq[r], or r / rows_per_slot when null
  int rows_per_slot;
  const long* cl;  // valid count per row, or (cl_start + (r % rows_per_slot) + 1) / cl_ratio when null
  long cl_start;
  int cl_ratio;
  int n_pos;         // columns of the output row
  int write_masked;  // write -inf for cl <= t < n_pos
  float* out;
  long out_rstride;
};

DSV41_DEV long row_cl(const ScoreArgs& a, int r) {
  if (a.cl) return a.cl[r];
  return (a.cl_start + (long)(r % a.rows_per_slot) + 1) / a.cl_ratio;
}

constexpr int kHT = 4;  // head tiles of 16 (up to 64 indexer heads)

template <int KFMT>
__global__ void __launch_bounds__(256) index_score_kernel(const ScoreArgs a) {
  const int r = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int kt0 = blockIdx.x * 256 + wave * 64;
  if (kt0 >= a.n_pos) return;
  long cl = row_cl(a, r);
  if (cl > a.n_pos) cl = a.n_pos;
  float* orow = a.out + (long)r * a.out_rstride;
  if (kt0 >= cl) {
    if (a.write_masked) {
      const int t = kt0 + lane;
      if (t < a.n_pos) orow[t] = -__builtin_inff();
    }
    return;
  }
  const long slot = a.seq ? a.seq[r] : (long)(r / a.rows_per_slot);
  const int nht = (a.HI + 15) / 16;

  // ---- query fragments and folded head weights
  i32x8_t qa8[kHT];
  uint4 qa16[kHT][4];
  float wl[kHT];  // weight (x query scale) of head ht*16 + l16
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    const int h = ht * 16 + l16;
    const bool hv = ht < nht && h < a.HI;
    const uint16_t* qrow = a.q + (long)r * a.q_rstride + (long)h * 128;
    const float wv = hv ? a.w[(long)r * a.w_rstride + h] : 0.0f;
    if (KFMT == 1) {
      float x[32];
      float amax = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint4 v = hv ? *(const uint4*)(qrow + g * 32 + u * 8) : make_uint4(0, 0, 0, 0);
        const uint32_t ww[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[u * 8 + 2 * e] = __uint_as_float(ww[e] << 16);
          x[u * 8 + 2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(x[e]));
      amax = fmaxf(amax, wave_shfl_xor(amax, 16));
      amax = fmaxf(amax, wave_shfl_xor(amax, 32));
      int ex = ceil_log2_f(fmaxf(amax, 1e-30f) / 448.0f);
      ex = ex < -126 ? -126 : ex;
      const float inv = pow2i(-ex);
      uint32_t pk[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        uint32_t b = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          b |= e4m3_bits(round_e4m3(fminf(fmaxf(x[d * 4 + e] * inv, -448.0f), 448.0f))) << (8 * e);
        pk[d] = b;
      }
      qa8[ht] = i32x8_t{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3], (int)pk[4], (int)pk[5], (int)pk[6], (int)pk[7]};
      wl[ht] = wv * pow2i(ex);
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        qa16[ht][ks] = hv ? *(const uint4*)(qrow + ks * 32 + g * 8) : make_uint4(0, 0, 0, 0);
      wl[ht] = wv;
    }
  }
  float wr[kHT][4];  // weights of the heads this lane's accumulators hold: ht*16 + 4g + i
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wl[ht], 4 * g + i, 64);

  const int lim = (int)cl;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int t = kt0 + nt * 16 + l16;
    const bool tv = t < lim;
    f32x4_t acc[kHT];
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) acc[ht] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float ksc = 1.0f;
    if (KFMT == 1) {
      const uint8_t* krow = (const uint8_t*)a.keys + slot * a.k_sstride + (long)t * 128 + g * 32;
      uint4 k0 = make_uint4(0, 0, 0, 0), k1 = make_uint4(0, 0, 0, 0);
      if (tv) {
        k0 = *(const uint4*)krow;
        k1 = *(const uint4*)(krow + 16);
        ksc = a.kscale[slot * a.ks_sstride + t];
      }
      const i32x8_t kb = i32x8_t{(int)k0.x, (int)k0.y, (int)k0.z, (int)k0.w, (int)k1.x, (int)k1.y, (int)k1.z, (int)k1.w};
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht)
        if (ht < nht) acc[ht] = mfma_fp8_16x16x128(qa8[ht], kb, acc[ht]);
    } else {
      const uint16_t* krow = (const uint16_t*)a.keys + slot * a.k_sstride + (long)t * 128 + g * 8;
      uint4 kb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kb[ks] = tv ? *(const uint4*)(krow + ks * 32) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht)
        if (ht < nht)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) acc[ht] = mfma_bf16_16x16x32(qa16[ht][ks], kb[ks], acc[ht]);
    }
    float s = 0.0f;
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) s += wr[ht][i] * fmaxf(acc[ht][i], 0.0f);
    s += wave_shfl_xor(s, 16);
    s += wave_shfl_xor(s, 32);
    if (g == 0 && t < a.n_pos) {
      if (tv) orow[t] = s * ksc;
      else if (a.write_masked) orow[t] = -__builtin_inff();
    }
  }
}

// ------------------------------------------------------------------------------------------------ top-k
constexpr int kTopkThreads = 1024;
constexpr int kTopkCache = 32768;  // rows up to this many valid positions are staged in LDS once

struct TopkArgs {
  const float* score;
  long ld;
  const long* cl;  // per row, or (cl_start + (r % rows_per_seq) + 1) / cl_ratio when null
  long cl_start;
  int cl_ratio;
  int rows_per_seq;
  int n, k;
  int* out;
  long out_rstride;
  int offset;
};

// Block-wide exclusive scan of one int per thread (1024 threads = 16 waves).  Returns the prefix; *total = sum.
DSV41_DEV int block_excl_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < 16 ? tmp[lane] : 0;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) {
      const int y = __shfl_up(w, d, 64);
      if (lane >= d) w += y;
    }
    if (lane < 16) tmp[16 + lane] = w;  // inclusive wave prefix
  }
  __syncthreads();
  const int before = wave ? tmp[16 + wave - 1] : 0;
  *total = tmp[31];
  const int r = before + x - v;
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(kTopkThreads) topk_kernel(const TopkArgs a) {
  __shared__ uint32_t keys[kTopkCache];
  __shared__ int hist[2048];
  __shared__ int scan_tmp[32];
  __shared__ int s_digit, s_rem;
  if (threadIdx.x == 0) {
    s_digit = 0;
    s_rem = 0;
  }
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* row = a.score + (long)r * a.ld;
  int* orow = a.out + (long)r * a.out_rstride;
  long clr = a.cl ? a.cl[r] : (a.cl_start + (long)(r % a.rows_per_seq) + 1) / a.cl_ratio;
  const int c = (int)(clr < 0 ? 0 : (clr > a.n ? a.n : clr));
  const int k = a.k;
  if (c <= k) {
    for (int i = tid; i < k; i += kTopkThreads) orow[i] = i < c ? i + a.offset : -1;
    return;
  }
  const bool cached = c <= kTopkCache;
  if (cached)
    for (int i = tid; i < c; i += kTopkThreads) keys[i] = score_key(row[i]);
  uint32_t prefix = 0u, pmask = 0u;
  int remaining = k;
  const int shifts[3] = {21, 10, 0};
  const int nbits[3] = {11, 11, 10};
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = shifts[pass], nb = 1 << nbits[pass];
    for (int i = tid; i < 2048; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < c; i += kTopkThreads) {
      const uint32_t key = cached ? keys[i] : score_key(row[i]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & (nb - 1)], 1);
    }
    __syncthreads();
    // descending suffix counts: thread t owns bins 2u, 2u+1 with u = 1023 - t (so the scan runs high -> low)
    const int u = kTopkThreads - 1 - tid;
    const int hlo = 2 * u < nb ? hist[2 * u] : 0, hhi = 2 * u + 1 < nb ? hist[2 * u + 1] : 0;
    int total;
    const int greater_hi = block_excl_scan(hlo + hhi, scan_tmp, &total);  // elements in bins > 2u+1
    if (2 * u + 1 < nb && greater_hi < remaining && remaining <= greater_hi + hhi) {
      s_digit = 2 * u + 1;
      s_rem = remaining - greater_hi;
    }
    const int greater_lo = greater_hi + hhi;
    if (2 * u < nb && greater_lo < remaining && remaining <= greater_lo + hlo) {
      s_digit = 2 * u;
      s_rem = remaining - greater_lo;
    }
    __syncthreads();
    prefix |= (uint32_t)s_digit << shift;
    pmask |= (uint32_t)(nb - 1) << shift;
    remaining = s_rem;
    __syncthreads();
  }
  const uint32_t thr = prefix;
  // ordered emission: thread t owns a contiguous span; two block scans give each thread its output offset
  const int span = (c + kTopkThreads - 1) / kTopkThreads;
  const int i0 = min(c, tid * span), i1 = min(c, i0 + span);
  int gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = cached ? keys[i] : score_key(row[i]);
    gt += key > thr;
    eq += key == thr;
  }
  int total;
  const int eq_before = block_excl_scan(eq, scan_tmp, &total);
  int take = remaining - eq_before;
  take = take < 0 ? 0 : (take > eq ? eq : take);
  int pos = block_excl_scan(gt + take, scan_tmp, &total);
  for (int i = i0; i < i1; ++i) {
    const uint32_t key = cached ? keys[i] : score_key(row[i]);
    if (key > thr) {
      if (pos < k) orow[pos] = i + a.offset;
      ++pos;
    } else if (key == thr && take > 0) {
      if (pos < k) orow[pos] = i + a.offset;
      ++pos;
      --take;
    }
  }
}

int launch_score(ScoreArgs& a, hipStream_t st) {
  if (a.R <= 0 || a.n_pos <= 0) return 0;
  if (a.HI <= 0 || a.HI > 64) return (int)hipErrorInvalidValue;
  dim3 grid((a.n_pos + 255) / 256, a.R);
  if (a.kfmt == 1) index_score_kernel<1><<<grid, 256, 0, st>>>(a);
  else index_score_kernel<0><<<grid, 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // namespace

extern "C" {

int dsv41_index_score(const void* q, long q_rstride, const float* w, long w_rstride, int R, int HI, int D, int kfmt,
                      const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                      int rows_per_slot, const long* cl, long cl_start, int cl_ratio, int n_pos, int write_masked,
                      float* out, long out_rstride, void* stream) {
  if (D != 128 || (kfmt == 1 && !kscale) || (!cl && cl_ratio <= 0)) return (int)hipErrorInvalidValue;
  ScoreArgs a{};
  a.q = (const uint16_t*)q;
  a.q_rstride = q_rstride;
  a.w = w;
  a.w_rstride = w_rstride;
  a.HI = HI;
  a.R = R;
  a.kfmt = kfmt;
  a.keys = keys;
  a.k_sstride = k_sstride;
  a.kscale = kscale;
  a.ks_sstride = ks_sstride;
  a.seq = seq;
  a.rows_per_slot = rows_per_slot > 0 ? rows_per_slot : 1;
  a.cl = cl;
  a.cl_start = cl_start;
  a.cl_ratio = cl_ratio;
  a.n_pos = n_pos;
  a.write_masked = write_masked;
  a.out = out;
  a.out_rstride = out_rstride;
  return launch_score(a, (hipStream_t)stream);
}

int dsv41_topk_indices(const float* score, long ld, int R, int n, int k, const long* cl, long cl_start, int cl_ratio,
                       int rows_per_seq, int offset, int* out, long out_rstride, void* stream) {
  if (R <= 0 || k <= 0) return 0;
  if (n < 0 || (!cl && cl_ratio <= 0)) return (int)hipErrorInvalidValue;
  TopkArgs a{};
  a.score = score;
  a.ld = ld;
  a.cl = cl;
  a.cl_start = cl_start;
  a.cl_ratio = cl_ratio;
  a.rows_per_seq = rows_per_seq > 0 ? rows_per_seq : 1;
  a.n = n;
  a.k = k;
  a.out = out;
  a.out_rstride = out_rstride;
  a.offset = offset;
  topk_kernel<<<R, kTopkThreads, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
