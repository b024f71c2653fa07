// Decode top-k selection over the indexer scores, spread over many workgroups (dsv41/fused3.py:65-75 semantics:
// the k largest of score[r, 0..cl) in ascending index order, -1 padding, ties lowest index first).
//
// The score kernel has already built hist[r][4096]: counts of the top 12 bits of the order-preserving score key
// (sign, exponent, 3 mantissa bits -> 8 bins per octave).  Then:
//   select_chunks   grid (chunks of 1024 positions, rows): every workgroup finds the threshold bin B of its row from
//                   the histogram (the bin holding the k-th largest key), and writes, in ascending index order, the
//                   positions of its chunk whose bin is above B ("above") and those in bin B ("candidates", with
//                   their keys) into chunk-owned regions of the workspace, plus the two counts.
//   finalize        one workgroup per row: gathers the candidates (only bin B: typically a few percent of the row),
//                   resolves the exact threshold key with two 10-bit radix passes in LDS, marks above + taken
//                   candidates in an LDS bitmap over the row and emits the set in index order from the bitmap's
//                   popcount prefix.  It leaves hist[r] zeroed for the next step.
// The row is read once (select) and never re-scanned; the finalize work is proportional to k plus the candidates.
#include "common.h"

namespace {

constexpr int kBins = 4096;
constexpr int kChunk = 1024;        // positions per select workgroup (256 threads x 4)
constexpr int kFinThreads = 1024;
constexpr int kCandCap = 12288;     // candidates staged in LDS by finalize (more: read from the workspace)
constexpr int kMaxBitmapWords = 8448;  // rows up to 270336 positions

struct SelArgs {
  const float* score;
  long ld;
  const long* cl;
  int n, k, R;
  int* hist;         // [R, kBins]
  int* counts;       // [R, nchunks, 2]
  int* above;        // [R, n]   (chunk-owned regions)
  int* cand_idx;     // [R, n]
  uint32_t* cand_key;  // [R, n]
  int nchunks;
  int* out;          // [R, k]
  long out_rstride;
  int offset;
};

DSV41_DEV int row_c(const SelArgs& a, int r) {
  long c = a.cl[r];
  return (int)(c < 0 ? 0 : (c > a.n ? a.n : c));
}

// Exclusive scan over the threads of a block of NT threads (NT/64 waves); tmp holds >= 2 * NT/64 ints.
template <int NT>
DSV41_DEV int block_scan(int v, int* tmp, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
#pragma unroll 1
    for (int w = 0; w < NW; ++w) {
      const int t = tmp[w];
      tmp[NW + w] = acc;
      acc += t;
    }
    tmp[2 * NW] = acc;
  }
  __syncthreads();
  const int r = tmp[NW + wave] + x - v;
  *total = tmp[2 * NW];
  __syncthreads();
  return r;
}

// Threshold bin of a row: the bin b with above(b) < k <= above(b) + hist[b], above(b) = sum of bins > b.
// 256 threads, 16 bins each (thread t: bins 4095-16t .. 4080-16t, scanned high to low).  Returns -1 when the
// histogram holds fewer than k entries (everything is selected).
DSV41_DEV void find_threshold_bin(const int* __restrict__ gh, int k, int* tmp, int* s_bin, int* s_above) {
  const int t = threadIdx.x;
  int h[16];
  const int4* p = (const int4*)(gh + kBins - 16 * (t + 1));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int4 v = p[u];
    h[4 * u] = v.x;
    h[4 * u + 1] = v.y;
    h[4 * u + 2] = v.z;
    h[4 * u + 3] = v.w;
  }
  int local = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) local += h[i];
  if (t == 0) {
    *s_bin = -1;
    *s_above = 0;
  }
  int total;
  int above = block_scan<256>(local, tmp, &total);  // entries in bins above this thread's range
  if (above < k && k <= above + local) {
#pragma unroll 1
    for (int i = 15; i >= 0; --i) {  // h[15] is this thread's highest bin
      if (k <= above + h[i]) {
        *s_bin = kBins - 16 * (t + 1) + i;
        *s_above = above;
        break;
      }
      above += h[i];
    }
  }
  __syncthreads();
}

__global__ void __launch_bounds__(256) select_chunks_kernel(const SelArgs a) {
  __shared__ int tmp[16];
  __shared__ int s_bin, s_above;
  __shared__ int wa[4], wc[4];
  const int ch = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = row_c(a, r);
  if (c <= a.k || ch * kChunk >= c) return;  // uniform per block
  // scores of this wave's 256 consecutive positions (4 x 64), issued with the histogram loads
  const int p0 = ch * kChunk + wave * 256;
  const float* row = a.score + (long)r * a.ld;
  float v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = p0 + u * 64 + lane;
    v[u] = row[i < c ? i : 0];
  }
  find_threshold_bin(a.hist + (long)r * kBins, a.k, tmp, &s_bin, &s_above);
  const int B = s_bin;
  uint32_t key[4];
  int n_above = 0, n_cand = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const bool in = p0 + u * 64 + lane < c;
    key[u] = score_key(v[u]);
    const int b = (int)(key[u] >> 20);
    n_above += __popcll(__ballot(in && b > B));
    n_cand += __popcll(__ballot(in && b == B));
  }
  if (lane == 0) {
    wa[wave] = n_above;
    wc[wave] = n_cand;
  }
  __syncthreads();
  int base_a = 0, base_c = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    base_a += w < wave ? wa[w] : 0;
    base_c += w < wave ? wc[w] : 0;
  }
  if (tid == 0) {
    int* cnt = a.counts + ((long)r * a.nchunks + ch) * 2;
    cnt[0] = wa[0] + wa[1] + wa[2] + wa[3];
    cnt[1] = wc[0] + wc[1] + wc[2] + wc[3];
  }
  const long reg = (long)r * a.n + (long)ch * kChunk;
  const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = p0 + u * 64 + lane;
    const bool in = i < c;
    const int b = (int)(key[u] >> 20);
    const unsigned long long ba = __ballot(in && b > B), bc = __ballot(in && b == B);
    if (in && b > B) a.above[reg + base_a + __popcll(ba & lt)] = i;
    if (in && b == B) {
      const long q = reg + base_c + __popcll(bc & lt);
      a.cand_idx[q] = i;
      a.cand_key[q] = key[u];
    }
    base_a += __popcll(ba);
    base_c += __popcll(bc);
  }
}

__global__ void __launch_bounds__(kFinThreads) finalize_kernel(const SelArgs a) {
  __shared__ uint32_t bitmap[kMaxBitmapWords];
  __shared__ uint32_t ck[kCandCap];
  __shared__ int ci[kCandCap];
  __shared__ int hist[1024];
  __shared__ int tmp[40];
  __shared__ int pa[1024], pc[1024];  // per-chunk exclusive prefix of above / candidate counts (<= 1024 chunks)
  __shared__ int s_digit, s_rem;
  DSV41_TS(0);
  const int r = blockIdx.x, tid = threadIdx.x;
  const int c = row_c(a, r), k = a.k;
  int* orow = a.out + (long)r * a.out_rstride;
  int* gh = a.hist + (long)r * kBins;
  if (c <= k) {
#pragma unroll 1
    for (int i = tid; i < k; i += kFinThreads) orow[i] = i < c ? i + a.offset : -1;
#pragma unroll 1
    for (int i = tid; i < kBins; i += kFinThreads) gh[i] = 0;
    return;
  }
  const int nch = (c + kChunk - 1) / kChunk;
  const int words = (c + 31) / 32;
  // ---- chunk counts -> prefixes (thread t owns chunk t; nch <= kFinThreads is checked by the host)
  int na = 0, nc = 0;
  if (tid < nch) {
    const int* cnt = a.counts + ((long)r * a.nchunks + tid) * 2;
    na = cnt[0];
    nc = cnt[1];
  }
  DSV41_TS(1);
  int tot_a, tot_c;
  const int ea = block_scan<kFinThreads>(na, tmp, &tot_a);
  const int ec = block_scan<kFinThreads>(nc, tmp, &tot_c);
  if (tid < nch) {
    pa[tid] = ea;
    pc[tid] = ec;
  }
#pragma unroll 1
  for (int i = tid; i < words; i += kFinThreads) bitmap[i] = 0u;
  __syncthreads();
  DSV41_TS(2);
  const int need = k - tot_a;  // candidates to take (1 <= need <= tot_c)
  const bool staged = tot_c <= kCandCap;
  const long reg = (long)r * a.n;
  // ---- stage candidates (index order) and mark the above positions: flat loops, every load independent
  auto chunk_of = [&](const int* pre, int j) {  // last chunk q with pre[q] <= j
    int lo = 0, hi = nch - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= j) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  if (staged) {
#pragma unroll 1
    for (int j = tid; j < tot_c; j += kFinThreads) {
      const int q = chunk_of(pc, j);
      const long src = reg + (long)q * kChunk + (j - pc[q]);
      ck[j] = a.cand_key[src];
      ci[j] = a.cand_idx[src];
    }
  }
#pragma unroll 1
  for (int j = tid; j < tot_a; j += kFinThreads) {
    const int q = chunk_of(pa, j);
    const int i = a.above[reg + (long)q * kChunk + (j - pa[q])];
    atomicOr(&bitmap[i >> 5], 1u << (i & 31));
  }
  __syncthreads();
  DSV41_TS(3);
  // candidate j (0 <= j < tot_c, index order) -> (key, position)
  auto cand = [&](int j, uint32_t* key, int* pos) {
    if (staged) {
      *key = ck[j];
      *pos = ci[j];
    } else {  // read it from its chunk's region
      const int lo = chunk_of(pc, j);
      const long q = reg + (long)lo * kChunk + (j - pc[lo]);
      *key = a.cand_key[q];
      *pos = a.cand_idx[q];
    }
  };
  // ---- radix select of the need-th largest among the candidates on the low 20 key bits (2 x 10 bits)
  uint32_t prefix = 0u, pmask = 0u;
  int remaining = need;
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 10 : 0;
    hist[tid] = 0;
    __syncthreads();
#pragma unroll 1
    for (int j = tid; j < tot_c; j += kFinThreads) {
      uint32_t key;
      int pos;
      cand(j, &key, &pos);
      const uint32_t d = key & 0xfffffu;
      if ((d & pmask) == prefix) atomicAdd(&hist[(d >> shift) & 1023], 1);
    }
    __syncthreads();
    const int u = kFinThreads - 1 - tid;  // bin u, scanned high to low
    const int hv = hist[u];
    int total;
    const int greater = block_scan<kFinThreads>(hv, tmp, &total);
    if (greater < remaining && remaining <= greater + hv) {
      s_digit = u;
      s_rem = remaining - greater;
    }
    __syncthreads();
    prefix |= (uint32_t)s_digit << shift;
    pmask |= 1023u << shift;
    remaining = s_rem;
    __syncthreads();
  }
  DSV41_TS(4);
  // ---- take candidates with low bits > prefix, and the first `remaining` equal ones in index order
  int eq_seen = 0;
#pragma unroll 1
  for (int j0 = 0; j0 < tot_c; j0 += kFinThreads) {
    const int j = j0 + tid;
    uint32_t key = 0;
    int pos = 0;
    if (j < tot_c) cand(j, &key, &pos);
    const uint32_t d = key & 0xfffffu;
    const bool in = j < tot_c;
    const bool gt = in && d > prefix, eq = in && d == prefix;
    int tot_eq;
    const int rank = eq_seen + block_scan<kFinThreads>(eq ? 1 : 0, tmp, &tot_eq);
    if (gt || (eq && rank < remaining)) atomicOr(&bitmap[pos >> 5], 1u << (pos & 31));
    eq_seen += tot_eq;
  }
  __syncthreads();
  DSV41_TS(5);
  // ---- ordered emission from the bitmap: thread t owns words [t*wpt, (t+1)*wpt)
  const int wpt = (words + kFinThreads - 1) / kFinThreads;
  const int w0 = tid * wpt;
  int cnt = 0;
#pragma unroll 1
  for (int w = w0; w < w0 + wpt && w < words; ++w) cnt += __popc(bitmap[w]);
  int tot;
  int o = block_scan<kFinThreads>(cnt, tmp, &tot);
#pragma unroll 1
  for (int w = w0; w < w0 + wpt && w < words; ++w) {
    uint32_t m = bitmap[w];
    while (m) {
      const int b = __ffs(m) - 1;
      m &= m - 1u;
      if (o < k) orow[o] = w * 32 + b + a.offset;
      ++o;
    }
  }
  DSV41_TS(6);
#pragma unroll 1
  for (int i = tot + tid; i < k; i += kFinThreads) orow[i] = -1;
#pragma unroll 1
  for (int i = tid; i < kBins; i += kFinThreads) gh[i] = 0;
}

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_ts(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ts), sizeof(g_dsv41_ts)); }
#endif

long dsv41_select_workspace_bytes(int R, int n) {
  const long nch = (n + kChunk - 1) / kChunk;
  return (long)R * (kBins + nch * 2 + 3L * n) * 4;
}

int dsv41_select_topk(const float* score, long ld, int R, int n, int k, const long* cl, int offset, void* ws,
                      long ws_bytes, int* out, long out_rstride, void* stream) {
  if (R <= 0 || k <= 0) return 0;
  const int nch = (n + kChunk - 1) / kChunk;
  if (n <= 0 || !cl || nch > 1024 || (n + 31) / 32 > kMaxBitmapWords || k > n)
    return (int)hipErrorInvalidValue;
  if (!ws || ws_bytes < dsv41_select_workspace_bytes(R, n)) return (int)hipErrorInvalidValue;
  int* w = (int*)ws;
  SelArgs a{};
  a.score = score;
  a.ld = ld;
  a.cl = cl;
  a.n = n;
  a.k = k;
  a.R = R;
  a.hist = w;
  a.counts = w + (long)R * kBins;
  a.above = a.counts + (long)R * nch * 2;
  a.cand_idx = a.above + (long)R * n;
  a.cand_key = (uint32_t*)(a.cand_idx + (long)R * n);
  a.nchunks = nch;
  a.out = out;
  a.out_rstride = out_rstride;
  a.offset = offset;
  hipStream_t st = (hipStream_t)stream;
  select_chunks_kernel<<<dim3(nch, R), 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  finalize_kernel<<<R, kFinThreads, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
