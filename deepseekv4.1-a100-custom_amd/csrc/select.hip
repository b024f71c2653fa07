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
// When a row's chunks fit one resident grid (at most 64 workgroups per XCD), select_group does both steps in one
// launch: the chunks of a row run on one XCD and meet at a row barrier (see the kernel).
#include "select_core.h"

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
  int* above;        // [R, rs]   (chunk-owned regions; rs = n rounded up to 32: rows never share a cache line)
  int* cand_idx;     // [R, rs]
  uint32_t* cand_key;  // [R, rs]
  long rs;
  int nchunks;
  int* out;          // [R, k]
  long out_rstride;
  int offset;
  int* rowbin;       // [R]: the row's threshold bin, written by select_chunks for emit_kernel
};

DSV41_DEV int row_c(const SelArgs& a, int r) {
  long c = a.cl[r];
  return (int)(c < 0 ? 0 : (c > a.n ? a.n : c));
}

// Exclusive scan over the threads of a block of NT threads (NT/64 waves); tmp holds >= NT/64 ints.  (DPP wave
// scans, two barriers; tmp may be reused right after.)
template <int NT>
DSV41_DEV int block_scan(int v, int* tmp, int* total) {
  return block_scan_dpp<NT>(v, tmp, total);
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
  if (ch == 0 && tid == 0 && a.rowbin) a.rowbin[r] = B;
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
  const long reg = (long)r * a.rs + (long)ch * kChunk;
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
  const long reg = (long)r * a.rs;
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

// Per-chunk emission (replaces finalize for rows of few chunk groups): grid (chunks, rows) as select_chunks.  Every
// workgroup of a row resolves the row's exact threshold itself -- the chunk counts, the candidates' keys (bin B) and
// two 10-bit radix passes over them in LDS -- then counts per chunk the candidates above / equal to the threshold
// key, and from the prefix over earlier chunks of (above B + taken candidates) writes its own chunk's taken positions
// in index order (it re-reads its 1024 scores).  Ties at the threshold go to the lowest positions.
// The work is proportional to the candidates (a few percent of the row) per workgroup, and the row's workgroups run
// in parallel where finalize ran one workgroup per row.  Each workgroup clears a slice of the row's histogram as its
// last stores (this kernel reads the threshold bin select_chunks stored, not the histogram).
constexpr int kEmitLead = 32;     // leading candidate keys per chunk brought to LDS with the chunk counts
constexpr int kEmitChunks = 264;  // chunks per row (kMaxBitmapWords bounds n)
static_assert(kMaxBitmapWords * 32 <= kEmitChunks * kChunk && kEmitChunks % 8 == 0, "emit chunk bound");
// Leading keys in LDS: block m (chunks 8m .. 8m+7) at word m * kEmitBlock; key group g (keys 4g .. 4g+3) of chunk q
// at word (q >> 3) * kEmitBlock + 32 g + 4 (q & 7) -- one direct load per block, and the blocks' 32-word offset in
// bank keeps 16 consecutive chunks' reads of one key group on 16 distinct bank quads.
constexpr int kEmitBlock = 8 * kEmitLead + 32;
#ifndef DSV41_EMIT
#define DSV41_EMIT 1
#endif
constexpr bool kEmit = DSV41_EMIT;
#ifndef DSV41_EMIT_MAX_GRID
#define DSV41_EMIT_MAX_GRID 2048
#endif
constexpr long kEmitMaxGrid = DSV41_EMIT_MAX_GRID;  // emit grids up to this many workgroups (each redoes the radix)

// Thread t owns chunks t*nch/256 .. (t+1)*nch/256 - 1 (at most CPT = 1 or 2): thread order is chunk order, so block
// scans over the threads give prefixes over chunks.  The first kEmitLead candidate keys of every chunk come to LDS by
// direct loads issued with the counts (8 chunks per wave instruction); each pass over the candidates (the two radix
// histograms, the per-chunk tally) walks the owned chunks' keys there, the rest of a chunk (rare) from the
// workspace.  Code is kept loop-shaped and LDS traffic low: the kernel is latency-bound.
template <int CPT>
__global__ void __launch_bounds__(256) emit_kernel(const SelArgs a) {
  __shared__ uint32_t sk[kEmitChunks / 8 * kEmitBlock];
  __shared__ int hist0[1024], hist1[1024];
  __shared__ int2 t0[4], t1[4], t2[4], t3[4];
  __shared__ int s_d0, s_r0, s_d1, s_r1, s_out0, s_eq0;
  DSV41_TS(0);
  const int ch = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = row_c(a, r), k = a.k;
  int* orow = a.out + (long)r * a.out_rstride;
  int* gh = a.hist + (long)r * kBins;
  if (c <= k) {  // every valid position, then -1
    if (ch == 0) {
#pragma unroll 1
      for (int i = tid; i < k; i += 256) orow[i] = i < c ? i + a.offset : -1;
#pragma unroll 1
      for (int i = tid; i < kBins; i += 256) gh[i] = 0;
    }
    return;
  }
  const int nch = (c + kChunk - 1) / kChunk;
  if (ch >= nch) return;
  // chunk scores (4 consecutive positions per thread), the owned chunks' counts, every chunk's leading keys
  const int p0 = ch * kChunk + 4 * tid;
  const float* srow = a.score + (long)r * a.ld;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = srow[p0 + e < c ? p0 + e : 0];
  const int B = a.rowbin[r];
  const long reg = (long)r * a.rs;
#pragma unroll 1
  for (int m = wave; 8 * m < nch; m += 4) {  // (a chunk's region holds kChunk keys: reads past its count stay inside)
    const int q = min(8 * m + (lane & 7), nch - 1);
    lds_dma16_at(a.cand_key + reg + (long)q * kChunk + 4 * (lane >> 3), lds_addr_of(sk) + m * kEmitBlock * 4);
  }
  const int qb = (tid * nch) >> 8, qe = ((tid + 1) * nch) >> 8;
  int na[CPT], nc[CPT], la = 0, lc = 0;
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    int2 cv = make_int2(0, 0);
    if (qb + u < qe) cv = *(const int2*)(a.counts + ((long)r * a.nchunks + qb + u) * 2);
    na[u] = cv.x;
    nc[u] = cv.y;
    la += cv.x;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    hist0[4 * tid + u] = 0;
    hist1[4 * tid + u] = 0;
  }
  int2 tot;
  const int2 ex = block_scan2_dpp<256>(la, 0, t0, &tot);  // above-B entries in earlier threads' chunks
  const int need = k - tot.x;  // candidates to take (<= 0: the above entries alone reach k)
  int pa_ch = 0;               // above-B entries before chunk ch (meaningful in its owner thread)
  {
    int ea = ex.x;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      pa_ch = qb + u == ch ? ea : pa_ch;
      ea += na[u];
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the direct loads into sk
  __syncthreads();
  DSV41_TS(1);
  // fn(u, key) for every candidate of owned chunk u: the leading keys from sk (8 per LDS round trip), the rest of a
  // chunk from the workspace (8 per round trip; reads stay inside the chunk's region)
  auto visit = [&](auto&& fn) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int q = qb + u, n = nc[u];
#pragma unroll 1
      for (int i0 = 0; i0 < min(n, kEmitLead); i0 += 8) {
        const uint32_t* row = &sk[(q >> 3) * kEmitBlock + (i0 / 4) * 32 + 4 * (q & 7)];
        const uint4 x = *(const uint4*)row, y = *(const uint4*)(row + 32);
        const uint32_t kk[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (i0 + e < n) fn(u, kk[e]);
      }
      const uint32_t* base = a.cand_key + reg + (long)q * kChunk;
#pragma unroll 1
      for (int i0 = kEmitLead; i0 < n; i0 += 8) {
        const uint4 x = *(const uint4*)(base + i0), y = *(const uint4*)(base + i0 + 4);
        const uint32_t kk[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (i0 + e < n) fn(u, kk[e]);
      }
    }
  };
  // the digit (of 1023 - 4t - u, thread t) holding the rank-th largest entry of h, and the rank within it
  auto find_digit = [&](const int* h, int rank, int2* tmp, int* s_d, int* s_r) {
    int hb[4], local = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      hb[u] = h[1023 - 4 * tid - u];
      local += hb[u];
    }
    int2 t;
    int greater = block_scan2_dpp<256>(local, 0, tmp, &t).x;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (greater < rank && rank <= greater + hb[u]) {
        *s_d = 1023 - 4 * tid - u;
        *s_r = rank - greater;
      }
      greater += hb[u];
    }
    __syncthreads();
  };
  uint32_t T = 0xffffffffu;  // threshold key (candidates above it are taken, `remaining` equal ones)
  int remaining = 0;
  int g[CPT], e[CPT];  // per owned chunk: candidates above / equal to T
#pragma unroll
  for (int u = 0; u < CPT; ++u) g[u] = e[u] = 0;
  if (need > 0) {
    visit([&](int, uint32_t key) { atomicAdd(&hist0[(key >> 10) & 1023], 1); });  // bits 19..10 (bin: 31..20)
    __syncthreads();
    find_digit(hist0, need, t1, &s_d0, &s_r0);
    const uint32_t d0 = (uint32_t)s_d0;
    visit([&](int, uint32_t key) {  // bits 9..0 of the candidates with digit d0
      if (((key >> 10) & 1023) == d0) atomicAdd(&hist1[key & 1023], 1);
    });
    __syncthreads();
    find_digit(hist1, s_r0, t2, &s_d1, &s_r1);
    T = ((uint32_t)B << 20) | (d0 << 10) | (uint32_t)s_d1;
    remaining = s_r1;
    visit([&](int u, uint32_t key) {
#pragma unroll
      for (int w = 0; w < CPT; ++w) {
        g[w] += w == u && key > T;
        e[w] += w == u && key == T;
      }
    });
  }
  DSV41_TS(4);
  // Equal candidates are taken lowest position first, so the equal ones taken before chunk q are
  // min(remaining, equal candidates before q), and chunk q's output offset is
  // (above B before q) + (candidates above T before q) + that.
  {
    int lg = 0, le = 0;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      lg += g[u];
      le += e[u];
    }
    int2 gx = block_scan2_dpp<256>(lg, le, t3, &tot);
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      if (qb + u == ch) {
        s_out0 = pa_ch + gx.x + min(remaining, gx.y);
        s_eq0 = gx.y;
      }
      gx.x += g[u];
      gx.y += e[u];
    }
  }
  __syncthreads();
  DSV41_TS(5);
  const int out0 = s_out0, avail = max(0, remaining - s_eq0);  // equal candidates this chunk may take
  // ---- this chunk's taken positions in index order
  int ne = 0, ns = 0;
  bool is_eq[4], strict[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool in = p0 + i < c;
    const uint32_t key = score_key(v[i]);
    const int b = (int)(key >> 20);
    is_eq[i] = in && need > 0 && b == B && key == T;
    strict[i] = in && (b > B || (need > 0 && b == B && key > T));
    ne += is_eq[i];
    ns += strict[i];
  }
  const int2 px = block_scan2_dpp<256>(ne, ns, t0, &tot);
  int er = px.x, o = out0 + px.y + min(px.x, avail);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (strict[i] || (is_eq[i] && er < avail)) {
      if (o < k) orow[o] = p0 + i + a.offset;
      ++o;
    }
    er += is_eq[i];
  }
  DSV41_TS(6);
  // the row's histogram back to zero for the next step, a slice per chunk (last: no wait ever covers these stores)
  const int per = (kBins + nch - 1) / nch, h1 = min(kBins, (ch + 1) * per);
#pragma unroll 1
  for (int i = ch * per + tid; i < h1; i += 256) gh[i] = 0;
}

// ------------------------------------------------------------------------------------------------ one launch
// Rows of at most kGroupPerXcd chunks: the chunks of a row form one group of workgroups on one XCD (row r on XCD
// r / rpx; workgroup b runs on XCD b % 8), all resident at once, that meet once at a per-row barrier:
//   A. scores of the chunk (4 positions per thread), the row's histogram and length: one round trip
//   B. threshold bin B (where the running count from the top reaches k); need = k - (entries above B)
//   C. classify: entries above B are counted; bin-B candidates are stored as key << 32 | ~position (a larger value
//      is the better candidate: higher key, then lower position) in the chunk's slot region, with the counts
//   D. barrier: a 64-bit arrival counter per row that only grows (launch e waits for (e + 1) * slots arrivals)
//   E. the counts of every chunk and the first kGroupSpec candidates of each chunk in one round trip
//   F. unless all of bin B is taken: T = the candidate of rank need - 1 (rank = candidates larger than it)
//   G. the chunk's taken positions (above B, or candidates >= T) at offset sum over earlier chunks of
//      (above + taken candidates) plus the in-chunk prefix.
// A workgroup that finds itself off its XCD publishes with a device-scope fence and adds kAwayFlag to its arrival;
// readers that see any such flag (or are misplaced themselves) acquire with a device-scope fence, so results never
// depend on placement (a workspace that ever saw a misplaced workgroup keeps taking the fenced exchange).
constexpr int kGroupPerXcd = 64;   // 2 per CU of a 32-CU XCD: every chunk of a row is resident at the barrier
constexpr int kGroupSpec = 32;     // candidates per chunk read together with the counts
constexpr int kGroupCand = 2048;   // candidates staged in LDS (more: read from the workspace)
constexpr int kSpinLimit = 1 << 22;
constexpr unsigned long long kAwayFlag = 1ull << 48, kArriveMask = kAwayFlag - 1;

struct GroupArgs {
  SelArgs s;
  unsigned long long* cand;   // [R, rs] (chunk ch: slots ch * kChunk ..)
  unsigned long long* epoch;  // [R] arrival counters (bits 0..47: arrivals; 48..: misplaced arrivals)
  int* err;                   // set when a barrier wait gives up (kSpinLimit polls)
  int rpx;                    // rows per XCD
};

// The rows' arrival counters (u64) lie 128 bytes apart: device-scope atomics on one cache line serialise at the
// memory side.
constexpr int kEpochStride = 16;

__global__ void __launch_bounds__(256) select_group_kernel(const GroupArgs g) {
  const SelArgs& a = g.s;
  const int home = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int ch = j % a.nchunks, r = home * g.rpx + j / a.nchunks;
  if (r >= a.R) return;
  __shared__ int tmp[4];
  __shared__ int s_bin, s_need, s_cnt, s_selb;
  __shared__ int wcnt[4][2];
  __shared__ int pc[kGroupPerXcd + 1];
  __shared__ int na_q[kGroupPerXcd], nc_q[kGroupPerXcd];
  __shared__ unsigned long long lc[kGroupCand + 2];  // (+ a zero pad after the last candidate)
  __shared__ RankScratch rs;
  __shared__ int s_over;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nslots = a.nchunks;
  DSV41_PH(0);
  // ---- A. loads
  const long cl = a.cl[r];
  const int p = ch * kChunk + 4 * t;
  const float4 v = p < a.n ? *(const float4*)(a.score + (long)r * a.ld + p) : make_float4(0.f, 0.f, 0.f, 0.f);
  int* gh = a.hist + (long)r * kBins;
  int4 h4[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) h4[u] = *(const int4*)(gh + kBins - 16 * (t + 1) + 4 * u);
  const int c = (int)(cl < 0 ? 0 : (cl > a.n ? a.n : cl)), k = a.k;
  int* orow = a.out + (long)r * a.out_rstride;
  unsigned long long* ep = g.epoch + (long)r * kEpochStride;
  const int zb = (kBins + nslots - 1) / nslots, z0 = ch * zb, z1 = min(kBins, z0 + zb);  // histogram slice to clear
  if (c <= k) {  // everything is selected; arrive without waiting (keeps the epoch count)
    if (ch == 0) {
#pragma unroll 1
      for (int i = t; i < k; i += 256) orow[i] = i < c ? i + a.offset : -1;
    }
#pragma unroll 1
    for (int i = z0 + t; i < z1; i += 256) gh[i] = 0;
    if (t == 0) __hip_atomic_fetch_add(ep, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // ---- B. threshold bin (thread t: bins 4095-16t down to 4080-16t)
  if (t == 0) {  // (a histogram holding fewer than k entries of a row longer than k is a caller error)
    s_bin = 0;
    s_need = k;
    s_cnt = 0;
  }
  {
    const int h[16] = {h4[3].w, h4[3].z, h4[3].y, h4[3].x, h4[2].w, h4[2].z, h4[2].y, h4[2].x,
                       h4[1].w, h4[1].z, h4[1].y, h4[1].x, h4[0].w, h4[0].z, h4[0].y, h4[0].x};
    int local = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) local += h[i];
    int total;
    int above = block_scan_dpp<256>(local, tmp, &total);
    if (above < k && k <= above + local) {
#pragma unroll 1
      for (int i = 0; i < 16; ++i) {
        if (k <= above + h[i]) {
          s_bin = kBins - 1 - 16 * t - i;
          s_need = k - above;
          s_cnt = h[i];
          break;
        }
        above += h[i];
      }
    }
    __syncthreads();
  }
  DSV41_PH(1);
  const uint32_t lo = (uint32_t)s_bin << 20, hi = (uint32_t)(s_bin + 1) << 20;  // bin B = [lo, hi)
  const int need = s_need, cnt = s_cnt;
  // ---- C. classify
  const uint32_t key[4] = {score_key(v.x), score_key(v.y), score_key(v.z), score_key(v.w)};
  int na = 0, nc = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bool ok = p + e < c;
    na += ok && key[e] >= hi;
    nc += ok && key[e] >= lo && key[e] < hi;
  }
  const int ia = wave_incl_scan(na), ic = wave_incl_scan(nc);
  if (lane == 63) {
    wcnt[wave][0] = ia;
    wcnt[wave][1] = ic;
  }
  __syncthreads();
  int cbase = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) cbase += w < wave ? wcnt[w][1] : 0;
  unsigned long long* crow = g.cand + (long)r * a.rs;
  if (nc > 0) {
    int o = ch * kChunk + cbase + ic - nc;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (p + e < c && key[e] >= lo && key[e] < hi)
        crow[o++] = (unsigned long long)key[e] << 32 | (uint32_t)~(uint32_t)(p + e);
  }
  if (t == 0) {
    const int ta = wcnt[0][0] + wcnt[1][0] + wcnt[2][0] + wcnt[3][0];
    const int tc = wcnt[0][1] + wcnt[1][1] + wcnt[2][1] + wcnt[3][1];
    *(int2*)(a.counts + ((long)r * nslots + ch) * 2) = make_int2(ta, tc);
  }
  // ---- D. row barrier
  DSV41_PH(2);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const bool away = xcd_id() != home;
    if (away) __threadfence();
    const unsigned long long old =
        __hip_atomic_fetch_add(ep, away ? 1ull + kAwayFlag : 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long target = ((old & kArriveMask) / nslots + 1) * nslots;
    unsigned long long cur;
    int spins = 0;
    while (((cur = __hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) & kArriveMask) < target &&
           spins < kSpinLimit) {
      __builtin_amdgcn_s_sleep(2);
      ++spins;
    }
    if (spins >= kSpinLimit) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (away || cur >= kAwayFlag) __threadfence();  // some workgroup of this workspace ever ran off its XCD
  }
  __syncthreads();
  DSV41_PH(3);
  // the histogram is consumed (every chunk read it before arriving)
#pragma unroll 1
  for (int i = z0 + t; i < z1; i += 256) gh[i] = 0;
  // ---- E. counts of all chunks + speculative candidate prefixes
  if (t < nslots) {
    const long long cv = __hip_atomic_load((long long*)(a.counts + ((long)r * nslots + t) * 2), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    na_q[t] = (int)(cv & 0xffffffff);
    nc_q[t] = (int)(cv >> 32);
  }
  constexpr int kSpecPer = kGroupPerXcd * kGroupSpec / 256;
  unsigned long long sv[kSpecPer];
#pragma unroll
  for (int u = 0; u < kSpecPer; ++u) {
    const int idx = u * 256 + t, q = idx / kGroupSpec, e = idx % kGroupSpec;
    sv[u] = q < nslots ? crow[q * kChunk + e] : 0ull;
  }
  __syncthreads();
  if (wave == 0) {  // prefix of the candidate counts; entries above B in earlier chunks; largest chunk count
    const int x = lane < nslots ? nc_q[lane] : 0;
    const int ix = wave_incl_scan(x);
    pc[lane + 1] = ix;
    if (lane == 0) pc[0] = 0;
    const int y = lane < ch ? na_q[lane] : 0;
    const int iy = wave_incl_scan(y);
    if (lane == 63) s_selb = iy;
    const bool over = __ballot(x > kGroupSpec) != 0;
    if (lane == 0) s_over = over;
    const int mtot = __shfl(ix, 63, 64);
    if (lane == 0 && mtot <= kGroupCand) lc[mtot] = 0ull;  // pad for pairwise reads
  }
  __syncthreads();
  const int m = pc[nslots];
  const bool staged = m <= kGroupCand;
#pragma unroll
  for (int u = 0; u < kSpecPer; ++u) {
    const int idx = u * 256 + t, q = idx / kGroupSpec, e = idx % kGroupSpec;
    if (staged && q < nslots && e < nc_q[q]) lc[pc[q] + e] = sv[u];
  }
  if (staged && s_over) {  // chunks with more than kGroupSpec candidates
#pragma unroll 1
    for (int q = 0; q < nslots; ++q)
      for (int e = kGroupSpec + t; e < nc_q[q]; e += 256) lc[pc[q] + e] = crow[q * kChunk + e];
  }
  __syncthreads();
  auto cand_at = [&](int i) -> unsigned long long {
    if (staged) return lc[i];
    int q = 0;
    while (pc[q + 1] <= i) ++q;
    return crow[q * kChunk + (i - pc[q])];
  };
  DSV41_PH(4);
  // ---- F. threshold candidate
  const unsigned long long T = threshold_candidate(cand_at, lc, staged, m, need, lo, rs);
  int sb = 0;  // taken candidates of earlier chunks
#pragma unroll 1
  for (int i = t; i < pc[ch]; i += 256) sb += cand_at(i) >= T;
  int tot;
  block_scan_dpp<256>(sb, tmp, &tot);
  const int base = s_selb + tot;
  DSV41_PH(5);
  // ---- G. ordered emission of this chunk
  bool take[4];
  int nt = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bool ok = p + e < c;
    take[e] = ok && (key[e] >= hi ||
                     (key[e] >= lo && ((unsigned long long)key[e] << 32 | (uint32_t)~(uint32_t)(p + e)) >= T));
    nt += take[e];
  }
  int o = base + block_scan_dpp<256>(nt, tmp, &tot);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (take[e]) orow[o++] = p + e + a.offset;
  DSV41_PH(6);
}

// Workspace: histograms [R, kBins] | chunk counts [R, nch, 2] | above, candidate positions, candidate keys [R, rs]
// each (rs = n rounded up to 32, so rows never share a cache line; the one-launch path uses the first two as 64-bit
// candidate slots [R, rs]) | threshold bins [R] (padded to 8 bytes) | arrival counters [R] (64-bit) | timeout flag.
long row_stride(int n) { return ((long)n + 31) / 32 * 32; }
// Chunk count pairs, rounded up to 16 bytes: the per-chunk regions after them stay 16-byte aligned (the emission's
// vector and direct-to-LDS loads of candidate keys).
long count_ints(int R, long nch) { return ((long)R * nch * 2 + 3) / 4 * 4; }

long select_base_bytes(int R, int n) {
  const long nch = (n + kChunk - 1) / kChunk;
  return ((long)R * kBins + count_ints(R, nch) + 3L * R * row_stride(n) + (R + 1L) / 2 * 2) * 4;  // (+ row bins)
}

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_ts(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ts), sizeof(g_dsv41_ts)); }
int dsv41_read_ph_sel(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ph), sizeof(g_dsv41_ph)); }
int dsv41_read_ck_sel(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ck), sizeof(g_dsv41_ck)); }
#endif

long dsv41_select_workspace_bytes(int R, int n) {
  return select_base_bytes(R, n) + (R * (long)kEpochStride + 2L) * 8;  // + per-row arrival counters, timeout flag
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
  a.rs = row_stride(n);
  a.above = a.counts + count_ints(R, nch);
  a.cand_idx = a.above + (long)R * a.rs;
  a.cand_key = (uint32_t*)(a.cand_idx + (long)R * a.rs);
  a.nchunks = nch;
  a.out = out;
  a.out_rstride = out_rstride;
  a.offset = offset;
  hipStream_t st = (hipStream_t)stream;
  const int rpx = (R + kXcds - 1) / kXcds;
  if (rpx * nch <= kGroupPerXcd && ld % 4 == 0 && ((uintptr_t)score & 15) == 0) {  // one launch
    GroupArgs g{a, (unsigned long long*)a.above, nullptr, nullptr, rpx};
    unsigned long long* ctl = (unsigned long long*)((char*)ws + select_base_bytes(R, n));
    g.epoch = ctl;
    g.err = (int*)(ctl + (long)R * kEpochStride);
    select_group_kernel<<<kXcds * rpx * nch, 256, 0, st>>>(g);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  a.rowbin = (int*)(a.cand_key + (long)R * a.rs);
  select_chunks_kernel<<<dim3(nch, R), 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  if ((long)R * nch <= kEmitMaxGrid && kEmit) {  // few rows: every chunk's workgroup emits its own positions
    if (nch <= 256) emit_kernel<1><<<dim3(nch, R), 256, 0, st>>>(a);
    else emit_kernel<2><<<dim3(nch, R), 256, 0, st>>>(a);
  } else {
    finalize_kernel<<<R, kFinThreads, 0, st>>>(a);
  }
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
