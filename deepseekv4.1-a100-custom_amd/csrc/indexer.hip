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
// column tiles of 16 keys, loads issued before the query preparation); the query fragments live in VGPRs.  MFMA output layout: lane l holds key (l & 15) and
// heads 4*(l >> 4) + i, so the head reduction is 16 in-lane FMAs plus two cross-lane shuffles.
// Keys at positions >= cl are never read: the scan is bounded by the valid count, not the allocated capacity.
#include "score_core.h"

#include <type_traits>

namespace {

template <int KFMT, bool HIST, int WV = 4>
__global__ void __launch_bounds__(64 * WV) index_score_kernel(const ScoreArgs a, int nx) {
  // 1-D grid: block b runs on XCD b % 8 (round-robin dispatch); key chunk x belongs to XCD x % 8 and its R rows
  // follow one another there, so rows of one sequence (MTP drafts) read the chunk's keys from that XCD's L2
  const int bxcd = blockIdx.x % kXcds, bj = blockIdx.x / kXcds;
  const int by = bj % a.R, bx = (bj / a.R) * kXcds + bxcd;
  if (bx >= nx) return;
  if (!a.write_masked) {  // a workgroup wholly past its row's valid count has nothing to score or count
    long cl0 = row_cl(a, by);
    if (cl0 > a.n_pos) cl0 = a.n_pos;
    if ((long)bx * (WV * kKeysPerWave) >= cl0) return;
  }
  DSV41_TS(30);
  DSV41_WG_TS(0);
  if (by == 0) DSV41_PH(0);
  __shared__ int lhist[HIST ? kHistBins : 1];
  const int r = by;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (HIST) {
#pragma unroll 1
    for (int i = threadIdx.x; i < kHistBins; i += 64 * WV) lhist[i] = 0;
    __syncthreads();
  }
  const int l16 = lane & 15, g = lane >> 4;
  const int kt0 = bx * (WV * kKeysPerWave) + wave * kKeysPerWave;
  long cl = row_cl(a, r);
  if (cl > a.n_pos) cl = a.n_pos;
  float* orow = a.out + (long)r * a.out_rstride;
  if (kt0 >= cl) {  // nothing to score in this wave (the whole-block barrier below is still reached)
    if (a.write_masked)
      for (int t = kt0 + lane; t < kt0 + kKeysPerWave && t < a.n_pos; t += 64) orow[t] = -__builtin_inff();
    if (!HIST) return;
  } else {
  if (by == 0) DSV41_PH(1);
  const long slot = a.seq ? a.seq[r] : (long)(r / a.rows_per_slot);
  const int nht = (a.HI + 15) / 16;
  const int lim = (int)cl;

  // ---- issue the key loads of the first column tiles before the query preparation
  constexpr int NT = 4;  // column tiles prefetched per round
  uint4 k0[NT], k1[NT];
  uint4 kb16[NT][4];
  float ksc[NT];
  auto load_round = [&](int base) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int t = base + nt * 16 + l16;
      const bool tv = t < lim;
      if (KFMT == 1) {
        const uint8_t* krow = (const uint8_t*)a.keys + slot * a.k_sstride + (long)t * 128 + g * 32;
        k0[nt] = tv ? *(const uint4*)krow : make_uint4(0, 0, 0, 0);
        k1[nt] = tv ? *(const uint4*)(krow + 16) : make_uint4(0, 0, 0, 0);
        ksc[nt] = tv ? a.kscale[slot * a.ks_sstride + t] : 0.0f;
      } else {
        const uint16_t* krow = (const uint16_t*)a.keys + slot * a.k_sstride + (long)t * 128 + g * 8;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) kb16[nt][ks] = tv ? *(const uint4*)(krow + ks * 32) : make_uint4(0, 0, 0, 0);
        ksc[nt] = 1.0f;
      }
    }
  };
  load_round(kt0);

  // ---- query fragments and head weights.  e4m3 keys: q is the prepared e4m3 query [64 heads][128 bytes] and w the
  // folded weights [64] (dsv41_index_qprep); bf16 keys: q is bf16 [HI][128] and w fp32 [HI].
  i32x8_t qa8[kHT];
  uint4 qa16[kHT][4];
  float wl[kHT];  // weight of head ht*16 + l16
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    const int h = ht * 16 + l16;
    const bool hv = ht < nht && h < a.HI;
    const int hc = hv ? h : 0;
    if (KFMT == 1) {
      const uint4* qrow = (const uint4*)((const uint8_t*)a.q + (long)r * a.q_rstride + (long)hc * 128 + g * 32);
      const uint4 u0 = qrow[0], u1 = qrow[1];
      qa8[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
    } else {
      const uint16_t* qrow = a.q + (long)r * a.q_rstride + (long)hc * 128;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qa16[ht][ks] = *(const uint4*)(qrow + ks * 32 + g * 8);
    }
    wl[ht] = a.w[(long)r * a.w_rstride + hc];
    if (!hv) wl[ht] = 0.0f;
  }
  DSV41_TS(31);
  if (by == 0) DSV41_PH(2);
  float wr[kHT][4];  // weights of the heads this lane's accumulators hold: ht*16 + 4g + i
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wl[ht], 4 * g + i, 64);

  for (int base = kt0; base < kt0 + kKeysPerWave; base += NT * 16) {
    if (base != kt0) load_round(base);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int t = base + nt * 16 + l16;
      const float sum = score_tile<KFMT>(qa8, qa16, wr, nht, k0[nt], k1[nt], kb16[nt]);
      if (g == 0 && t < a.n_pos) {
        if (t < lim) {
          const float v = is_cand(a, r, t) ? sum * ksc[nt] : -__builtin_inff();
          orow[t] = v;
          if (HIST) atomicAdd(&lhist[score_key(v) >> 20], 1);
        } else if (a.write_masked) {
          orow[t] = -__builtin_inff();
        }
      }
    }
  }
  }  // kt0 < cl
  DSV41_TS(32);
  if (by == 0) DSV41_PH(3);
  if (HIST) {
    __syncthreads();
    int* gh = a.hist + (long)r * kHistBins;
    if (((uintptr_t)gh & 7) == 0) {
#pragma unroll 1
      for (int i = threadIdx.x; i < kHistBins / 2; i += 64 * WV) {  // bins in pairs: one 64-bit add (no carry
        const uint32_t lo = (uint32_t)lhist[2 * i], hi = (uint32_t)lhist[2 * i + 1];  // out of a bin: < 2^32)
        if (lo | hi) atomicAdd((unsigned long long*)(gh + 2 * i), ((unsigned long long)hi << 32) | lo);
      }
    } else {
#pragma unroll 1
      for (int i = threadIdx.x; i < kHistBins; i += 64 * WV) {
        const int v = lhist[i];
        if (v) atomicAdd(&gh[i], v);
      }
    }
  }
  if (by == 0) DSV41_PH(4);
  DSV41_WG_TS(1);
}

constexpr int kLoopMaxRows = 64;  // rows of the grouped decode score kernel's tables

// Prefill score kernel (many query rows of one sequence; e4m3 keys + prepared e4m3 queries): a workgroup owns 8
// consecutive query rows (one per wave, 8 waves) and a range of key positions, streamed through LDS in 256-key chunks
// (direct-to-LDS loads, double buffered) and shared by the 8 waves.  Per step a wave runs its row's 4 head tiles of
// 16x16x128 fp8 MFMAs on two 16-key B fragments, then the two epilogues (ReLU, weighted head sum).  One row per wave
// keeps a wave under 128 VGPRs: four waves per SIMD hide the MFMA and LDS latencies of each other's steps (two rows
// per wave held 228 VGPRs, two waves per SIMD).  Key tiles past a row's causal limit are skipped.
constexpr int kPQ = 8;        // query rows per workgroup
constexpr int kPThreads = 512;
constexpr int kPChunk = 256;  // keys per LDS chunk (32 KB)

template <int NHT>  // 16-head tiles: ceil(HI / 16)
__global__ void __launch_bounds__(kPThreads, 2) index_score_prefill_kernel(const ScoreArgs a, int key_split) {
  __shared__ __align__(16) uint8_t kbuf[2][kPChunk * 128];
  __shared__ float sbuf[2][kPChunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int r0 = blockIdx.y * kPQ;
  const int slot = r0 / a.rows_per_slot;  // all rows of a block belong to one sequence (host-checked)
  // causal limits of the block's rows (increasing with the row)
  long cl_hi = row_cl(a, min(r0 + kPQ, a.R) - 1);
  if (cl_hi > a.n_pos) cl_hi = a.n_pos;
  const int span = (a.n_pos + key_split - 1) / key_split;
  const int kb0 = blockIdx.x * span;
  const int kb1 = min((long)(kb0 + span), cl_hi);
  if (kb0 >= kb1) return;
  const uint8_t* kbase = (const uint8_t*)a.keys + (long)slot * a.k_sstride;
  const float* sbase = a.kscale + (long)slot * a.ks_sstride;
  const int nchunks = (kb1 - kb0 + kPChunk - 1) / kPChunk;
  // (direct-to-LDS loads as inline assembly: the compiler does not wait for them before every LDS read; the
  // chunk loop waits for them explicitly)
  const uint32_t kb_lds = lds_addr_of(&kbuf[0][0]), sb_lds = lds_addr_of(&sbuf[0][0]);
  auto issue = [&](int ci) {  // 256 keys x 128 B = 2048 chunks of 16 B: 4 per thread; + 256 scales
    const int c0 = kb0 + ci * kPChunk;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // LDS unit q holds key q / 8, 16-byte part (q % 8) ^ (key % 8) (XOR swizzle against bank conflicts)
      const int q = u * kPThreads + threadIdx.x;
      const int kl = q >> 3;
      int key = c0 + kl;
      key = key < kb1 ? key : kb1 - 1;
      lds_dma16_at(kbase + (long)key * 128 + ((q & 7) ^ (kl & 7)) * 16,
                   kb_lds + (uint32_t)((ci & 1) * kPChunk * 128 + (u * kPThreads + wave * 64) * 16));
    }
    if (wave < 4) {
      int key = c0 + threadIdx.x;
      key = key < kb1 ? key : kb1 - 1;
      lds_dma4_at(sbase + key, sb_lds + (uint32_t)((ci & 1) * kPChunk + wave * 64) * 4);
    }
  };
  issue(0);
  // query fragments of this wave's row and its head weights
  i32x8_t qa[kHT];
  float wr[kHT][4];
  constexpr int nht = NHT;
  const int row = r0 + wave;
  {
    const int r = min(row, a.R - 1);
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      const int h = ht * 16 + l16;
      const bool hv = ht < nht && h < a.HI;
      const uint4* qrow = (const uint4*)((const uint8_t*)a.q + (long)r * a.q_rstride + (long)(hv ? h : 0) * 128 + g * 32);
      const uint4 u0 = qrow[0], u1 = qrow[1];
      qa[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
      const float wv = hv ? a.w[(long)r * a.w_rstride + h] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wv, 4 * g + i, 64);
    }
  }
  long clr = row < a.R ? row_cl(a, row) : 0;
  if (clr > a.n_pos) clr = a.n_pos;
  const long wave_lim = clr < kb1 ? clr : kb1;
  float* orow = a.out + (long)(row < a.R ? row : 0) * a.out_rstride;
  for (int ci = 0; ci < nchunks; ++ci) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (ci + 1 < nchunks) issue(ci + 1);
    const int c0 = kb0 + ci * kPChunk;
    const uint8_t* kb = kbuf[ci & 1];
    const float* sb = sbuf[ci & 1];
    // two 16-key tiles per step: all 2 x NHT MFMAs first, then the epilogues (the first tile's VALU work covers
    // the second tile's MFMA latency)
#pragma unroll 1
    for (int kt = 0; kt < kPChunk / 16; kt += 2) {
      const int t0 = c0 + kt * 16;
      if (t0 >= wave_lim) break;  // wave-uniform
      f32x4_t acc[2][kHT];  // [tile][head tile]
      const float ksc = sb[(kt + (lane >> 5)) * 16 + l16];  // scale of the key this lane writes
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int kl = (kt + u) * 16 + l16;
        const uint4 k0 = *(const uint4*)(kb + kl * 128 + (((2 * g) ^ (kl & 7)) << 4));
        const uint4 k1 = *(const uint4*)(kb + kl * 128 + (((2 * g + 1) ^ (kl & 7)) << 4));
        const i32x8_t bfrag = i32x8_t{(int)k0.x, (int)k0.y, (int)k0.z, (int)k0.w, (int)k1.x, (int)k1.y, (int)k1.z,
                                      (int)k1.w};
#pragma unroll
        for (int ht = 0; ht < nht; ++ht)
          acc[u][ht] = mfma_fp8_16x16x128(qa[ht], bfrag, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
      }
      // every MFMA of the step is issued before the epilogues start (the empty statements pin the results here)
      if constexpr (NHT == 4)
        __asm__ volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]), "+v"(acc[1][0]),
                         "+v"(acc[1][1]), "+v"(acc[1][2]), "+v"(acc[1][3]));
      float xs[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float part[kHT] = {0.0f, 0.0f, 0.0f, 0.0f};  // one chain per head tile
#pragma unroll
        for (int ht = 0; ht < nht; ++ht)
#pragma unroll
          for (int i = 0; i < 4; ++i) part[ht] += wr[ht][i] * relu(acc[u][ht][i]);
        xs[u] = (part[0] + part[1]) + (part[2] + part[3]);
      }
      // both tiles' head sums in one reduction: tile (lane >> 5) in each half; lanes 0-15 and 32-47 write
      const float sum = row_sum4_pair(xs[0], xs[1]);
      const int uu = lane >> 5;
      const int t = t0 + uu * 16 + l16;
      if ((g & 1) == 0 && row < a.R && t < wave_lim)
        orow[t] = is_cand(a, row, t) ? sum * ksc : -__builtin_inff();
    }
  }
}

// Decode rows with e4m3 keys and a histogram, grouped by sequence (a sequence's draft rows are consecutive rows with
// the same slot): a group is a run of up to 6 consecutive rows of one slot, and its key chunks (256 keys, the
// group's longest valid count) are streamed through LDS once for all its rows (direct-to-LDS loads, double
// buffered).  Two waves per row score its two 128-key halves of the chunk with the row's query fragments in VGPRs
// (12 waves, three per SIMD, one workgroup per CU; the next 32-key pair's fragments are read before the current
// pair's epilogue).  Work items are the (group, chunk) pairs, numbered per XCD (chunk c on XCD c mod 8) and taken
// in contiguous runs.  Each row's histogram is counted in LDS as 16-bit bins (two per word; a run adds at most 255
// chunks of 256 keys to a bin before it is flushed) and added to the row's device histogram when the run leaves
// the group, after the next item's loads are issued (their wait covers the adds).  Rows of other layouts form
// groups of one row (correct, slower).
constexpr int kGRows = 6;                          // rows per group
constexpr int kGSplit = 2;                         // waves per row (each scores a 1/kGSplit slice of the chunk)
constexpr int kGThreads = 64 * kGRows * kGSplit;   // 12 waves: three per SIMD
constexpr int kGFlushItems = 255;  // chunks counted into the 16-bit bins between flushes
constexpr int kGItemCost = 20, kGStartCost = 13;  // a run's cost per item and per group it starts (~3.1 / ~2 us)

__global__ void __launch_bounds__(kGThreads, 1) index_score_group_kernel(const ScoreArgs a) {
  __shared__ __align__(16) uint8_t kbuf[2][kPChunk * 128];
  __shared__ float sbuf[2][kPChunk];
  __shared__ uint32_t gh[kGRows][kHistBins / 2];
  __shared__ int gstart[kLoopMaxRows + 1];  // group g: rows [gstart[g], gstart[g + 1])
  __shared__ int gpre[kLoopMaxRows + 1];    // items of this XCD in groups < g
  __shared__ int gwpre[kLoopMaxRows + 1];   // their cost (kGItemCost per item + kGStartCost per group started)
  __shared__ int glim[kLoopMaxRows];        // longest valid count of group g (clamped to n_pos)
  __shared__ long gslot[kLoopMaxRows];
  __shared__ int rlim[kLoopMaxRows];
  __shared__ int ngroups;
  const int x = blockIdx.x % kXcds, m = blockIdx.x / kXcds, M = gridDim.x / kXcds;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll 1
  for (int i = threadIdx.x; i < kGRows * kHistBins / 2; i += kGThreads) (&gh[0][0])[i] = 0;
  if (wave == 0) {
    // groups: runs of equal slots, split every 8 rows
    const bool in = lane < a.R;
    long s = 0;
    int cl = 0;
    if (in) {
      s = a.seq ? a.seq[lane] : (long)(lane / a.rows_per_slot);
      long c = row_cl(a, lane);
      cl = (int)(c > a.n_pos ? a.n_pos : c);
      rlim[lane] = cl;
    }
    const long sp = __shfl_up(s, 1, 64);
    const bool head = in && (lane == 0 || sp != s);
    const unsigned long long below = (2ull << lane) - 1;  // lanes <= this one
    const unsigned long long hm = __ballot(head) & below;
    const int run0 = 63 - __builtin_clzll(hm | 1ull);
    const bool head2 = in && ((lane - run0) % kGRows == 0);
    const unsigned long long h2 = __ballot(head2);
    const int gi = __popcll(h2 & below) - 1;
    const int G = __popcll(h2);
    // the group's longest count: a max over its rows (at most 8 consecutive lanes)
    int gl = cl;
#pragma unroll
    for (int d = 1; d < kGRows; d <<= 1) {
      const int o = __shfl_down(gl, d, 64);
      const int og = __shfl_down(gi, d, 64);
      if (lane + d < a.R && og == gi) gl = gl > o ? gl : o;
    }
    if (head2) {
      gstart[gi] = lane;
      glim[gi] = gl;
      gslot[gi] = s;
    }
    if (lane == 0) {
      gstart[G] = a.R;
      ngroups = G;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const int G = ngroups;
    int cnt = 0;
    if (lane < G) {
      const int nx = (glim[lane] + kPChunk - 1) / kPChunk;
      cnt = nx > x ? (nx - x + kXcds - 1) / kXcds : 0;
    }
    const int inc = wave_incl_scan(cnt);
    const int winc = wave_incl_scan(cnt > 0 ? cnt * kGItemCost + kGStartCost : 0);
    if (lane < G) gpre[lane + 1] = inc, gwpre[lane + 1] = winc;
    if (lane == 0) gpre[0] = 0, gwpre[0] = 0;
  }
  __syncthreads();
  const int G = ngroups;
  // the workgroup's items: an equal share of the XCD's cost, an item of group g at cost gwpre[g] + start + item *
  // i taken by the share its cost starts in (a run that starts a group pays its histogram flush and query loads)
  auto item_at = [&](long w) {  // the first item whose cost starts at or after w (workgroup-uniform)
    const bool le = lane < G && gwpre[lane] <= w;
    const int g = __popcll(__ballot(le)) - 1;
    if (g < 0) return 0;
    if (g >= G) return gpre[G];
    const long d = w - gwpre[g] - kGStartCost;
    const int cnt = gpre[g + 1] - gpre[g];
    const int i = d <= 0 ? 0 : (int)((d + kGItemCost - 1) / kGItemCost);
    return gpre[g] + (i < cnt ? i : cnt);
  };
  const long wtot = gwpre[G];
  const int j0 = item_at((long)m * wtot / M), j1 = item_at((long)(m + 1) * wtot / M);
  if (j0 >= j1) return;
  struct Item {
    int grp, c0;
  };
  auto locate = [&](int j) {  // (workgroup-uniform)
    const bool le = lane < G && gpre[lane] <= j;
    Item it;
    it.grp = __popcll(__ballot(le)) - 1;
    it.c0 = (x + kXcds * (j - gpre[it.grp])) * kPChunk;
    return it;
  };
  // (direct-to-LDS loads as inline assembly: the compiler does not wait for them before every LDS read; the
  // loop waits for them explicitly)
  const uint32_t kb_lds = lds_addr_of(&kbuf[0][0]), sb_lds = lds_addr_of(&sbuf[0][0]);
  auto issue = [&](const Item& it, int buf) {  // 256 keys x 128 B: 4 16-byte units per thread; + 256 scales
    const long slot = gslot[it.grp];
    const int lim = glim[it.grp];
    const uint8_t* kbase = (const uint8_t*)a.keys + slot * a.k_sstride;
#pragma unroll
    for (int u = 0; u < (kPChunk * 8 + kGThreads - 1) / kGThreads; ++u) {
      // LDS unit q holds key q / 8, 16-byte part (q % 8) ^ (key % 8) (XOR swizzle against bank conflicts)
      const int q = u * kGThreads + threadIdx.x;
      if (u * kGThreads + wave * 64 >= kPChunk * 8) break;  // (wave-uniform)
      const int kl = q >> 3;
      int key = it.c0 + kl;
      key = key < lim ? key : lim - 1;
      lds_dma16_at(kbase + (long)key * 128 + ((q & 7) ^ (kl & 7)) * 16,
                   kb_lds + (uint32_t)(buf * kPChunk * 128 + (u * kGThreads + wave * 64) * 16));
    }
    if (wave < 4) {
      int key = it.c0 + threadIdx.x;
      key = key < lim ? key : lim - 1;
      lds_dma4_at(a.kscale + slot * a.ks_sstride + key, sb_lds + (uint32_t)(buf * kPChunk + wave * 64) * 4);
    }
  };
  i32x8_t qa[kHT];
  float wr[kHT][4];
  auto load_q = [&](int r) {
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      const int h = ht * 16 + l16;
      const bool hv = h < a.HI;
      const uint4* qrow = (const uint4*)((const uint8_t*)a.q + (long)r * a.q_rstride + (long)(hv ? h : 0) * 128 + g * 32);
      const uint4 u0 = qrow[0], u1 = qrow[1];
      qa[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
      const float wv = hv ? a.w[(long)r * a.w_rstride + h] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wv, 4 * g + i, 64);
    }
  };
  auto flush = [&](int grp) {  // the group's LDS histograms into its rows' (16-bit bin pairs -> one 64-bit add)
    __syncthreads();
    const int rs = gstart[grp], nr = gstart[grp + 1] - rs;
#pragma unroll 1
    for (int w = 0; w < nr; ++w) {
      int* dh = a.hist + (long)(rs + w) * kHistBins;
      const bool al = ((uintptr_t)dh & 7) == 0;
#pragma unroll 1
      for (int i = threadIdx.x; i < kHistBins / 2; i += kGThreads) {
        const uint32_t v = gh[w][i];
        if (v) {
          const uint32_t lo = v & 0xffffu, hi = v >> 16;
          if (al) {
            atomicAdd((unsigned long long*)(dh + 2 * i), ((unsigned long long)hi << 32) | lo);
          } else {
            if (lo) atomicAdd(dh + 2 * i, (int)lo);
            if (hi) atomicAdd(dh + 2 * i + 1, (int)hi);
          }
          gh[w][i] = 0;
        }
      }
    }
    __syncthreads();
  };
  Item cur = locate(j0);
  issue(cur, 0);
  int grp = -1, since = 0, row = 0, lim_r = 0;
  const int wrow = wave % kGRows, wpart = wave / kGRows;  // this wave's row of the group and slice of the chunk
  constexpr int kPairs = kPChunk / 32 / kGSplit;          // 32-key tile pairs per slice
#pragma unroll 1
  for (int j = j0; j < j1; ++j) {
    const bool newg = cur.grp != grp;
    const int oldg = grp;
    if (newg) {  // the query of this wave's row of the new group (loaded before the wait below)
      grp = cur.grp;
      const int rs = gstart[grp], nr = gstart[grp + 1] - rs;
      row = wrow < nr ? rs + wrow : -1;
      lim_r = row >= 0 ? rlim[row] : 0;
      load_q(row >= 0 ? row : rs);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this item's keys and the query have landed (and the last flush's adds)
    __syncthreads();                // ... for every wave; every wave is done with the other buffer and the counts
    Item nxt = cur;
    if (j + 1 < j1) {
      nxt = locate(j + 1);
      issue(nxt, (j + 1 - j0) & 1);
    }
    if ((newg && oldg >= 0) || since == kGFlushItems) {  // (after the next item's loads: its wait covers the adds)
      flush(newg ? oldg : grp);
      since = 0;
    }
    ++since;
    const int buf = (j - j0) & 1;
    const uint8_t* kb = kbuf[buf];
    const float* sb = sbuf[buf];
    const int c0 = cur.c0;
    const int wlim = lim_r < c0 + kPChunk ? lim_r : c0 + kPChunk;
    float* orow = a.out + (long)(row >= 0 ? row : 0) * a.out_rstride;
    // 16-key tiles in pairs; the next pair's fragments are read from LDS before this pair's epilogue (whose LDS
    // adds then do not hold up those reads)
    i32x8_t bfr[2][2];
    float bsc[2];  // scale of the key this lane records: tile 2p + (lane >> 5), key l16
    auto frag = [&](int kt, i32x8_t& b) {
      const int kl = kt * 16 + l16;
      const uint4 k0 = *(const uint4*)(kb + kl * 128 + (((2 * g) ^ (kl & 7)) << 4));
      const uint4 k1 = *(const uint4*)(kb + kl * 128 + (((2 * g + 1) ^ (kl & 7)) << 4));
      b = i32x8_t{(int)k0.x, (int)k0.y, (int)k0.z, (int)k0.w, (int)k1.x, (int)k1.y, (int)k1.z, (int)k1.w};
    };
    const int p0 = wpart * kPairs;
    frag(2 * p0, bfr[0][0]);
    frag(2 * p0 + 1, bfr[0][1]);
    bsc[0] = sb[(2 * p0 + (lane >> 5)) * 16 + l16];
#pragma unroll
    for (int pp = 0; pp < kPairs; ++pp) {
      const int cs = pp & 1, p = p0 + pp;
      const int t0 = c0 + p * 32;
      if (t0 >= wlim) break;  // wave-uniform
      f32x4_t acc[2][kHT];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ht = 0; ht < kHT; ++ht)
          acc[u][ht] = mfma_fp8_16x16x128(qa[ht], bfr[cs][u], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
      if (pp + 1 < kPairs) {
        frag(2 * p + 2, bfr[cs ^ 1][0]);
        frag(2 * p + 3, bfr[cs ^ 1][1]);
        bsc[cs ^ 1] = sb[(2 * p + 2 + (lane >> 5)) * 16 + l16];
      }
      __asm__ volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]), "+v"(acc[1][0]),
                       "+v"(acc[1][1]), "+v"(acc[1][2]), "+v"(acc[1][3]));
      float xs[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float part[kHT];
#pragma unroll
        for (int ht = 0; ht < kHT; ++ht) {
          part[ht] = wr[ht][0] * relu(acc[u][ht][0]);
#pragma unroll
          for (int i = 1; i < 4; ++i) part[ht] += wr[ht][i] * relu(acc[u][ht][i]);
        }
        xs[u] = (part[0] + part[1]) + (part[2] + part[3]);
      }
      // both tiles' head sums in one reduction: tile (lane >> 5) in each half; lanes 0-15 and 32-47 record
      const float sum = row_sum4_pair(xs[0], xs[1]);
      const int uu = lane >> 5;
      const int t = t0 + uu * 16 + l16;
      if ((g & 1) == 0 && t < wlim) {
        const float v = is_cand(a, row, t) ? sum * bsc[cs] : -__builtin_inff();
        orow[t] = v;
        const uint32_t bin = score_key(v) >> 20;
        atomicAdd(&gh[wrow][bin >> 1], 1u << ((bin & 1) * 16));
      }
    }
    cur = nxt;
  }
  flush(grp);
}

// ------------------------------------------------------------------------------------------------ top-k

// Lanes 0 .. n-1 as a wave mask (n clamped to 0 .. 64); whether this lane is set in a mask; a lane's rank among
// the set lanes of m below it.
DSV41_DEV unsigned long long lanes_below(int n) {
  return n >= 64 ? ~0ull : (n <= 0 ? 0ull : (1ull << n) - 1ull);
}
DSV41_DEV bool lane_in(unsigned long long m) { return __builtin_amdgcn_inverse_ballot_w64(m); }  // (exec = m)
DSV41_DEV int lane_rank(unsigned long long m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// A wave's pass over positions [i0, i1) in batches of 64 B: key_of(i) for position b0 + 64 u + lane, then
// body(b0, keys, full) -- full (a compile-time flag) when the whole batch lies inside the range, so its reads need
// no clamp; the last, partial batch reads position i1 - 1 in place of those past the range.
template <int B, typename KeyOf, typename Body>
DSV41_DEV void wave_batches(int i0, int i1, int lane, KeyOf key_of, Body body) {
  int b0 = i0;
  for (; b0 + 64 * B <= i1; b0 += 64 * B) {
    uint32_t kk[B];
#pragma unroll
    for (int u = 0; u < B; ++u) kk[u] = key_of(b0 + u * 64 + lane);
    body(b0, kk, std::true_type{});
  }
  if (b0 < i1) {
    uint32_t kk[B];
#pragma unroll
    for (int u = 0; u < B; ++u) kk[u] = key_of(min(b0 + u * 64 + lane, i1 - 1));
    body(b0, kk, std::false_type{});
  }
}

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

// Block-wide exclusive scan of one int per thread (NT threads = NT/64 waves).  Returns the prefix; *total = sum.
template <int NT>
DSV41_DEV int block_excl_scan(int v, int* tmp, int* total) {
  return block_scan_dpp<NT>(v, tmp, total);
}

// Top-k of a row in ascending index order (ties at the threshold taken lowest index first).  Every wave owns a
// contiguous chunk of the row for the counting and emission passes.
// Rows of <= CACHE valid positions (staged in LDS as order-preserving keys): the load also builds a 4096-bin
// histogram of the keys' top 12 bits (sign, exponent, 3 mantissa bits), whose scan gives the bin Bn holding the k-th
// largest key; one pass then counts each wave's entries above Bn and lists its bin-Bn candidates, the exact threshold
// is a radix select over the listed candidates' low 20 bits, and the emission pass places each wave's selected
// indices with ballots: three passes over the row.  Rows not staged, or with more candidates than a wave's list
// holds: radix select on d = key - kmin (the row's own key range) with 11-bit digits from the top of the range down,
// then a counting pass and the emission pass.
template <int NT, int CACHE>
__global__ void __launch_bounds__(NT) topk_kernel(const TopkArgs a) {
  constexpr int kTopkThreads = NT;
  constexpr int kTopkCache = CACHE;
  constexpr int NW = NT / 64;
  constexpr int B = 8;              // independent loads in flight per thread per batch
  constexpr int kList = 2048 / NW;  // candidates listed per wave (the lists reuse the histogram's 8 KB)
  __shared__ uint32_t keys[kTopkCache];
  __shared__ int hist[2048];    // general path: 2048 bins; staged rows: 4096 16-bit bins, then the candidate lists
  __shared__ uint32_t h2[512];  // 1024 16-bit bins over the listed candidates' digits
  __shared__ int scan_tmp[32];
  __shared__ uint32_t red_min[NW], red_max[NW];
  __shared__ int w_gt[NW], w_eq[NW], w_take[NW], w_base[NW], w_nc[NW];
  __shared__ int s_digit, s_rem, s_bin, s_over;
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: the wave's chunk bounds and masks stay scalar)
  const float* row = a.score + (long)r * a.ld;
  int* orow = a.out + (long)r * a.out_rstride;
  long clr = a.cl ? a.cl[r] : (a.cl_start + (long)(r % a.rows_per_seq) + 1) / a.cl_ratio;
  const int c = (int)(clr < 0 ? 0 : (clr > a.n ? a.n : clr));
  const int k = a.k;
  if (c <= k) {
    for (int i = tid; i < k; i += kTopkThreads) orow[i] = i < c ? i + a.offset : -1;
    return;
  }
  DSV41_PX(0);
  const bool cached = c <= kTopkCache;
  uint32_t* hb16 = (uint32_t*)hist;  // 16-bit bin b: half (b & 1) of word b >> 1
  if (cached) {
#pragma unroll 1
    for (int i = tid; i < 2048; i += kTopkThreads) hb16[i] = 0u;
    if (tid == 0) s_over = 0;
    __syncthreads();
  }
  // key of element i (i < c), from LDS when staged
  auto key_at = [&](int i) -> uint32_t { return cached ? keys[i] : score_key(row[i]); };

  uint32_t kmin = 0xffffffffu, kmax = 0u;
  auto stage_key = [&](float v) -> uint32_t {  // the key, counted in the histogram (staged rows) and the range
    const uint32_t key = score_key(v);
    if (cached) atomicAdd(&hb16[key >> 21], 1u << ((key >> 16) & 16));  // bin key >> 20
    kmin = min(kmin, key);
    kmax = max(kmax, key);
    return key;
  };
  auto stage = [&](int i, float v) {
    const uint32_t key = stage_key(v);
    if (cached) keys[i] = key;
  };
  if ((((uintptr_t)row) & 15) == 0) {  // 16-byte aligned row: float4 loads, 4 x B elements per thread per batch
    for (int i0 = 4 * tid; i0 < c; i0 += 4 * B * kTopkThreads) {
      float4 v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = i0 + 4 * u * kTopkThreads;
        v[u] = *(const float4*)(row + (i + 3 < c ? i : 0));
        if (i + 3 >= c) {  // tail: element-wise
          v[u].x = row[i < c ? i : 0];
          v[u].y = row[i + 1 < c ? i + 1 : 0];
          v[u].z = row[i + 2 < c ? i + 2 : 0];
          v[u].w = row[0];
        }
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = i0 + 4 * u * kTopkThreads;
        const float vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        if (i + 3 < c) {  // the 4 keys in one 16-byte LDS store (consecutive lanes, consecutive 16 bytes)
          uint32_t kq[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) kq[e] = stage_key(vv[e]);
          if (cached) *(uint4*)&keys[i] = make_uint4(kq[0], kq[1], kq[2], kq[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (i + e < c) {
              const uint32_t key = stage_key(vv[e]);
              if (cached) keys[i + e] = key;
            }
        }
      }
    }
  } else {
    for (int i0 = tid; i0 < c; i0 += B * kTopkThreads) {
      float v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = i0 + u * kTopkThreads;
        v[u] = row[i < c ? i : 0];
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = i0 + u * kTopkThreads;
        if (i < c) stage(i, v[u]);
      }
    }
  }
  DSV41_PX(1);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, m, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, m, 64));
  }
  if (lane == 0) {
    red_min[wave] = kmin;
    red_max[wave] = kmax;
  }
  __syncthreads();  // (also completes the staged keys and their histogram)
  kmin = red_min[0];
  kmax = red_max[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    kmin = min(kmin, red_min[w]);
    kmax = max(kmax, red_max[w]);
  }
  DSV41_PX(2);
  const int chunk = ((c + NW * 64 - 1) / (NW * 64)) * 64;
  const int i0 = min(c, wave * chunk), i1 = min(c, i0 + chunk);
  uint32_t thr = 0u;  // the k-th largest key; `remaining` elements equal to it are taken
  int remaining = k;
  bool fast = cached;
  if (fast) {
    // ---- threshold bin: thread t owns bins 4095 - BPT t .. 4096 - BPT (t + 1) (high to low)
    constexpr int BPT = 4096 / NT;
    int hb[BPT], local = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int b = 4095 - BPT * tid - i;
      hb[i] = (int)((hb16[b >> 1] >> ((b & 1) * 16)) & 0xffffu);
      local += hb[i];
    }
    int total;
    int greater = block_excl_scan<NT>(local, scan_tmp, &total);
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      if (greater < k && k <= greater + hb[i]) {
        s_bin = 4095 - BPT * tid - i;
        s_rem = k - greater;
      }
      greater += hb[i];
    }
    __syncthreads();
    DSV41_PX(3);
    const uint32_t bn = (uint32_t)s_bin;
    const int need = s_rem;  // candidates of bin bn to take
    // ---- per wave: entries above bn, and the list of bin-bn candidates
    uint32_t* wl = hb16 + wave * kList;
    // masks of 64 positions at a time: two compares per key (bin >= bn, bin > bn), the counts and the candidates'
    // list slots from the ballots (scalar popcounts, mbcnt lane ranks)
    const uint32_t lo = bn << 20, hi_incl = lo | 0xfffffu;
    int gt = 0, nc = 0;
    wave_batches<B>(i0, i1, lane, [&](int i) { return keys[i]; }, [&](int b0, const uint32_t(&kk)[B], auto full) {
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const unsigned long long inm = full ? ~0ull : lanes_below(i1 - (b0 + u * 64));
        const unsigned long long gem = __ballot(kk[u] >= lo) & inm, gtm = __ballot(kk[u] > hi_incl) & inm;
        const unsigned long long cm = gem & ~gtm;
        gt += __popcll(gtm);
        if (cm) {
          const int p = nc + lane_rank(cm);
          if (lane_in(cm) && p < kList) wl[p] = kk[u];
          nc += __popcll(cm);
        }
      }
    });
    if (lane == 0) {
      w_gt[wave] = gt;
      w_nc[wave] = nc;
      if (nc > kList) s_over = 1;
    }
    __syncthreads();
    DSV41_PX(4);
    if (s_over == 0) {
      // ---- radix select of the need-th largest listed candidate on the low 20 bits (10 + 10)
      uint32_t prefix = 0u, pmask = 0u;
      int rem = need;
#pragma unroll 1
      for (int pass = 0; pass < 2; ++pass) {
        const int shift = pass == 0 ? 10 : 0;
        for (int i = tid; i < 512; i += kTopkThreads) h2[i] = 0u;
        __syncthreads();
        // every wave's list as one index space: slot j of list j / kList (all loads independent)
        static_assert(NW * kList % kTopkThreads == 0, "list slots per thread");
#pragma unroll
        for (int q = 0; q < NW * kList / kTopkThreads; ++q) {
          const int j = q * kTopkThreads + tid, w = j / kList;
          if (j - w * kList < min(w_nc[w], kList)) {
            const uint32_t d = hb16[j] & 0xfffffu;
            if ((d & pmask) == prefix) {
              const uint32_t dg = (d >> shift) & 1023u;
              atomicAdd(&h2[dg >> 1], 1u << ((dg & 1u) * 16));
            }
          }
        }
        __syncthreads();
        constexpr int BP2 = 1024 / NT;  // thread t owns digits 1023 - BP2 t .. (high to low)
        int hd[BP2], loc2 = 0;
#pragma unroll
        for (int i = 0; i < BP2; ++i) {
          const int dg = 1023 - BP2 * tid - i;
          hd[i] = (int)((h2[dg >> 1] >> ((dg & 1) * 16)) & 0xffffu);
          loc2 += hd[i];
        }
        int tot2;
        int gr = block_excl_scan<NT>(loc2, scan_tmp, &tot2);
#pragma unroll
        for (int i = 0; i < BP2; ++i) {
          if (gr < rem && rem <= gr + hd[i]) {
            s_digit = 1023 - BP2 * tid - i;
            s_rem = rem - gr;
          }
          gr += hd[i];
        }
        __syncthreads();
        prefix |= (uint32_t)s_digit << shift;
        pmask |= 1023u << shift;
        rem = s_rem;
        __syncthreads();
      }
      DSV41_PX(5);
      thr = (bn << 20) | prefix;
      remaining = rem;
      // per wave: its listed candidates above / equal to the threshold
      int g2 = 0, e2 = 0;
#pragma unroll 1
      for (int j = lane; j < nc; j += 64) {
        const uint32_t key = wl[j];
        g2 += key > thr;
        e2 += key == thr;
      }
      g2 = __reduce_add_sync(~0ull, g2);
      e2 = __reduce_add_sync(~0ull, e2);
      if (lane == 0) {
        w_gt[wave] += g2;
        w_eq[wave] = e2;
      }
    } else {
      fast = false;  // (uniform: s_over is read after the barrier)
    }
  }
  if (!fast) {
    const uint32_t range = kmax - kmin;
    int shift = range ? 32 - __clz((int)range) : 0;
    uint32_t prefix = 0u, pmask = 0u;
    remaining = k;
    while (shift > 0) {
      const int bits = shift < 11 ? shift : 11;
      shift -= bits;
      const int nb = 1 << bits;
      for (int i = tid; i < 2048; i += kTopkThreads) hist[i] = 0;
      __syncthreads();
      for (int j0 = tid; j0 < c; j0 += B * kTopkThreads) {
        uint32_t d[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int i = j0 + u * kTopkThreads;
          d[u] = key_at(i < c ? i : 0) - kmin;
        }
#pragma unroll
        for (int u = 0; u < B; ++u)
          if (j0 + u * kTopkThreads < c && (d[u] & pmask) == prefix) atomicAdd(&hist[(d[u] >> shift) & (nb - 1)], 1);
      }
      __syncthreads();
      // descending suffix counts: thread t owns BPT consecutive bins starting at BPT*u, u = NT-1-t (high -> low)
      constexpr int BPT = 2048 / NT;
      const int u = kTopkThreads - 1 - tid;
      int hb[BPT];
      int local = 0;
#pragma unroll
      for (int i = 0; i < BPT; ++i) {
        hb[i] = BPT * u + i < nb ? hist[BPT * u + i] : 0;
        local += hb[i];
      }
      int total;
      int greater = block_excl_scan<NT>(local, scan_tmp, &total);  // elements in bins above this thread's range
#pragma unroll
      for (int i = BPT - 1; i >= 0; --i) {
        if (BPT * u + i < nb && greater < remaining && remaining <= greater + hb[i]) {
          s_digit = BPT * u + i;
          s_rem = remaining - greater;
        }
        greater += hb[i];
      }
      __syncthreads();
      prefix |= (uint32_t)s_digit << shift;
      pmask |= (uint32_t)(nb - 1) << shift;
      remaining = s_rem;
      __syncthreads();
    }
    thr = kmin + prefix;
    int gt = 0, eq = 0;
    for (int b0 = i0; b0 < i1; b0 += 64 * B) {
      uint32_t kk[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = b0 + u * 64 + lane;
        kk[u] = key_at(i < i1 ? i : i0);
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const bool in = b0 + u * 64 + lane < i1;
        gt += in && kk[u] > thr;
        eq += in && kk[u] == thr;
      }
    }
    gt = __reduce_add_sync(~0ull, gt);
    eq = __reduce_add_sync(~0ull, eq);
    if (lane == 0) {
      w_gt[wave] = gt;
      w_eq[wave] = eq;
    }
  }
  __syncthreads();
  if (tid == 0) {
    int eq_before = 0, sel_before = 0;
    for (int w = 0; w < NW; ++w) {
      int take = remaining - eq_before;
      take = take < 0 ? 0 : (take > w_eq[w] ? w_eq[w] : take);
      w_take[w] = take;
      w_base[w] = sel_before;
      eq_before += w_eq[w];
      sel_before += w_gt[w] + take;
    }
  }
  __syncthreads();
  DSV41_PX(6);
  // ---- ordered emission over the wave's chunk, 64 positions per step: the selected lanes as a mask (keys above
  // the threshold, and the wave's first `take` keys equal to it), their output slots from mbcnt lane ranks
  const int take = w_take[wave];
  int base = w_base[wave], eq_seen = 0;
  auto emit = [&](auto key_of) {
    wave_batches<B>(i0, i1, lane, key_of, [&](int b0, const uint32_t(&kk)[B], auto full) {
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = b0 + u * 64 + lane;
        const unsigned long long inm = full ? ~0ull : lanes_below(i1 - (b0 + u * 64));
        unsigned long long selm = __ballot(kk[u] > thr) & inm;
        const unsigned long long eqm = __ballot(kk[u] == thr) & inm;
        if (eqm) {  // (uniform) equal keys: taken in position order until `take` are
          const int avail = take - eq_seen;
          if (avail >= (int)__popcll(eqm))  // (signed: avail < 0 once the wave's share is taken)
            selm |= eqm;
          else if (avail > 0)
            selm |= __ballot(lane_in(eqm) && lane_rank(eqm) < avail);
          eq_seen += __popcll(eqm);
        }
        const int p = base + lane_rank(selm);
        if (lane_in(selm) && p < k) orow[(uint32_t)p] = i + a.offset;
        base += __popcll(selm);
      }
    });
  };
  if (cached)
    emit([&](int i) { return keys[i]; });
  else
    emit([&](int i) { return score_key(row[i]); });
  DSV41_PX(7);
}

// Compute units of the current device (queried once per device; 256 when the query fails).
int score_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}

int launch_score(ScoreArgs& a, hipStream_t st) {
  if (a.R <= 0 || a.n_pos <= 0) return 0;
  if (a.HI <= 0 || a.HI > 64) return (int)hipErrorInvalidValue;
  if (a.kfmt == 1 && !a.seq && !a.hist && !a.write_masked && !a.cl && a.R >= 64 && a.rows_per_slot % kPQ == 0) {
    // prefill: causal rows of one sequence per block of kPQ rows; positions >= the row's limit are not written
    const int qblocks = (a.R + kPQ - 1) / kPQ;
    int split = (512 + qblocks - 1) / qblocks;
    split = split < 1 ? 1 : (split > 16 ? 16 : split);
    switch ((a.HI + 15) / 16) {
      case 1: index_score_prefill_kernel<1><<<dim3(split, qblocks), kPThreads, 0, st>>>(a, split); break;
      case 2: index_score_prefill_kernel<2><<<dim3(split, qblocks), kPThreads, 0, st>>>(a, split); break;
      case 3: index_score_prefill_kernel<3><<<dim3(split, qblocks), kPThreads, 0, st>>>(a, split); break;
      default: index_score_prefill_kernel<4><<<dim3(split, qblocks), kPThreads, 0, st>>>(a, split); break;
    }
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  // A few long rows with a histogram: 16-wave workgroups (1024 keys each), so a quarter as many workgroups add
  // their partial histograms to the row's with device-scope atomics (one 262144-key row: 22.7 -> 15.6 us; without
  // the histogram 11.5 us).  Not for many rows: 48 draft rows of 65536 keys took 117 instead of 110 us.
  const int nx16 = (a.n_pos + 16 * kKeysPerWave - 1) / (16 * kKeysPerWave);
  if (a.hist && a.R <= 4 && (long)nx16 * a.R >= 256) {
    const dim3 grid16((nx16 + kXcds - 1) / kXcds * kXcds * a.R);
    if (a.kfmt == 1) index_score_kernel<1, true, 16><<<grid16, 1024, 0, st>>>(a, nx16);
    else index_score_kernel<0, true, 16><<<grid16, 1024, 0, st>>>(a, nx16);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  const int nx = (a.n_pos + kKeysPerWG - 1) / kKeysPerWG;
  if (a.hist && a.kfmt == 1 && !a.write_masked && a.R > 4 && a.R <= kLoopMaxRows) {
    // many rows (draft rows of a few sequences): (group, chunk) items over one workgroup per CU
    index_score_group_kernel<<<dim3((unsigned)((score_cus() + kXcds - 1) / kXcds * kXcds)), kGThreads, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
    return 0;
  }
  const dim3 grid((nx + kXcds - 1) / kXcds * kXcds * a.R);
  if (a.hist) {
    if (a.kfmt == 1) index_score_kernel<1, true><<<grid, 256, 0, st>>>(a, nx);
    else index_score_kernel<0, true><<<grid, 256, 0, st>>>(a, nx);
  } else {
    if (a.kfmt == 1) index_score_kernel<1, false><<<grid, 256, 0, st>>>(a, nx);
    else index_score_kernel<0, false><<<grid, 256, 0, st>>>(a, nx);
  }
  DSV41_CHECK_LAUNCH();
  return 0;
}


// ------------------------------------------------------------------------------------------------ candidate blocks
// select_candidate_blocks (dsv41/model.py:256-265): per row the maxima of the masked scores over blocks of bs
// positions (positions >= cl(r) count as -inf), the block of position cl(r) - 1 forced to +inf, the topk_blocks
// largest blocks (ties lowest block first) kept when their value is finite, expanded to a per-position mask.
struct CandArgs {
  const float* score;
  long ld;
  int R, n, width, bs, nb, kb;
  const long* cl;
  long cl_start;
  int cl_ratio, rows_per_seq;
  float* bmax;  // [R, nbp]
  long nbp;
  int* sel;  // [R, kb] selected blocks, ascending
  uint8_t* mask;
  long mask_rstride;
};

DSV41_DEV long cand_row_cl(const CandArgs& a, int r) {
  if (a.cl) return a.cl[r];
  return (a.cl_start + (long)(r % a.rows_per_seq) + 1) / a.cl_ratio;
}

__global__ void __launch_bounds__(256) cand_blockmax_kernel(const CandArgs a) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)a.R * a.nb) return;
  const int r = (int)(i / a.nb), b = (int)(i - (long)r * a.nb);
  long c = cand_row_cl(a, r);
  c = c < 0 ? 0 : (c > a.n ? a.n : c);
  float m = -__builtin_inff();
  const float* row = a.score + (long)r * a.ld;
  const long t1 = min((long)(b + 1) * a.bs, c);
  for (long t = (long)b * a.bs; t < t1; ++t) m = fmaxf(m, row[t]);
  if (c > 0 && b == (int)((c - 1) / a.bs)) m = __builtin_inff();
  a.bmax[(long)r * a.nbp + b] = m;
}

__global__ void __launch_bounds__(256) cand_expand_kernel(const CandArgs a) {
  const int r = blockIdx.y;
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= a.width) return;
  const int b = (int)(t / a.bs);
  const int* srow = a.sel + (long)r * a.kb;
  int lo = 0, hi = a.kb;  // srow is ascending (with -1 padding only when a row has fewer blocks than kb)
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const int v = srow[mid];
    if (v >= 0 && v < b) lo = mid + 1; else hi = mid;
  }
  bool keep = false;
  if (lo < a.kb && srow[lo] == b && b < a.nb) keep = a.bmax[(long)r * a.nbp + b] > -__builtin_inff();
  a.mask[(long)r * a.mask_rstride + t] = keep ? 1 : 0;
}

long cand_nbp(int n, int bs) { return ((n + bs - 1) / bs + 3) / 4 * 4; }

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_px_idx(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_px), sizeof(g_dsv41_px)); }
int dsv41_read_ts_idx(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ts), sizeof(g_dsv41_ts)); }
int dsv41_read_ph_idx(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ph), sizeof(g_dsv41_ph)); }
int dsv41_read_wg_idx(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_wg), sizeof(g_dsv41_wg)); }
#endif


int dsv41_index_score(const void* q, long q_rstride, const float* w, long w_rstride, int R, int HI, int D, int kfmt,
                      const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                      int rows_per_slot, const long* cl, long cl_start, int cl_ratio, int n_pos, int write_masked,
                      float* out, long out_rstride, int* hist, const void* cand, long cand_rstride, void* stream) {
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
  a.hist = hist;
  a.cand = (const uint8_t*)cand;
  a.cand_rstride = cand_rstride;
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
  if (R >= 512 && n <= 17408) topk_kernel<512, 17408><<<R, 512, 0, (hipStream_t)stream>>>(a);  // many short rows
  else topk_kernel<1024, 32768><<<R, 1024, 0, (hipStream_t)stream>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

long dsv41_candidate_blocks_workspace_bytes(int R, int n, int topk_blocks, int block_size) {
  if (R <= 0 || n <= 0 || block_size <= 0 || topk_blocks <= 0) return 0;
  const int nb = (n + block_size - 1) / block_size, kb = topk_blocks < nb ? topk_blocks : nb;
  return (long)R * cand_nbp(n, block_size) * 4 + (long)R * kb * 4;
}

int dsv41_candidate_blocks(const float* score, long ld, int R, int n, int width, const long* cl, long cl_start,
                           int cl_ratio, int rows_per_seq, int topk_blocks, int block_size, void* mask,
                           long mask_rstride, void* ws, long ws_bytes, void* stream) {
  if (R <= 0 || width <= 0) return 0;
  if (n <= 0 || n > width || block_size <= 0 || topk_blocks <= 0 || (!cl && cl_ratio <= 0) || !mask)
    return (int)hipErrorInvalidValue;
  if (!ws || ws_bytes < dsv41_candidate_blocks_workspace_bytes(R, n, topk_blocks, block_size))
    return (int)hipErrorInvalidValue;
  CandArgs a{};
  a.score = score;
  a.ld = ld;
  a.R = R;
  a.n = n;
  a.width = width;
  a.bs = block_size;
  a.nb = (n + block_size - 1) / block_size;
  a.kb = topk_blocks < a.nb ? topk_blocks : a.nb;
  a.cl = cl;
  a.cl_start = cl_start;
  a.cl_ratio = cl_ratio;
  a.rows_per_seq = rows_per_seq > 0 ? rows_per_seq : 1;
  a.nbp = cand_nbp(n, block_size);
  a.bmax = (float*)ws;
  a.sel = (int*)((char*)ws + (long)R * a.nbp * 4);
  a.mask = (uint8_t*)mask;
  a.mask_rstride = mask_rstride;
  hipStream_t st = (hipStream_t)stream;
  cand_blockmax_kernel<<<(int)(((long)R * a.nb + 255) / 256), 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  // the kb largest block maxima of every row (all nb blocks valid: cl = (nb - 1 + 0 + 1) / 1)
  const int rc = dsv41_topk_indices(a.bmax, a.nbp, R, a.nb, a.kb, nullptr, a.nb - 1, 1, 1, 0, a.sel, a.kb, stream);
  if (rc) return rc;
  cand_expand_kernel<<<dim3((width + 255) / 256, R), 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
