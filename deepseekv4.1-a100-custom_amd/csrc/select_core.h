// Exact threshold among the candidates of a top-k threshold bin (shared by the selection kernels).
#pragma once
#include "common.h"

namespace {

constexpr int kRankDirect = 64;  // up to this many candidates: direct ranks; more: radix passes

struct RankScratch {
  int rh[1024];
  int tmp[8];
  int digit, rem, eq;
  unsigned long long T;
};

// NT threads (256 or 512).  The m candidates are values key << 32 | ~position whose keys share the threshold bin
// (top 12 bits lo); the need largest values are taken (higher key, then lower position).  Returns T such that exactly the
// candidates >= T are taken (0 when all are).  cand_at(i) reads candidate i; when staged, lc holds the m candidates
// followed by a zero pad (pairwise reads).
//   m <= kRankDirect: direct ranks (rank = candidates larger than it), T = the candidate of rank need - 1
//   otherwise: two 10-bit LDS histogram passes over key bits 19..10 and 9..0 give the exact key Tk and the number
//   rem of candidates with key Tk that are taken; T = (Tk << 32) when all of them are, else the one whose position
//   ranks rem - 1 among them.
template <int NT = 256, class At>
DSV41_DEV unsigned long long threshold_candidate(At cand_at, const unsigned long long* lc, bool staged, int m,
                                                 int need, uint32_t lo, RankScratch& sm) {
  constexpr int BP = 1024 / NT;  // histogram bins per thread
  const int t = threadIdx.x;
  if (t == 0) sm.T = 0ull;  // every candidate is taken
  __syncthreads();
  if (m != need) {
    if (staged && m <= kRankDirect) {  // direct ranks, two candidates per LDS read
      const uint4* l4 = (const uint4*)lc;
      const int m2 = (m + 1) / 2;
#pragma unroll 1
      for (int i = t; i < m; i += NT) {
        const unsigned long long me = lc[i];
        int rk = 0;
#pragma unroll 8
        for (int q = 0; q < m2; ++q) {
          const uint4 w = l4[q];
          rk += ((unsigned long long)w.y << 32 | w.x) > me;
          rk += ((unsigned long long)w.w << 32 | w.z) > me;
        }
        if (rk == need - 1) sm.T = me;
      }
    } else {
      // two 10-bit histogram passes over key bits 19..10 and 9..0 give the exact key Tk and the number rem of
      // candidates with key Tk that are taken; among those, the one whose position ranks rem - 1 is T
      uint32_t prefix = lo, mask = 0xfff00000u;
      int rem = need;
#pragma unroll 1
      for (int pass = 0; pass < 2; ++pass) {
        const int shift = pass == 0 ? 10 : 0;
#pragma unroll
        for (int i = 0; i < BP; ++i) sm.rh[BP * t + i] = 0;
        __syncthreads();
#pragma unroll 1
        for (int i = t; i < m; i += NT) {
          const uint32_t kk = (uint32_t)(cand_at(i) >> 32);
          if ((kk & mask) == prefix) atomicAdd(&sm.rh[(kk >> shift) & 1023], 1);
        }
        __syncthreads();
        int h[BP];  // digits 1023 - BP*t down to 1024 - BP*(t+1)
        int hs = 0;
#pragma unroll
        for (int i = 0; i < BP; ++i) {
          h[i] = sm.rh[1023 - BP * t - i];
          hs += h[i];
        }
        int tot;
        int greater = block_scan_dpp<NT>(hs, sm.tmp, &tot);
#pragma unroll
        for (int i = 0; i < BP; ++i) {
          if (greater < rem && rem <= greater + h[i]) {
            sm.digit = 1023 - BP * t - i;
            sm.rem = rem - greater;
            sm.eq = h[i];
          }
          greater += h[i];
        }
        __syncthreads();
        prefix |= (uint32_t)sm.digit << shift;
        mask |= 1023u << shift;
        rem = sm.rem;
      }
      if (t == 0 && sm.eq == rem) sm.T = (unsigned long long)prefix << 32;  // every candidate with key Tk is taken
#pragma unroll 1
      for (int i = t; i < m && sm.eq != rem; i += NT) {
        const unsigned long long me = cand_at(i);
        if ((uint32_t)(me >> 32) != prefix) continue;
        int rk = 0;  // candidates of the same key at lower positions (larger values)
#pragma unroll 1
        for (int q = 0; q < m; ++q) {
          const unsigned long long o = cand_at(q);
          rk += (uint32_t)(o >> 32) == prefix && o > me;
        }
        if (rk == rem - 1) sm.T = me;
      }
    }
    __syncthreads();
  }
  return sm.T;
}

}  // namespace
