// One decode layer-step in one launch: the step's cache appends, the lightning indexer (scores + exact top-k) and the
// sparse attention over the SWA ring plus the selected compressed rows -- DecodeRuntime.attention2 between the
// projections and the o-projection (dsv41/decode.py:106-174 with the indexer of :267-319; scores as
// dsv41/fused3.py:20-62, selection as dsv41/fused3.py:65-75, attention as dsv41/fused2.py:334-446).
//
// Grid: G = R * NC workgroups of 512 threads, one per CU (every workgroup of a row takes part in two row-wide
// exchanges, so all must be resident at once).  NC = chunks of 512 positions per row (a multiple of 4), S = NC / 4
// attention splits per row.  Workgroup b has two roles:
//   scoring  : chunk ch of row r (positions ch*512 .. +511)
//   attention: 16-head group hg and split sp of row r
// with x = b % 8 (its XCD), j = b / 8, hg = j % 4, unit u = x + 8 (j / 4) = r * S + sp and ch = 4 sp + hg: the four
// head groups of a (row, split) share an XCD, so the compressed rows they all gather come from one L2.
//
// Phases of a workgroup:
//   A. row data, e4m3 index-query preparation (every workgroup), its chunk's key scores (fp8 MFMA) and their
//      4096-bin histogram in LDS; the chunk holding a closing group's new index key computes, stores and scores it.
//      Independent of the indexer: the attention's Q (16 heads) is staged, and the workgroups that will attend over
//      the new ring row or the new compressed row compute those rows themselves (the ring / table writes of this
//      launch are not visible to other workgroups' loads).
//   B. publish: the chunk's candidates -- every position whose histogram bin is at or above the chunk's boundary bin
//      (the bin at which the chunk's own count from the top reaches kStLocalTop) -- in position order, then its count
//      word (launch epoch, boundary bin, count) with device-scope stores.
//   C. while the row's other chunks publish: the cache writes of the step (ring row, compressed row, spare-row index
//      key; one workgroup each) and, for splits 0 .. W/64-1, their SWA ring tile of the attention.
//   D. every workgroup of the row waits for all count words, reads all candidates, finds the threshold bin B of the
//      k largest and, when every chunk's boundary bin is at most B (all candidates at or above B are published),
//      the exact threshold among bin B's candidates; otherwise the chunks whose boundary lies above B publish all
//      their positions from B up and the row reads once more (exact in any case).  The selected positions, in
//      ascending order, form the row's index list (in LDS; also written to idx_out).
//   E. attention over the split's part of the index list (64-row tiles gathered to LDS, bf16 MFMA, online softmax),
//      bf16-normalised partials published with device-scope stores, and the cooperative merge of the S splits of
//      each (row, head group) (each split merges a slice), with the sink and the inverse rope of the output.
// Waits give up after kStSpinLimit polls and set the error word (every wave still exits).
#include "attn_core.h"
#include "rowop.h"
#include "score_core.h"
#include "select_core.h"

namespace {

constexpr int kStThreads = 512;
constexpr int kStChunk = 512;         // positions scored per workgroup
constexpr int kStTile = 64;           // key rows per attention tile
constexpr int kStLocalTop = 64;       // a chunk publishes at least its kStLocalTop largest scores (whole bins)
constexpr int kStMaxK = 2048;         // index-list capacity in LDS
constexpr int kStMaxChunks = 64;      // chunks per row (positions <= 32768)
constexpr int kStSpinLimit = 1 << 20;
constexpr int kStTagShift = 18;       // candidate value: key << 32 | epoch tag << 18 | ~position (18 bits)
constexpr int kStCandBufBytes = 2 * kStTile * 576 * 2;  // the two tile buffers (largest row width 576)
constexpr int kStRec = 24;            // u64 words per chunk record

struct StepArgs {
  ScoreArgs s;   // e4m3 keys + scales (written into by the appends), seq, cl, n_pos; out: optional scores
  // appends
  const uint16_t* kv_raw;  // [R, Dw]
  const uint16_t* kv_norm;
  uint16_t* ring;
  long ring_sstride;
  int W, Dw;
  const uint16_t* latent;  // [R, Dw] or null
  uint16_t* ckv;
  long ckv_sstride;
  int cap;
  const uint16_t* k_raw;   // [R, 128]
  const uint16_t* k_norm;
  uint16_t* kbf;
  long kbf_sstride;
  uint8_t* k8;
  long k8_sstride;
  float* ks;
  long ks_sstride;
  int kcap;
  const long* pos;
  int ratio, rd;
  const float* cos_t;
  const float* sin_t;
  float eps;
  const uint16_t* q_idx;   // [R, HI, 128] bf16, w_idx [R, HI] bf16
  const uint16_t* w_idx;
  // selection
  int k, offset;
  int* idx_out;  // [R, k] or null
  long idx_rstride;
  int nc, S;
  unsigned long long* rec;   // [R, nc, 2, kStRec]: the records (count word + bin-count table) of round 0 and 1
  unsigned long long* cand;  // [R, nc, 2, kStChunk]: the candidates of round 0 and round 1
  int* err;
  // attention (kv1 = ring, kv2 = compressed table, mode 1 validity; nsplit = S; coop counters, partials)
  AttnArgs at;
};

DSV41_DEV unsigned long long st_cand_value(uint32_t key, int p, uint32_t tag) {
  return (unsigned long long)key << 32 | tag << kStTagShift | (~(uint32_t)p & ((1u << kStTagShift) - 1));
}
DSV41_DEV int st_cand_pos(unsigned long long v) { return (int)(~(uint32_t)v & ((1u << kStTagShift) - 1)); }

// Count word of a chunk: epoch (24 bits) << 40 | top bin << 22 | boundary bin << 10 | candidates (<= 512).
constexpr uint32_t kStEpochMask = (1u << 24) - 1;
DSV41_DEV unsigned long long st_count_word(uint32_t epoch, int tq, int bq, int n) {
  return (unsigned long long)(epoch & kStEpochMask) << 40 | (unsigned long long)tq << 22 |
         (unsigned long long)bq << 10 | (unsigned)n;
}
DSV41_DEV uint32_t st_word_epoch(unsigned long long w) { return (uint32_t)(w >> 40) & kStEpochMask; }

// row_load + row_compute, the computed row left in g.
template <int NT, bool LB = false>
DSV41_DEV void row_op_keep(const RowOp& o, RowRegs<NT>& g, float* red) {
  row_load<NT>(o, g);
  row_compute<NT, LB>(o, g, red);
}

template <int DQK, int DV>
__global__ void __launch_bounds__(kStThreads, 1) decode_step_kernel(const StepArgs g) {
  constexpr int KS = DQK / 32;  // QK k-steps
  constexpr int CTH = DV / 32;  // 16-column output tiles per wave (half of DV)
  constexpr int U = DQK / 8;    // 16-byte chunks per row; chunk c of tile row j at j*U + (c ^ (j & 7))
  constexpr int TILE_ELEMS = kStTile * DQK;
  constexpr int kLoadsPerTile = kStTile * U / kStThreads;
  static_assert(U % 8 == 0 && kLoadsPerTile < 16 && kLoadsPerTile * kStThreads == kStTile * U, "tile geometry");
  constexpr float kRescale = 8.0f;
  // ---- shared memory: the two tile buffers, aliased by the scoring and selection phases
  __shared__ __align__(16) uint8_t smem[kStCandBufBytes];
  __shared__ int selidx[kStMaxK];
  __shared__ const uint16_t* rptr[3][kStTile];
  __shared__ float wm[4][16], wl[4][16], wf[4][16], hM[16], hL[16], redf[8], ksnew;
  __shared__ int tmp[8], wcnt[8][2];
  __shared__ int cnt_q[kStMaxChunks], bq_q[kStMaxChunks], tq_q[kStMaxChunks], rg_q[kStMaxChunks];
  __shared__ int lump_q[kStMaxChunks], ab_q[kStMaxChunks], nb_q[kStMaxChunks], sb_q[kStMaxChunks];
  __shared__ int pu[kStMaxChunks + 1];
  __shared__ uint16_t stab[64];
  __shared__ int s_bin, s_above, s_tq, s_bq, s_npub, s_lump, s_nu;
  __shared__ unsigned long long s_T;
  __shared__ int s_sb, s_need2, s_nsb;
  uint16_t* const B0 = (uint16_t*)smem;                        // tile buffer 0
  uint16_t* const B1 = (uint16_t*)(smem + kStCandBufBytes / 2);  // tile buffer 1
  int* const lhist = (int*)smem;                                  // A: 4096 bins (B0 bytes 0..16K); D: reused
  float* const sc = (float*)(smem + 16384);                       // A..D: the chunk's 512 scores (B0 16K..18K)
  uint8_t* const qs = smem + 18432;                               // A: prepared queries 64 x 128 (B0 18K..26K)
  float* const wfl = (float*)(smem + 26624);                      // A: folded head weights (B0)
  uint8_t* const knew = smem + 26880;                             // A: the new index key, e4m3 (B0)
  uint16_t* const tblq = (uint16_t*)(smem + 18432);               // D: the chunks' tables, u16 [128][64] (B0)
  unsigned long long* const lcb = (unsigned long long*)(smem + 34816);  // D: bin-B candidates (B0)
  constexpr int kLcbCap = 2048;
  RankScratch& rs = *(RankScratch*)(smem + 34816 + (kLcbCap + 2) * 8);  // D: threshold scratch (B0)
  static_assert(34816 + (kLcbCap + 2) * 8 + sizeof(RankScratch) <= kStCandBufBytes / 2, "B0 layout");

  const ScoreArgs& a = g.s;
  AttnArgs at = g.at;
  const int NC = g.nc, S = g.S, R = a.R;
  const int b = blockIdx.x, xcd = b % kXcds, jj = b / kXcds;
  const int hg = jj & 3, unit = xcd + kXcds * (jj >> 2);
  const int r = unit / S, sp = unit % S, ch = sp * 4 + hg;
  if (r >= R) return;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int rw = wave & 3, half = wave >> 2;
  const int h0 = hg * 16;

  // ================================================================ A. row data, queries, Q staging, scores
  DSV41_PH(0);
  const long slot = a.seq[r];
  // the chunk's key loads first: they depend on the slot only (positions past the valid count are masked later)
  constexpr int NT = 64 / 16;  // 16-key column tiles per wave (64 keys per wave, 512 per workgroup)
  uint4 k0[NT], k1[NT];
  float ksc[NT];
  const int pw = ch * kStChunk + wave * 64;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int p = pw + nt * 16 + l16;
    const bool pv = p < a.n_pos;
    const uint8_t* krow = (const uint8_t*)a.keys + slot * a.k_sstride + (long)p * 128 + g4 * 32;
    k0[nt] = pv ? *(const uint4*)krow : make_uint4(0, 0, 0, 0);
    k1[nt] = pv ? *(const uint4*)(krow + 16) : make_uint4(0, 0, 0, 0);
    ksc[nt] = pv ? a.kscale[slot * a.ks_sstride + p] : 0.0f;
  }
  const long clr = row_cl(a, r);
  const long ppos = g.pos[r];
  const long pmax = at.pmax[r];
  const long plim = at.plim ? at.plim[r] : ppos;
  unsigned long long* const rrec = g.rec + (long)r * NC * 2 * kStRec;
  const __amdgpu_buffer_rsrc_t rec_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)g.rec, 0, 0x7fffffff, 0x00020000);
  unsigned long long* const crow = g.cand + (long)r * NC * 2 * kStChunk;
  const uint32_t epoch =
      st_word_epoch(__hip_atomic_load(rrec + 2 * ch * kStRec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + 1;
  const uint32_t tag = epoch & ((1u << (32 - kStTagShift)) - 1);
  const int c = (int)(clr < 0 ? 0 : (clr > a.n_pos ? a.n_pos : clr)), k = g.k;
  const int kk = c < k ? c : k;  // entries of the index list
  if (clr > a.n_pos && ch == 0 && t == 0) __hip_atomic_store(g.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool closes = ((ppos + 1) % g.ratio) == 0;
  const long knew_row = closes ? (ppos + 1) / g.ratio - 1 : -1;
  // attention: split sp < W/64 takes ring tile sp, then every split the selected rows of its unit's four chunks
  const int nring = g.W / kStTile;
  const long ring_new = ppos < 0 ? 0 : ppos % g.W;  // ring slot of this step's row
  const bool need_ring = sp < nring && ring_new / kStTile == sp;
  const bool ring_writer = need_ring && hg == 0;

  auto make_op = [&](int which, bool to_global) {
    RowOp o{};
    o.cos_t = g.cos_t;
    o.sin_t = g.sin_t;
    o.rd = g.rd;
    o.eps = g.eps;
    if (which == 0) {  // SWA ring row: rmsnorm -> rope -> fp8 grid (dsv41/fused2.py:276-330)
      o.x = g.kv_raw + (long)r * g.Dw;
      o.D = g.Dw;
      o.norm_w = g.kv_norm;
      o.pos = ppos < 0 ? 0 : ppos;
      o.qmode = 0;
      o.group = 32;
      o.out = to_global ? g.ring + slot * g.ring_sstride + ring_new * (long)g.Dw : nullptr;
    } else if (which == 1) {  // compressed row: rope -> fp4 grid, e4m3 scale per 16 (dsv41/decode.py:157-162)
      const long row = closes ? knew_row : g.cap - 1;
      o.x = g.latent + (long)r * g.Dw;
      o.D = g.Dw;
      o.pos = ppos + 1 - g.ratio;
      o.qmode = 2;
      o.group = 16;
      o.out = to_global ? g.ckv + slot * g.ckv_sstride + row * (long)g.Dw : nullptr;
    } else {  // index key: rmsnorm -> rope -> fp4 grid per 32 (dsv41/decode.py:270-282), e4m3 copy + scale
      const long row = closes ? knew_row : g.kcap - 1;
      o.x = g.k_raw + (long)r * 128;
      o.D = 128;
      o.norm_w = g.k_norm;
      o.pos = ppos + 1 - g.ratio;
      o.qmode = 1;
      o.group = 32;
      o.out = g.kbf ? g.kbf + slot * g.kbf_sstride + row * 128L : nullptr;
      o.k8 = g.k8 + slot * g.k8_sstride + row * 128L;
      o.ks = g.ks + slot * g.ks_sstride + row;
      o.k8_lds = knew;
      o.ks_lds = &ksnew;
    }
    return o;
  };

  // Q of the head group, staged through B1 (direct-to-LDS loads), read into VGPRs after the scores
  {
    constexpr int QCH = 16 * DQK / 8, PR = DQK / 8;
#pragma unroll
    for (int u = 0; u < (QCH + kStThreads - 1) / kStThreads; ++u) {
      if (u * kStThreads + wave * 64 < QCH) {
        const int cid = u * kStThreads + wave * 64 + lane, hh = cid / PR, part = cid - hh * PR;
        lds_dma16(at.q + (long)r * at.q_rstride + (long)(h0 + hh) * DQK + part * 8, B1 + (u * kStThreads + wave * 64) * 8);
      }
    }
  }
  // the new index key (chunk holding it), the ring row and the compressed row this workgroup attends over
  const bool key_here = closes && ch == (int)(knew_row / kStChunk);
  RowRegs<kStThreads> kreg, rreg, creg;
  if (key_here) row_load<kStThreads>(make_op(2, true), kreg);
  Qprep512 qp;
  qprep512_load(g.q_idx + (long)r * a.HI * 128, g.w_idx + (long)r * a.HI, a.HI, qp);
#pragma unroll 1
  for (int i = t; i < kHistBins; i += kStThreads) lhist[i] = 0;
  DSV41_PX(16);
  if (key_here) row_compute<kStThreads, true>(make_op(2, true), kreg, redf);  // (LDS barriers: keys stay in flight)
  qprep512_store(qp, a.HI, qs, wfl);
  lds_barrier();
  DSV41_PX(17);
  const int nht = (a.HI + 15) / 16;
  i32x8_t qa8[kHT];
  uint4 qa16[kHT][4];
  float wr[kHT][4];
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    const int h = ht * 16 + l16;
    const int hc = ht < nht && h < a.HI ? h : 0;
    const uint4 u0 = *(const uint4*)(qs + hc * 128 + g4 * 32), u1 = *(const uint4*)(qs + hc * 128 + g4 * 32 + 16);
    qa8[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
    const float wv = ht < nht && h < a.HI ? wfl[h] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wv, 4 * g4 + i, 64);
  }
  if (key_here && knew_row >= pw && knew_row < pw + 64) {  // score the new key from the values computed here
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (pw + nt * 16 + l16 == knew_row) {
        k0[nt] = *(const uint4*)(knew + g4 * 32);
        k1[nt] = *(const uint4*)(knew + g4 * 32 + 16);
        ksc[nt] = ksnew;
      }
    }
  }
  const bool sel = c > k;  // otherwise every valid position is selected
  float* orow = a.out ? a.out + (long)r * a.out_rstride : nullptr;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int p = pw + nt * 16 + l16;
    const float sum = score_tile<1>(qa8, qa16, wr, nht, k0[nt], k1[nt], nullptr);
    if (g4 == 0) {
      const float v = p < c ? sum * ksc[nt] : 0.0f;
      sc[p - ch * kStChunk] = v;
      if (p < c && sel) atomicAdd(&lhist[score_key(v) >> 20], 1);
      if (orow && p < a.n_pos) orow[p] = p < c ? v : -__builtin_inff();
    }
  }
  DSV41_PX(18);
  __builtin_amdgcn_s_waitcnt(0);  // (Q staged)
  __syncthreads();
  DSV41_PH(1);
  // Q fragments of the lane's head (l16) into VGPRs; B1 is free afterwards
  uint4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const uint4*)(B1 + l16 * DQK + ks * 32 + g4 * 8);

  // ================================================================ B. publish the chunk's candidates
  // Per chunk and round, a record of 24 u64 words: word 0 the count word (epoch << 40 | top bin << 22 | boundary bin
  // << 10 | candidates), words 1..22 a table of bin counts, three u16 per word with the epoch's low 16 bits on top
  // (entry e < 63: candidates in bin top - e; entry 63: candidates below bin top - 62); then the candidates grouped
  // by bin, highest bin first (the order within a bin is arbitrary).  Every word read from another workgroup carries
  // this launch's epoch, so a reader polls the whole record in one round trip.
  const int p_mine = ch * kStChunk + t;  // one position per thread
  const uint32_t key_mine = score_key(sc[t]);
  const int bin_mine = (int)(key_mine >> 20);
  const bool valid_mine = p_mine < c;
  const unsigned long long etag = (unsigned long long)(epoch & 0xffff) << 48;
  auto publish = [&](int round, int bq_given) {  // (lhist: the chunk's bin counts; left as cursors)
    constexpr int BP = kHistBins / kStThreads;
    int h[BP], local = 0, total;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      h[i] = lhist[kHistBins - 1 - BP * t - i];
      local += h[i];
    }
    const int above = block_scan_dpp<kStThreads>(local, tmp, &total);
    const int L = round == 0 ? kStLocalTop : 0;
    if (t == 0) {
      s_bq = round == 0 ? 0 : bq_given;
      s_npub = total;  // (round 0 with fewer than kStLocalTop valid positions: all of them)
      s_lump = 0;
    }
    if (t < 64) stab[t] = 0;
    __syncthreads();
    int cum = above;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int bin = kHistBins - 1 - BP * t - i;
      if (h[i] > 0 && cum == 0) s_tq = bin;
      if (round == 0 && cum < L && cum + h[i] >= L) {
        s_bq = bin;
        s_npub = cum + h[i];
      }
      if (round == 1 && bin == bq_given) s_npub = cum + h[i];
      lhist[bin] = cum;  // cursor: candidates in higher bins
      cum += h[i];
    }
    __syncthreads();
    const int tq = s_tq, bq = s_bq;
    int lump = 0;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int bin = kHistBins - 1 - BP * t - i, e = tq - bin;
      if (bin >= bq && h[i] > 0) {
        if (e < 63) stab[e] = (uint16_t)h[i];
        else lump += h[i];
      }
    }
    if (lump) atomicAdd(&s_lump, lump);
    if (valid_mine && bin_mine >= bq) {
      const int slot_c = atomicAdd(&lhist[bin_mine], 1);
      __hip_atomic_store(crow + (2 * ch + round) * kStChunk + slot_c, st_cand_value(key_mine, p_mine, tag),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    unsigned long long* rec = rrec + (2 * ch + round) * kStRec;
    if (t >= 1 && t < kStRec) {  // table words (the count word goes out last)
      const int e0 = 3 * (t - 1);
      auto ent = [&](int e) -> unsigned long long { return e < 63 ? stab[e] : (e == 63 ? (unsigned)s_lump : 0u); };
      const unsigned long long w = ent(e0) | ent(e0 + 1) << 16 | ent(e0 + 2) << 32 | etag;
      __hip_atomic_store(rec + t, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the candidates and the table have landed before the count word goes out
    __syncthreads();
    if (t == 0)
      __hip_atomic_store(rec, st_count_word(epoch, tq, bq, s_npub), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (sel) {
    publish(0, 0);
  } else if (t == 0) {
    __hip_atomic_store(rrec + 2 * ch * kStRec, st_count_word(epoch, 0, 0, 0), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  DSV41_PH(2);

  // ================================================================ C. cache writes; the ring tile
  DSV41_PX(0);
  if (need_ring) row_op_keep<kStThreads>(make_op(0, ring_writer), rreg, redf);
  if (sp == 0 && hg == 1 && g.latent && g.ckv) row_op<kStThreads>(make_op(1, true), redf);
  if (sp == 0 && hg == 2 && !closes) row_op<kStThreads>(make_op(2, true), redf);
  const float sl2 = at.scale * kLog2e;
  float m_ref = -1e30f, l_run = 0.0f;
  f32x4_t o[CTH];
#pragma unroll
  for (int cc = 0; cc < CTH; ++cc) o[cc] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* const base_ring = at.kv1 + slot * at.kv1_sstride;
  const uint16_t* const base_c = at.kv2 + slot * at.kv2_sstride;

  auto issue = [&](uint16_t* buf, const uint16_t* const* rp) {
    const uint16_t* src[kLoadsPerTile];
#pragma unroll
    for (int q = 0; q < kLoadsPerTile; ++q) {
      const int qq = q * kStThreads + wave * 64 + lane;
      const int j = qq / U, cs = qq - j * U;
      const uint16_t* p = rp[j];
      src[q] = p ? p + (cs ^ (j & 7)) * 8 : g_zero_row;
    }
#pragma unroll
    for (int q = 0; q < kLoadsPerTile; ++q) lds_dma16(src[q], buf + (q * kStThreads + wave * 64) * 8);
  };
  // patch tile row j with a row computed in registers (element e = t + u * 512 of the row)
  auto patch = [&](uint16_t* buf, int j, const RowRegs<kStThreads>& rg) {
#pragma unroll
    for (int u = 0; u < RowRegs<kStThreads>::IT; ++u) {
      const int e = t + u * kStThreads;
      if (e < DQK) buf[j * DQK + (((e >> 3) ^ (j & 7)) << 3) + (e & 7)] = f2bf(rg.v[u]);
    }
  };
  auto compute = [&](const uint16_t* buf, const uint16_t* const* rp) {
    const int rb = rw * 16;
    f32x4_t s = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    {
      const int j = rb + l16;
      const uint16_t* krow = buf + j * DQK;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        s = mfma_bf16_16x16x32(*(const uint4*)(krow + (((ks * 4 + g4) ^ (j & 7)) * 8)), qf[ks], s);
    }
    float x[4], tmax = -1e30f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = rp[rb + 4 * g4 + i] ? s[i] * sl2 : -1e30f;
      tmax = fmaxf(tmax, x[i]);
    }
    tmax = row_max4(tmax);
    const bool bump = tmax > m_ref + kRescale;
    if (__ballot(bump)) {
      const float m_new = bump ? tmax : m_ref;
      const float alpha = exp2f(m_ref - m_new);
      l_run *= alpha;
      m_ref = m_new;
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g4 + i, 64);
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[ct][i] *= al[i];
    }
    float psum = 0.0f, p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = rp[rb + 4 * g4 + i] ? exp2f(x[i] - m_ref) : 0.0f;
      psum += p[i];
    }
    l_run += row_sum4(psum);
    const uint2 pa = make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
    const int vj = rb + 4 * g4 + (l16 >> 2);
    const uint16_t* vrow = buf + vj * DQK + ((l16 & 1) << 2);
    const int vsw = vj & 7;
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct) {
      const int cch = ((half * (DV / 2) + ct * 16) >> 3) + ((l16 & 3) >> 1);
      const uint2 vb = lds_read_tr16(vrow + ((cch ^ vsw) << 3));
      o[ct] = mfma_bf16_16x16x16(pa, vb, o[ct]);
    }
  };
  if (sp < nring) {  // ring slots 64 sp .. 64 sp + 63 (validity as dsv41/fused2.py:355-360); the tile goes to B1
    if (t < kStTile) {
      const int jr = sp * kStTile + t;
      int m = (int)((pmax - jr) % g.W);
      m = m < 0 ? m + g.W : m;
      const long held = pmax - m;
      rptr[2][t] = (held >= 0 && held <= plim && ppos - held < g.W) ? base_ring + (long)jr * DQK : nullptr;
    }
    __syncthreads();
    issue(B1, rptr[2]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (need_ring) {  // this step's row, from the values computed here
      patch(B1, (int)(ring_new - sp * kStTile), rreg);
      __syncthreads();
    }
    compute(B1, rptr[2]);
    __syncthreads();
  }
  DSV41_PH(3);

  // ================================================================ D. the unit's selected rows
  // (the unit's four chunks 4 sp .. 4 sp + 3; every workgroup of the unit builds the same list)
  int n_unit = 0;
  if (sel) {
    int round = 0, b0 = 0;
    unsigned long long uv[4];
#pragma unroll 1
    while (true) {
      // the chunks' records (count word + table), read together with device-coherent 16-byte loads until every
      // word carries this launch's epoch
      constexpr int RU = kStRec / 2;                               // 16-byte units per record
      constexpr int PU = (kStMaxChunks * RU + kStThreads - 1) / kStThreads;
      u32x4_t rv[PU];
      int spins = 0;
#pragma unroll 1
      while (true) {  // count words until every chunk's carries this launch's epoch (one load per chunk, spaced polls)
        bool ok = true;
        if (t < NC) {
          const int rg = round == 1 && bq_q[t] > b0;
          const unsigned long long cv =
              __hip_atomic_load(rrec + (2 * t + rg) * kStRec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = st_word_epoch(cv) == (epoch & kStEpochMask);
        }
        if (__syncthreads_and(ok)) break;
        if (++spins >= kStSpinLimit) {
          if (t == 0) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(8);
      }
#pragma unroll
      for (int u = 0; u < PU; ++u) {  // the records (count word + table), device-coherent 16-byte loads
        const int i = u * kStThreads + t, q = i / RU, part = i - q * RU;
        rv[u] = u32x4_t{0, 0, 0, 0};
        if (q < NC) {
          const int rg = round == 1 && bq_q[q] > b0;
          rv[u] = __builtin_amdgcn_raw_buffer_load_b128(rec_rsrc, (int)((((2 * q + rg) * kStRec) + 2 * part) * 8 +
                                                                        (long)r * NC * 2 * kStRec * 8), 0, kCpolDevice);
        }
      }
      DSV41_PX(1);
#pragma unroll 1
      for (int i = t; i < kHistBins; i += kStThreads) lhist[i] = 0;
      // count words first (the tables are relative to each chunk's top bin)
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const int i = u * kStThreads + t, q = i / RU, part = i - q * RU;
        if (q < NC && part == 0) {
          const unsigned long long cv = (unsigned long long)rv[u][1] << 32 | rv[u][0];
          cnt_q[q] = (int)(cv & 1023);
          tq_q[q] = (int)((cv >> 22) & 4095);
          if (round == 0) bq_q[q] = (int)((cv >> 10) & 4095);
          rg_q[q] = round == 1 && bq_q[q] > b0;
          lump_q[q] = 0;
        }
      }
      __syncthreads();
      // the unit's four chunks' candidates (all published ones), loaded now, filtered once B and T are known
#pragma unroll
      for (int cq = 0; cq < 4; ++cq) {
        const int q = sp * 4 + cq;
        uv[cq] = t < cnt_q[q] ? crow[(2 * q + rg_q[q]) * kStChunk + t] : 0ull;
      }
      bool any_lump = false;
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const int i = u * kStThreads + t, q = i / RU, part = i - q * RU;
        if (q >= NC) continue;
#pragma unroll
        for (int hw = 0; hw < 2; ++hw) {
          const int word = 2 * part + hw;  // record word (1..22: table)
          if (word < 1 || word > 22) continue;
          const unsigned long long w = (unsigned long long)rv[u][2 * hw + 1] << 32 | rv[u][2 * hw];
#pragma unroll
          for (int e3 = 0; e3 < 3; ++e3) {
            const int e = 3 * (word - 1) + e3, v = (int)((w >> (16 * e3)) & 0xffff);
            if (e < 64) tblq[q * 64 + e] = (uint16_t)v;
            if (v > 0) {
              if (e < 63) atomicAdd(&lhist[tq_q[q] - e], v);
              else if (e == 63) {
                lump_q[q] = 1;
                any_lump = true;
              }
            }
          }
        }
      }
      // chunks with candidates below their table's range: their candidates' bins, one wave per chunk
      if (__syncthreads_or(any_lump)) {
#pragma unroll 1
        for (int q = wave; q < NC; q += 8) {
          if (!lump_q[q]) continue;
          const unsigned long long* src = crow + (2 * q + rg_q[q]) * kStChunk;
          for (int e = lane; e < cnt_q[q]; e += 64) {
            const int bin = (int)((uint32_t)(src[e] >> 32) >> 20);
            if (bin <= tq_q[q] - 63) atomicAdd(&lhist[bin], 1);
          }
        }
        __syncthreads();
      }
      DSV41_PX(2);
      {  // threshold bin B: where the count from the top reaches k
        constexpr int BP = kHistBins / kStThreads;
        int h[BP], local = 0, total;
#pragma unroll
        for (int i = 0; i < BP; ++i) {
          h[i] = lhist[kHistBins - 1 - BP * t - i];
          local += h[i];
        }
        int above = block_scan_dpp<kStThreads>(local, tmp, &total);
        if (t == 0) {
          s_bin = 0;
          s_above = 0;
        }
        __syncthreads();
        if (above < k && k <= above + local) {
#pragma unroll 1
          for (int i = 0; i < BP; ++i) {
            if (k <= above + h[i]) {
              s_bin = kHistBins - 1 - BP * t - i;
              s_above = above;
              break;
            }
            above += h[i];
          }
        }
        __syncthreads();
      }
      // complete when every chunk published all of its positions at or above bin B
      const int ovf = __syncthreads_or(t < NC && rg_q[t] == 0 && bq_q[t] > s_bin);
      if (!ovf || round == 1) break;
      round = 1;
      b0 = s_bin;
      if (bq_q[ch] > b0) {  // republish from bin B0 (the histogram rebuilt from the chunk's scores)
#pragma unroll 1
        for (int i = t; i < kHistBins; i += kStThreads) lhist[i] = 0;
        __syncthreads();
        if (valid_mine) atomicAdd(&lhist[bin_mine], 1);
        __syncthreads();
        publish(1, b0);
      }
      __syncthreads();
    }
    DSV41_PX(3);
    const int B = s_bin, need = k - s_above;
    // per chunk: candidates above bin B (a prefix of its bin-grouped list) and in bin B: table entries in parallel
    if (t < NC) {
      ab_q[t] = 0;
      nb_q[t] = 0;
    }
    __syncthreads();
#pragma unroll 1
    for (int i = t; i < NC * 64; i += kStThreads) {
      const int q = i >> 6, e = i & 63, bin = tq_q[q] - e;
      if (e < 63 && !lump_q[q] && bin >= B) {
        const int v = tblq[i];
        if (v > 0) atomicAdd(bin > B ? &ab_q[q] : &nb_q[q], v);
      }
    }
    if (__syncthreads_or(t < NC && lump_q[t])) {  // (lumped chunks: scan their candidates, one wave per chunk)
#pragma unroll 1
      for (int q = wave; q < NC; q += 8) {
        if (!lump_q[q]) continue;
        const unsigned long long* src = crow + (2 * q + rg_q[q]) * kStChunk;
        int ab = 0, inb = 0;
        for (int e = lane; e < cnt_q[q]; e += 64) {
          const int bin = (int)((uint32_t)(src[e] >> 32) >> 20);
          ab += bin > B;
          inb += bin == B;
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
          ab += __shfl_xor(ab, m, 64);
          inb += __shfl_xor(inb, m, 64);
        }
        if (lane == 0) {
          ab_q[q] = ab;
          nb_q[q] = inb;
        }
      }
    }
    __syncthreads();
    // bin-B candidates of every chunk, compacted (their chunk's list holds them right after its ab_q entries
    // unless the chunk is lumped, where they are scattered: gathered by a scan)
    static_assert(kStMaxChunks <= 64, "one wave scans the chunks");
    if (wave == 0) {
      const int xq = lane < NC ? nb_q[lane] : 0;
      pu[lane + 1] = wave_incl_scan(xq);
      if (lane == 0) pu[0] = 0;
    }
    __syncthreads();
    const int mB = pu[NC];
    const bool bstaged = mB <= kLcbCap;
    if (bstaged) {
#pragma unroll 1
      for (int i = t; i < mB; i += kStThreads) {
        int lo = 0, hi = NC;
#pragma unroll 1
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (pu[mid] <= i) lo = mid;
          else hi = mid;
        }
        const unsigned long long* src = crow + (2 * lo + rg_q[lo]) * kStChunk;
        if (!lump_q[lo]) {
          lcb[i] = src[ab_q[lo] + i - pu[lo]];
        } else {
          int seen = 0;  // the (i - pu[lo])-th bin-B candidate of the lumped chunk
          for (int e = 0; e < cnt_q[lo]; ++e) {
            const unsigned long long v = src[e];
            if ((int)((uint32_t)(v >> 32) >> 20) == B && seen++ == i - pu[lo]) {
              lcb[i] = v;
              break;
            }
          }
        }
      }
      if (t == 0) lcb[mB] = 0ull;
    }
    __syncthreads();
    auto bcand_at = [&](int i) -> unsigned long long {
      if (bstaged) return lcb[i];
      int lo = 0;  // (a threshold bin past the LDS capacity: from memory)
      while (pu[lo + 1] <= i) ++lo;
      const unsigned long long* src = crow + (2 * lo + rg_q[lo]) * kStChunk;
      if (!lump_q[lo]) return src[ab_q[lo] + i - pu[lo]];
      int seen = 0;
      for (int e = 0; e < cnt_q[lo]; ++e) {
        const unsigned long long v = src[e];
        if ((int)((uint32_t)(v >> 32) >> 20) == B && seen++ == i - pu[lo]) return v;
      }
      return 0ull;
    };
    DSV41_PX(4);
    unsigned long long T;
    if (bstaged && mB <= kStThreads) {
      // the next 8 key bits (19..12) split bin B into 256 sub-bins: the sub-bin SB holding the need-th largest, then
      // direct ranks among SB's few candidates (all of bin B when SB holds too many: heavy ties)
      int* const sh = rs.rh;                                                  // 256 sub-bin counters
      unsigned long long* const lsb = (unsigned long long*)(rs.rh + 512);     // SB's candidates (<= 256)
      if (t < 256) sh[t] = 0;
      if (t == 0) {
        s_T = 0ull;  // (0: every bin-B candidate is taken)
        s_nsb = 0;
      }
      __syncthreads();
      const bool part = mB != need && t < mB;
      const unsigned long long me = part ? lcb[t] : 0ull;
      const int sbin = (int)((uint32_t)(me >> 32) >> 12) & 255;
      if (part) atomicAdd(&sh[sbin], 1);
      __syncthreads();
      if (mB != need && wave == 0) {  // lane l: sub-bins 255 - 4l .. 252 - 4l
        int c4[4], loc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c4[i] = sh[255 - 4 * lane - i];
          loc += c4[i];
        }
        const int incl = wave_incl_scan(loc);
        int run = incl - loc;
        if (run < need && need <= incl) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (run < need && need <= run + c4[i]) {
              s_sb = 255 - 4 * lane - i;
              s_need2 = need - run;
            }
            run += c4[i];
          }
        }
      }
      __syncthreads();
      if (mB != need) {
        const int SB = s_sb;
        if (part && sbin == SB) {
          const int o2 = atomicAdd(&s_nsb, 1);
          if (o2 < 256) lsb[o2] = me;
        }
        __syncthreads();
        const int nsb = s_nsb;
        if (nsb <= 256) {
          if (part && sbin == SB) {
            int rk = 0;
#pragma unroll 4
            for (int q2 = 0; q2 < nsb; ++q2) rk += lsb[q2] > me;
            if (rk == s_need2 - 1) s_T = me;
          }
        } else if (part) {  // (heavy ties: ranks among all of bin B)
          const uint4* l4 = (const uint4*)lcb;
          int rk = 0;
#pragma unroll 4
          for (int q2 = 0; q2 < (mB + 1) / 2; ++q2) {
            const uint4 w = l4[q2];
            rk += ((unsigned long long)w.y << 32 | w.x) > me;
            rk += ((unsigned long long)w.w << 32 | w.z) > me;
          }
          if (rk == need - 1) s_T = me;
        }
      }
      __syncthreads();
      T = s_T;
    } else {
      T = threshold_candidate<kStThreads>(bcand_at, lcb, bstaged, mB, need, (uint32_t)B << 20, rs);
    }
    DSV41_PX(5);
    // the unit's rows: each of its chunks' first ab_q candidates and its bin-B candidates >= T
    if (t == 0) s_nu = 0;
    if (t < NC) sb_q[t] = 0;
    __syncthreads();
#pragma unroll
    for (int cq = 0; cq < 4; ++cq) {
      const unsigned long long v = uv[cq];
      const int bin = (int)((uint32_t)(v >> 32) >> 20);
      if (t < cnt_q[sp * 4 + cq] && (bin > B || (bin == B && v >= T))) {
        const int o2 = atomicAdd(&s_nu, 1);
        if (o2 < kStMaxK) selidx[o2] = st_cand_pos(v);
      }
    }
    if (g.idx_out) {  // selected bin-B candidates per chunk (the index list's offsets)
#pragma unroll 1
      for (int i = t; i < mB; i += kStThreads) {
        const unsigned long long v = bcand_at(i);
        if (v >= T) atomicAdd(&sb_q[st_cand_pos(v) / kStChunk], 1);
      }
    }
    __syncthreads();
    n_unit = min(s_nu, kStMaxK);
  } else {  // every valid position is selected: the unit's positions below c
    const int p0 = sp * 4 * kStChunk;
    n_unit = max(0, min(c - p0, 4 * kStChunk));
#pragma unroll 1
    for (int i = t; i < n_unit; i += kStThreads) selidx[i] = p0 + i;
    __syncthreads();
  }
  DSV41_PH(4);

  // ================================================================ E. attention over the unit's selected rows
  const int nsel_tiles = (n_unit + kStTile - 1) / kStTile;
  auto resolve = [&](int ti) {
    if (t < kStTile) {
      const int li = ti * kStTile + t;
      const uint16_t* p = nullptr;
      if (li < n_unit) {
        const int ix = selidx[li];
        if (ix >= 0 && ix < at.n2) p = base_c + (long)ix * DQK;
      }
      rptr[ti % 3][t] = p;
    }
  };
  if (t == 0) s_bin = -1;
  if (nsel_tiles > 0) resolve(0);
  if (nsel_tiles > 1) resolve(1);
  __syncthreads();
  if (nsel_tiles > 0) issue(B0, rptr[0]);
  if (nsel_tiles > 1) issue(B1, rptr[1]);
  // while the first tiles load: a closing group's new compressed row among the rows, computed here (the table
  // write is another workgroup's)
  if (closes && g.latent) {
    for (int i = t; i < n_unit; i += kStThreads)
      if (selidx[i] == knew_row) s_bin = i;
  }
  lds_barrier();
  const int comp_at = s_bin;
  if (comp_at >= 0) row_op_keep<kStThreads, true>(make_op(1, false), creg, redf);
  DSV41_PX(7);
#pragma unroll 1
  for (int ti = 0; ti < nsel_tiles; ++ti) {
    if (ti + 1 < nsel_tiles)
      __builtin_amdgcn_s_waitcnt(kLoadsPerTile | (0x7 << 4) | (0xf << 8));  // vmcnt(kLoadsPerTile)
    else
      __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    uint16_t* buf = (ti & 1) ? B1 : B0;
    if (comp_at >= ti * kStTile && comp_at < (ti + 1) * kStTile) {
      patch(buf, comp_at - ti * kStTile, creg);
      lds_barrier();
    }
    if (ti == 0) DSV41_PX(8);
    compute(buf, rptr[ti % 3]);
    if (ti == 0) DSV41_PX(9);
    if (ti + 2 < nsel_tiles) {
      resolve(ti + 2);
      lds_barrier();
      issue(buf, rptr[(ti + 2) % 3]);
    }
  }
  __syncthreads();
  DSV41_PH(5);

  // ---- the 4 row-waves' states per head, then this split's bf16-normalised partial (or the output, S == 1)
  constexpr int DVP = DV + 4;
  if (half == 0 && g4 == 0) {
    wm[rw][l16] = m_ref;
    wl[rw][l16] = l_run;
  }
  __syncthreads();
  if (t < 16) {
    const float M = fmaxf(fmaxf(wm[0][t], wm[1][t]), fmaxf(wm[2][t], wm[3][t]));
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(wm[w][t] - M);
      wf[w][t] = f;
      L += wl[w][t] * f;
    }
    hM[t] = M;
    hL[t] = L;
  }
  __syncthreads();
  {
    float* xw = (float*)smem + rw * 16 * DVP + half * (DV / 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float fac = wf[rw][4 * g4 + i];
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct) xw[(4 * g4 + i) * DVP + ct * 16 + l16] = o[ct][i] * fac;
    }
  }
  __syncthreads();
  DSV41_PX(10);
  const float* xb = (const float*)smem;
  const long pr = ppos < 0 ? 0 : ppos;
  const float ln2 = 0.6931471805599453f;
  constexpr int CG = DV / 8;
  const int H = at.H;
#pragma unroll 1
  for (int e = t; e < 16 * CG; e += kStThreads) {
    const int hh = e / CG, c8 = (e - hh * CG) * 8, hout = h0 + hh;
    const float M = hM[hh], L = hL[hh];
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 x0 = *(const float4*)(xb + (w * 16 + hh) * DVP + c8);
      const float4 x1 = *(const float4*)(xb + (w * 16 + hh) * DVP + c8 + 4);
      v[0] += x0.x, v[1] += x0.y, v[2] += x0.z, v[3] += x0.w;
      v[4] += x1.x, v[5] += x1.y, v[6] += x1.z, v[7] += x1.w;
    }
    uint32_t pk[4];
    if (S == 1) {
      const float inv = 1.0f / (L + exp2f(at.sink[hout] * kLog2e - M));
#pragma unroll
      for (int q = 0; q < 8; q += 2) {
        float re = round_bf16(v[q] * inv), im = round_bf16(v[q + 1] * inv);
        const int cc = c8 + q;
        if (at.rd > 0 && cc >= DV - at.rd) {
          const int jr = (cc - (DV - at.rd)) >> 1;
          const float cs = at.cos_t[pr * (at.rd / 2) + jr], sn = -at.sin_t[pr * (at.rd / 2) + jr];
          const float yr = re * cs - im * sn, yi = re * sn + im * cs;
          re = yr;
          im = yi;
        }
        pk[q / 2] = pack_bf16x2(re, im);
      }
      *(uint4*)(at.out + (long)r * at.out_rstride + (long)hout * DV + c8) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
      for (int q = 0; q < 8; q += 2) pk[q / 2] = pack_bf16x2(v[q] * inv, v[q + 1] * inv);
      const long pi = ((long)r * H + hout) * S + sp;
      __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{pk[0], pk[1], pk[2], pk[3]}, pacc_rsrc(at.pacc),
                                             (int)((pi * DV + c8) * 2), 0, kCpolDevice);
      if (c8 == 0) {
        __hip_atomic_store(at.pm + pi, M * ln2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(at.pl + pi, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // the index list (idx_out, head group 0 of each unit): the unit's rows ranked in ascending order at the unit's
  // offset (the selected rows of the earlier units' chunks); split 0 also pads the list with -1 past kk
  auto write_idx = [&]() {
    if (!g.idx_out || hg != 0) return;
    int* orow_i = g.idx_out + (long)r * g.idx_rstride;
    int before = sp * 4 * kStChunk;
    if (sel) {
      before = 0;
      for (int q = 0; q < sp * 4; ++q) before += ab_q[q] + sb_q[q];
    }
#pragma unroll 1
    for (int i = t; i < n_unit; i += kStThreads) {
      const int me = selidx[i];
      int rank = 0;
#pragma unroll 4
      for (int j = 0; j < n_unit; ++j) rank += selidx[j] < me;
      if (before + rank < k) orow_i[before + rank] = me + g.offset;
    }
    if (sp == 0)
      for (int i = kk + t; i < k; i += kStThreads) orow_i[i] = -1;
  };
  if (S == 1) {
    write_idx();
    return;
  }
  // ---- cooperative merge of the (row, head group)'s S splits: counter = epoch * 256 + arrivals
  unsigned long long* cntm = at.coop + (long)r * 4 + hg;
  DSV41_PX(11);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  DSV41_PX(12);
  if (t == 0) {
    const unsigned long long old = __hip_atomic_fetch_add(cntm, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long base = old & ~255ull;
    if ((int)(old & 255) + 1 == S) {
      __hip_atomic_fetch_add(cntm, 256ull - S, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      int spins = 0;
#pragma unroll 1
      while (__hip_atomic_load(cntm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < base + S && ++spins < kStSpinLimit)
        __builtin_amdgcn_s_sleep(8);
      if (spins >= kStSpinLimit) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  DSV41_PH(6);
  at.nsplit = S;
  merge_slice<DV>(at, r, h0, pr, sp);
  DSV41_PH(7);
  write_idx();
}

int st_chunks(int n_pos) { return ((n_pos + kStChunk - 1) / kStChunk + 3) / 4 * 4; }

// Compute units of the current device (queried once per device).
int st_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

struct StLayout {
  long rec, cand, coop, pm, pl, pacc, total;
};

StLayout st_layout(int R, int n_pos, int h, int dv) {
  const long NC = st_chunks(n_pos), S = NC / 4;
  auto up = [](long x) { return (x + 255) / 256 * 256; };
  StLayout L{};
  L.rec = 256;  // (bytes 0..255: the error word)
  L.cand = L.rec + up(R * NC * 2 * kStRec * 8);
  L.coop = L.cand + up(R * NC * 2 * kStChunk * 8);
  L.pm = L.coop + up((long)R * 4 * 8);
  L.pl = L.pm + up((long)R * h * S * 4);
  L.pacc = L.pl + up((long)R * h * S * 4);
  L.total = L.pacc + up((long)R * h * S * dv * 2);
  return L;
}

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_ph_step(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ph), sizeof(g_dsv41_ph)); }
int dsv41_read_px_step(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_px), sizeof(g_dsv41_px)); }
int dsv41_read_ck_step(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ck), sizeof(g_dsv41_ck)); }
#endif

long dsv41_decode_step_workspace_bytes(int R, int n_pos, int h, int dv) {
  if (R <= 0 || n_pos <= 0 || h <= 0 || dv <= 0) return 0;
  return st_layout(R, n_pos, h, dv).total;
}

int dsv41_decode_step_fits(int R, int n_pos, int h, int k, int W, int dqk, int dv) {
  if (R <= 0 || n_pos <= 0) return 0;
  const int NC = st_chunks(n_pos), S = NC / 4, G = R * NC;
  const int cus = st_cus();
  return h == 64 && NC <= kStMaxChunks && G % 32 == 0 && cus > 0 && G <= cus && k > 0 && k <= kStMaxK &&
         W > 0 && W % kStTile == 0 && W / kStTile <= S && S <= 32 &&
         ((dqk == 576 && dv == 512) || (dqk == 512 && dv == 512));
}

int dsv41_decode_step(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                      const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw, const void* k_norm,
                      void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks, long ks_sstride, int kcap,
                      const long* pos, const long* seq, int R, int ratio, const float* cos_t, const float* sin_t,
                      int rd, float eps, const void* q_idx, const void* w_idx, int HI, const long* cl, int n_pos,
                      int k, int offset, const void* q, int h, const long* pmax, const long* plim, const float* sink,
                      int out_rd, float scale, void* out, int* idx_out, long idx_rstride, float* score_out,
                      long score_rstride, void* ws, long ws_bytes, void* stream) {
  if (R <= 0) return 0;
  const int dqk = Dw, dv = dqk == 576 ? 512 : dqk;
  if (!dsv41_decode_step_fits(R, n_pos, h, k, W, dqk, dv)) return (int)hipErrorInvalidValue;
  if (!kv_raw || !kv_norm || !ring || !ckv || !k_raw || !k_norm || !k8 || !ks || !pos || !seq || !cl || !q_idx ||
      !w_idx || !q || !pmax || !sink || !out || HI <= 0 || HI > 64 || ratio <= 0 || rd < 0 || rd % 2 || rd > 128 ||
      out_rd < 0 || out_rd % 2 || out_rd > dv || n_pos > kcap || n_pos > cap)
    return (int)hipErrorInvalidValue;
  const StLayout L = st_layout(R, n_pos, h, dv);
  if (!ws || ws_bytes < L.total || ((uintptr_t)ws & 255)) return (int)hipErrorInvalidValue;
  char* w = (char*)ws;
  StepArgs g{};
  ScoreArgs& a = g.s;
  a.q = nullptr;
  a.HI = HI;
  a.R = R;
  a.kfmt = 1;
  a.keys = k8;
  a.k_sstride = k8_sstride;
  a.kscale = ks;
  a.ks_sstride = ks_sstride;
  a.seq = seq;
  a.rows_per_slot = 1;
  a.cl = cl;
  a.n_pos = n_pos;
  a.write_masked = 1;
  a.out = score_out;
  a.out_rstride = score_rstride;
  g.kv_raw = (const uint16_t*)kv_raw;
  g.kv_norm = (const uint16_t*)kv_norm;
  g.ring = (uint16_t*)ring;
  g.ring_sstride = ring_sstride;
  g.W = W;
  g.Dw = Dw;
  g.latent = (const uint16_t*)latent;
  g.ckv = (uint16_t*)ckv;
  g.ckv_sstride = ckv_sstride;
  g.cap = cap;
  g.k_raw = (const uint16_t*)k_raw;
  g.k_norm = (const uint16_t*)k_norm;
  g.kbf = (uint16_t*)kbf;
  g.kbf_sstride = kbf_sstride;
  g.k8 = (uint8_t*)k8;
  g.k8_sstride = k8_sstride;
  g.ks = ks;
  g.ks_sstride = ks_sstride;
  g.kcap = kcap;
  g.pos = pos;
  g.ratio = ratio;
  g.rd = rd;
  g.cos_t = cos_t;
  g.sin_t = sin_t;
  g.eps = eps;
  g.q_idx = (const uint16_t*)q_idx;
  g.w_idx = (const uint16_t*)w_idx;
  g.k = k;
  g.offset = offset;
  g.idx_out = idx_out;
  g.idx_rstride = idx_rstride;
  g.nc = st_chunks(n_pos);
  g.S = g.nc / 4;
  g.rec = (unsigned long long*)(w + L.rec);
  g.cand = (unsigned long long*)(w + L.cand);
  g.err = (int*)w;
  AttnArgs& at = g.at;
  at.q = (const uint16_t*)q;
  at.q_rstride = (long)h * dqk;
  at.H = h;
  at.R = R;
  at.mode = 1;
  at.kv1 = (const uint16_t*)ring;
  at.kv1_sstride = ring_sstride;
  at.n1 = W;
  at.kv2 = (const uint16_t*)ckv;
  at.kv2_sstride = ckv_sstride;
  at.n2 = cap;
  at.pos = pos;
  at.seq = seq;
  at.pmax = pmax;
  at.plim = plim;
  at.scale = scale;
  at.sink = sink;
  at.out = (uint16_t*)out;
  at.out_rstride = (long)h * dv;
  at.nsplit = g.S;
  at.pm = (float*)(w + L.pm);
  at.pl = (float*)(w + L.pl);
  at.pacc = (float*)(w + L.pacc);
  at.coop = (unsigned long long*)(w + L.coop);
  at.err = (int*)w;
  at.cos_t = cos_t;
  at.sin_t = sin_t;
  at.rd = out_rd;
  const dim3 grid(R * g.nc);
  if (dqk == 576)
    decode_step_kernel<576, 512><<<grid, kStThreads, 0, (hipStream_t)stream>>>(g);
  else
    decode_step_kernel<512, 512><<<grid, kStThreads, 0, (hipStream_t)stream>>>(g);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
