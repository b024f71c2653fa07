// Decode lightning indexer in one launch: the scores of a row's compressed positions and the top-k selection
// (dsv41/decode.py:284-294, index_score followed by topk_indices; scores as dsv41/fused3.py:20-62, the k largest of
// score[r, 0..cl) in ascending index order with -1 padding as dsv41/fused3.py:65-75, ties lowest index first).
//
// Grid: R x nslots workgroups of 512 threads (chunk ch of row r is workgroup ch * R + r, so a row's chunks spread
// over the XCDs), all resident at once (at most kIsMaxWG: 2 per CU).  FUSED: chunk workgroups also do the step's
// cache appends while their key loads are in flight (the chunk holding the new key's position scores it itself).  Each
// workgroup scores its 512 positions (8 waves x 64 keys, every key load issued up front, e4m3 keys against the
// prepared e4m3 queries, fp8 MFMA) and keeps them in LDS.  Then, on the one-exchange path (pub_m > 0):
//   P. publishes the keys at or above a cut that keeps at least pub_m of its positions (4096 bins over its own key
//      range) and the largest key it leaves out, then a flag word with the launch epoch;
//   Q. reads every chunk's flag until all carry this epoch (the row barrier), then every published list (16-byte
//      loads); LB = the largest left-out key of the row, T = the k-th largest published key above LB;
//   R. when T exists and no key ties with T across the cut, writes its keys >= T at the offset counted from the
//      earlier chunks' published keys >= T (ascending positions).  Every chunk of a row reads the same published
//      data and takes the same decision; otherwise (a chunk holding more of the selection than it published, ties at
//      T) the row takes the two-exchange path, which is also the whole path when pub_m == 0:
//   A. the chunk's 4096-bin histogram (top 12 bits of the order-preserving key) added to the row's with device-scope
//      atomics
//   B. reads the row histogram until its total reaches the row's valid count (every chunk's additions have landed:
//      this read is the row barrier and its data at once); threshold bin B (where the running count from the top
//      reaches k) and need = k - (entries above B)
//   C. classifies its positions (one per thread): entries above B are counted, bin-B candidates
//      (key << 32 | epoch tag << 18 | ~position) stored in the chunk's slots, then the counts with the launch epoch
//   D. reads every chunk's count word and the first kIsSpec candidates of each chunk until all carry this launch's
//      epoch (the second row barrier and the gather in one round trip); clears its slice of the row histogram
//   E. threshold candidate T (exact ranks / radix passes over the candidates)
//   F. writes its taken positions (above B, or candidates >= T) at their global offset.
// Data exchanged between workgroups (lists, flags, histogram, counts, candidates) is written and read with
// device-scope operations (sc1), which the hardware keeps coherent across the XCDs' L2 caches, so no cache
// maintenance is needed; a publisher waits for its data stores to complete (s_waitcnt) before it stores the flag or
// count word a reader polls, and relies on the hardware keeping that order for device-scope accesses (an agent-scope
// release / acquire would write back / invalidate whole L2 caches).  The epoch of a launch is one more than the one
// the chunk's count word holds from the previous launch.  A wait gives up after kIsSpinLimit polls and sets the error
// word, so every wave exits.
#include <cstdlib>

#include "rowop.h"
#include "score_core.h"
#include "select_core.h"

namespace {

constexpr int kIsThreads = 512;                // 8 waves: two per SIMD
constexpr int kIsChunk = 512;                  // positions per workgroup
constexpr int kIsKeysPerWave = kIsChunk / 8;   // 4 column tiles of 16 keys
constexpr int kIsPer = kIsChunk / kIsThreads;  // positions per thread in the selection
// candidates per chunk read together with the counts: 16 up to 128 chunks per row, 1 beyond (every workgroup of a
// row reads every chunk's prefix; a long row's threshold bin holds well under one candidate per chunk on average)
template <int MAXC>
constexpr int is_spec() { return MAXC <= 128 ? 16 : 1; }
constexpr int kIsCand = 2048;                  // candidates staged in LDS (more: read from the workspace)
constexpr int kIsMaxChunks = 512;              // chunks per row (rows up to 262144 positions)
constexpr int kIsMaxWG = 512;                  // resident workgroups: 2 per CU
constexpr int kIsSpinLimit = 1 << 20;

constexpr int kIsLst = kIsChunk + 4;           // published-list slots per chunk (16-byte aligned lists)
constexpr int kIsRd = 16;                      // published-list slots read per thread (more: the two-exchange path)
// Per-chunk count words and flags (u64, written with device-scope stores by one chunk each) lie 128 bytes apart:
// device-scope writes to one cache line from different CUs serialise at the memory side.
constexpr int kIsWordStride = 16;
// 16-byte reads of the published lists with the device-scope cache policy (sc1) of the atomics that wrote them
typedef unsigned is_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kIsCpolDevice = 16;
constexpr int kIsTagShift = 18;  // candidate low word: epoch tag (14 bits) << 18 | (~position & 0x3ffff)
static_assert(kIsMaxChunks * kIsChunk <= (1 << kIsTagShift), "positions fit below the epoch tag");

// Candidate value: order by key, then by lower position; every candidate of one launch carries the same tag.
DSV41_DEV unsigned long long is_cand_value(uint32_t key, int p, uint32_t tag) {
  return (unsigned long long)key << 32 | tag << kIsTagShift | (~(uint32_t)p & ((1u << kIsTagShift) - 1));
}

// The decode step's cache appends done inside the launch (dsv41_decode_select; the operations of
// dsv41_decode_appends): the SWA ring row, the compressed row and the index key of every row, and the e4m3
// preparation of the index queries.
struct IsAppend {
  const uint16_t* kv_raw;  // [R, Dw] pre-norm KV rows, rmsnorm weight kv_norm
  const uint16_t* kv_norm;
  uint16_t* ring;          // [S, W, Dw]
  long ring_sstride;
  int W, Dw;
  const uint16_t* latent;  // [R, Dw] pooled latents (may be null: no compressed append)
  uint16_t* ckv;           // [S, cap, Dw]
  long ckv_sstride;
  int cap;
  const uint16_t* k_raw;   // [R, 128] index-key rows, rmsnorm weight k_norm
  const uint16_t* k_norm;
  uint16_t* kbf;           // optional bf16 key table [S, kcap, 128]
  long kbf_sstride;
  uint8_t* k8;             // e4m3 key table [S, kcap, 128] + scales (the keys this launch scores)
  long k8_sstride;
  float* ks;
  long ks_sstride;
  int kcap;
  const long* pos;
  const long* nw_tab;      // [S] no-write row per sequence (null: the tables' spare last row cap - 1 / kcap - 1)
  int ratio, rd;
  const float* cos_t;
  const float* sin_t;
  float eps;
  const uint16_t* q_idx;   // [R, HI, 128] bf16 index queries, w_idx [R, HI] bf16 head weights
  const uint16_t* w_idx;
};

// Row operation `which` of row r's appends (0: the SWA ring row, 1: the compressed row, 2: the index key, with an
// LDS copy of its e4m3 bytes and scale in knew / ksnew when given); position ppos, sequence slot.  Compressed /
// index-key rows go to compress_len - 1 when the step closes a group, else to the sequence's no-write row
// (nw_tab[slot]: the last row of the slot's own capacity, dsv41/decode.py:176-181) or, without a table, to the
// table's spare last row.
DSV41_DEV RowOp is_app_op(const IsAppend& ap, int r, long slot, long ppos, int which, uint8_t* knew, float* ksnew) {
  RowOp o{};
  o.cos_t = ap.cos_t;
  o.sin_t = ap.sin_t;
  o.rd = ap.rd;
  o.eps = ap.eps;
  const bool closes = ((ppos + 1) % ap.ratio) == 0;
  if (which == 0) {
    o.x = ap.kv_raw + (long)r * ap.Dw;
    o.D = ap.Dw;
    o.norm_w = ap.kv_norm;
    o.pos = ppos < 0 ? 0 : ppos;
    o.qmode = 0;
    o.group = 32;
    o.out = ap.ring + slot * ap.ring_sstride + (o.pos % ap.W) * (long)ap.Dw;
  } else if (which == 1) {
    const long row = closes ? (ppos + 1) / ap.ratio - 1 : ap.nw_tab ? ap.nw_tab[slot] : ap.cap - 1;
    o.x = ap.latent + (long)r * ap.Dw;
    o.D = ap.Dw;
    o.pos = ppos + 1 - ap.ratio;
    o.qmode = 2;
    o.group = 16;
    o.out = ap.ckv + slot * ap.ckv_sstride + row * (long)ap.Dw;
  } else {
    const long row = closes ? (ppos + 1) / ap.ratio - 1 : ap.nw_tab ? ap.nw_tab[slot] : ap.kcap - 1;
    o.x = ap.k_raw + (long)r * 128;
    o.D = 128;
    o.norm_w = ap.k_norm;
    o.pos = ppos + 1 - ap.ratio;
    o.qmode = 1;
    o.group = 32;
    o.out = ap.kbf ? ap.kbf + slot * ap.kbf_sstride + row * 128L : nullptr;
    o.k8 = ap.k8 + slot * ap.k8_sstride + row * 128L;
    o.ks = ap.ks + slot * ap.ks_sstride + row;
    o.k8_lds = knew;
    o.ks_lds = ksnew;
  }
  return o;
}

// The index-key append of a step that closes a group, to table row `row` (= compress_len - 1), with the LDS copy.
DSV41_DEV RowOp is_key_op(const IsAppend& ap, int r, long slot, long ppos, long row, uint8_t* knew, float* ksnew) {
  RowOp o{};
  o.cos_t = ap.cos_t;
  o.sin_t = ap.sin_t;
  o.rd = ap.rd;
  o.eps = ap.eps;
  o.x = ap.k_raw + (long)r * 128;
  o.D = 128;
  o.norm_w = ap.k_norm;
  o.pos = ppos + 1 - ap.ratio;
  o.qmode = 1;
  o.group = 32;
  o.out = ap.kbf ? ap.kbf + slot * ap.kbf_sstride + row * 128L : nullptr;
  o.k8 = ap.k8 + slot * ap.k8_sstride + row * 128L;
  o.ks = ap.ks + slot * ap.ks_sstride + row;
  o.k8_lds = knew;
  o.ks_lds = ksnew;
  return o;
}

// The appends in bit set `late` of row r (bit w: is_app_op's operation w), one after another (whole-block barriers).
DSV41_DEV void is_late_appends(const IsAppend& ap, int r, long slot, long ppos, int late, float* red) {
  if (late & 1) row_op<512>(is_app_op(ap, r, slot, ppos, 0, nullptr, nullptr), red);
  if (late & 2) row_op<512>(is_app_op(ap, r, slot, ppos, 1, nullptr, nullptr), red);
  if (late & 4) row_op<512>(is_app_op(ap, r, slot, ppos, 2, nullptr, nullptr), red);
}

// Largest u32 over the 64 lanes of a wave, in every lane: DPP lane moves as wave_incl_scan (lanes a move does not
// reach keep their own value), then lane 63's result.
DSV41_DEV uint32_t wave_umax(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x111, 0xf, 0xf, false));  // row_shr:1
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x112, 0xf, 0xf, false));  // row_shr:2
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x114, 0xf, 0xf, false));  // row_shr:4
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x118, 0xf, 0xf, false));  // row_shr:8
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x142, 0xa, 0xf, false));  // row_bcast:15
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// Largest of two u32 values each over the NT threads of a workgroup (red: 2 * NT / 64 words); one barrier, and
// red must not be written again before a later barrier.
template <int NT>
DSV41_DEV void block_umax2(uint32_t& x0, uint32_t& x1, uint32_t* red) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  x0 = wave_umax(x0);
  x1 = wave_umax(x1);
  if (lane == 0) red[wave] = x0, red[NW + wave] = x1;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) x0 = max(x0, red[w]), x1 = max(x1, red[NW + w]);
}

// Shift that maps a key range [0, range] onto at most 4096 bins.
DSV41_DEV int bin_shift(uint32_t range) {
  const int b = 32 - __clz(range);
  return b > 12 ? b - 12 : 0;
}

// Over 4096 LDS bins h (bin 0 first), the bin where the running count reaches x (1 <= x <= total): *bin and the
// count before it, *before (into shared s_out[0], s_out[1]); NT = 512 threads, 8 bins each.  Barriers inside.
DSV41_DEV void bins_reach(const int* h, int x, int* tmp, int* s_out) {
  const int t = threadIdx.x;
  int v[8], local = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = h[8 * t + i], local += v[i];
  int tot;
  int before = block_scan_dpp<512>(local, tmp, &tot);
  if (before < x && x <= before + local) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (before < x && x <= before + v[i]) {
        s_out[0] = 8 * t + i;
        s_out[1] = before;
      }
      before += v[i];
    }
  }
  __syncthreads();
}

struct IsArgs {
  ScoreArgs s;                // prepared e4m3 queries, folded weights, e4m3 keys + scales, seq, cl, n_pos; out or null
  int k, offset;
  int* idx;
  long idx_rstride;
  int nslots;                 // chunks per row
  int* hist;                  // [R, kHistBins], zero between launches
  unsigned long long* cnt;    // [R, nslots]: epoch << 32 | candidates << 16 | above
  unsigned long long* cand;   // [R, nslots * kIsChunk]
  int* err;
  IsAppend app;               // FUSED instances only
  // one-exchange selection (pub_m > 0): every chunk publishes its top entries (at least pub_m of the chunk's keys)
  int pub_m;
  unsigned long long* fl;     // [R, nslots]: epoch << 32 | entries published
  uint32_t* lst;              // [R, nslots, kIsLst]: entry 0 the largest unpublished key (0: none), then the keys
};

#ifdef DSV41_TIMING
__device__ int g_is_spins[1024][2];  // polls of the two waits per workgroup
#endif

// MAXC: the largest chunk count per row the instance handles (128: the candidate-prefix gather and the chunk
// prefix scans fit 4 loads per thread and two waves; kIsMaxChunks: 16 loads per thread and a workgroup scan).
template <int MAXC, bool FUSED>
__global__ void __launch_bounds__(kIsThreads, 4) index_select_kernel(const IsArgs g) {
  static_assert(MAXC <= kIsThreads && MAXC % 64 == 0, "one thread per chunk");
  const ScoreArgs& a = g.s;
  const int R = a.R, ns = g.nslots;
  const int bx = (int)blockIdx.x;
  const int r = bx % R, ch = bx / R;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  __shared__ int lhist[kHistBins];
  __shared__ float sc[kIsChunk];
  __shared__ int tmp[8];
  __shared__ int wcnt[8][2];
  __shared__ int s_bin, s_need, s_cnt, s_selb, s_over;
  __shared__ int pc[MAXC + 1], na_q[MAXC], nc_q[MAXC];
  __shared__ __align__(16) unsigned long long lc[kIsCand + 2];
  __shared__ RankScratch rs;
  __shared__ __align__(16) uint8_t qs[64 * 128];  // the row's prepared e4m3 queries, staged once
  __shared__ float wfl[FUSED ? 64 : 1];            // (FUSED) the prepared head weights
  __shared__ __align__(16) uint8_t knew[FUSED ? 128 : 16];  // (FUSED) the new index key, e4m3, and its scale
  __shared__ float ksnew, redf[kIsThreads / 64];
  __shared__ uint32_t ured[4 * kIsThreads / 64], s_T;  // (one-exchange path) reductions and scans
  __shared__ int s_ro[2], s_m1, s_tie;

  // ---- A. row data (independent loads), scores, histogram
  DSV41_PH(0);
  DSV41_PX(0);
  DSV41_TS(48);
  Qprep512 qp;
  // (FUSED) the row's queries first, in flight with the row data: issued after the key loads instead, they were
  // waited for before the key addresses could reuse their address registers
  if constexpr (FUSED)
    qprep512_load(g.app.q_idx + (long)r * a.HI * 128, g.app.w_idx + (long)r * a.HI, a.HI, qp);
  const long clr = row_cl(a, r);
  const long slot = a.seq ? a.seq[r] : (long)(r / a.rows_per_slot);
  // this launch's epoch: one more than the one this chunk's count word holds (earlier launches have completed).
  // Read after the key loads are issued: the device-scope load returns late, and a wait for any later load (loads
  // return in order) would wait for it too
  uint32_t epoch = 0, tag = 0;
  auto read_epoch = [&]() {
    // (the high word alone: a 64-bit load whose low half is dead lets the compiler reuse that register, which
    // then waits for the load -- the last one issued, so for every key load)
    epoch = __hip_atomic_load((const uint32_t*)(g.cnt + ((long)r * ns + ch) * kIsWordStride) + 1, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT) + 1;
    tag = epoch & ((1u << (32 - kIsTagShift)) - 1);
  };
  const int c = (int)(clr < 0 ? 0 : (clr > a.n_pos ? a.n_pos : clr)), k = g.k;
  const int nht = (a.HI + 15) / 16;
  i32x8_t qa8[kHT];
  uint4 qa16[kHT][4];  // (bf16 queries: unused here)
  float wl[kHT];
  // FUSED: the step's cache appends are done by chunk workgroups.  When the step closes a group, the chunk holding
  // the new key's position writes the key with one wave while its key loads are in flight (its operands loaded
  // before them, so waiting for those does not wait for the keys; every chunk issues those few loads, so that no
  // branch holds them) and scores it from its LDS copy in place of the table row its
  // loads read.  The ring row (chunk 0), the compressed row (chunk 1) and a non-closing step's key (chunk 2, to the
  // no-write row) are nothing this launch reads: they are written while the chunk waits at the row barrier (a row
  // of fewer chunks gives several to one).
  const IsAppend& ap = g.app;
  long ppos = 0, knew_row = -1;
  bool holder = false;  // (FUSED) this chunk holds the new key's position
  int late = 0;         // (FUSED) bit w: append w (0 ring, 1 compressed row, 2 index key) is this chunk's, written late
  RowRegs<64, 128> rr;  // (FUSED) the key's operands: one wave's share of a 128-wide row
  RowOp kop{};
  if constexpr (FUSED) {
    ppos = ap.pos[r];
    const bool closes = ((ppos + 1) % ap.ratio) == 0;
    if (closes) knew_row = (ppos + 1) / ap.ratio - 1;
    holder = closes && knew_row >= 0 && knew_row < c && ch == (int)(knew_row / kIsChunk);
    late = (ch == 0 ? 1 : 0) | (ch == min(1, ns - 1) && ap.latent && ap.ckv ? 2 : 0);
    if (!(closes && knew_row >= 0 && knew_row < c) && ch == min(2, ns - 1)) late |= 4;
    // (every chunk loads the key's operands -- valid addresses whether or not the step closes a group --, so no
    // branch holds the loads; only the holder uses them)
    kop = is_key_op(ap, r, slot, ppos, knew_row < 0 ? 0 : knew_row, knew, &ksnew);
    row_load<64, 128>(kop, rr);
  } else {
    // the row's queries (64 heads x 128 e4m3 = 512 chunks of 16 bytes) go to LDS once, one direct load per thread
    // (every wave needs all of them); heads >= HI are never read back
    if (t < a.HI * 8) lds_dma16((const uint16_t*)((const uint8_t*)a.q + (long)r * a.q_rstride) + t * 8,
                                (uint16_t*)qs + wave * 64 * 8);
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      const int h = ht * 16 + l16;
      const bool hv = ht < nht && h < a.HI;
      wl[ht] = hv ? a.w[(long)r * a.w_rstride + h] : 0.0f;
    }
  }
  DSV41_TS(49);
  DSV41_PX(1);
  static_assert(kHistBins % kIsThreads == 0, "histogram clear");
#pragma unroll
  for (int j = 0; j < kHistBins / kIsThreads; ++j) lhist[t + j * kIsThreads] = 0;  // (no loop between the loads)
  constexpr int NT = kIsKeysPerWave / 16;  // column tiles of 16 keys per wave, all loads issued up front
  uint4 k0[NT], k1[NT];
  float ksc[NT];
  const int pw = ch * kIsChunk + wave * kIsKeysPerWave;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    // positions past the row load row 0 (unconditional loads: a select on a loaded value would make the compiler
    // wait for it before the later tiles' loads are issued); their scores are not recorded
    const int p = pw + nt * 16 + l16, pl = p < c ? p : 0;
    const uint8_t* krow = (const uint8_t*)a.keys + slot * a.k_sstride + (long)pl * 128 + g4 * 32;
    k0[nt] = *(const uint4*)krow;
    k1[nt] = *(const uint4*)(krow + 16);
    ksc[nt] = a.kscale[slot * a.ks_sstride + pl];
  }
  read_epoch();
  // (stored after the row's loads are issued: a global store before them makes the compiler load the row data
  // through the vector path and wait for every earlier load)
  if (clr > a.n_pos && ch == 0 && t == 0)  // positions beyond n_pos were promised never to be valid
    __hip_atomic_store(g.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  DSV41_TS(50);
  DSV41_PX(2);
  if constexpr (FUSED) {
    DSV41_PX(4);
    qprep512_store(qp, a.HI, qs, wfl);
    // the new key by one wave (no barriers: a whole-block row operation's chain of barriers held every wave of the
    // holder up); the others go on to wait for their key loads
    if (holder && wave == 0) row_compute<64, true, 128>(kop, rr, redf);
    lds_barrier();  // queries and weights staged (and the new key's LDS copy)
    DSV41_PX(5);
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      const int h = ht * 16 + l16;
      wl[ht] = ht < nht && h < a.HI ? wfl[h] : 0.0f;
    }
  }
  float wr[kHT][4];  // weights of the heads this lane's accumulators hold: ht*16 + 4g + i
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wl[ht], 4 * g4 + i, 64);
  __syncthreads();  // histogram cleared, queries staged
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    const int h = ht * 16 + l16;
    const int hc = ht < nht && h < a.HI ? h : 0;
    const uint4 u0 = *(const uint4*)(qs + hc * 128 + g4 * 32), u1 = *(const uint4*)(qs + hc * 128 + g4 * 32 + 16);
    qa8[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
  }
  DSV41_TS(52);
  const bool sel = c > k;  // (otherwise every valid position is taken)
  float* orow = a.out ? a.out + (long)r * a.out_rstride : nullptr;
  uint32_t kmax = 0u, kmin_c = 0u;  // (one-exchange path) largest key and complement of the smallest, this lane
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int p = pw + nt * 16 + l16;
    if (FUSED && holder && p == knew_row) {  // the new key: this launch's LDS copy, not the table row loaded
      k0[nt] = *(const uint4*)(knew + g4 * 32);
      k1[nt] = *(const uint4*)(knew + g4 * 32 + 16);
      ksc[nt] = ksnew;
    }
    const float sum = score_tile<1>(qa8, qa16, wr, nht, k0[nt], k1[nt], nullptr);
    if (g4 == 0) {
      const float v = p < c ? (is_cand(a, r, p) ? sum * ksc[nt] : -__builtin_inff()) : 0.0f;
      sc[p - ch * kIsChunk] = v;
      if (p < c) {
        const uint32_t kv = score_key(v);
        kmax = max(kmax, kv);
        kmin_c = max(kmin_c, ~kv);
      }
      if (p < c && sel && g.pub_m == 0) atomicAdd(&lhist[score_key(v) >> 20], 1);
      if (orow && p < a.n_pos) orow[p] = p < c ? v : -__builtin_inff();
    }
  }
  DSV41_TS(53);
  DSV41_PX(6);
  if (g.pub_m > 0) {  // the chunk's key range, for the one-exchange path's cut (read after the barrier below)
    kmax = wave_umax(kmax);
    kmin_c = wave_umax(kmin_c);
    if (lane == 0) ured[wave] = kmax, ured[8 + wave] = kmin_c;
  }
  __syncthreads();
  DSV41_PH(1);
  DSV41_TS(54);
  int* gh = g.hist + (long)r * kHistBins;
  unsigned long long* rcnt = g.cnt + (long)r * ns * kIsWordStride;
  int* oidx = g.idx + (long)r * g.idx_rstride;
  if (!sel) {  // everything is selected: no exchange (every chunk of the row takes this branch); epoch advances
    if (FUSED && late) is_late_appends(ap, r, slot, ppos, late, redf);
    if (ch == 0) {
#pragma unroll 1
      for (int i = t; i < k; i += kIsThreads) oidx[i] = i < c ? i + g.offset : -1;
    }
    if (t == 0)
      __hip_atomic_store(rcnt + ch * kIsWordStride, (unsigned long long)epoch << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // ---- one-exchange selection.  Each chunk publishes the keys at or above a cut that keeps at least pub_m of its
  // valid positions (the cut falls between bins of the chunk's own key range: 4096 bins down from its largest key),
  // and the largest key it leaves out; then every chunk reads all published keys of the row.  Let LB be the largest
  // left-out key of any chunk and T the k-th largest published key: when T > LB and no published key ties with T
  // across the cut, the selection is exactly the keys >= T -- each chunk emits its own at the offset counted from
  // the earlier chunks' published keys, with no second exchange.  Otherwise (a chunk holding more of the selection
  // than it published, or a tie at T) every chunk of the row, reading the same published data, takes the same
  // decision and falls back to the histogram and candidate exchanges below.  Only keys above LB can reach the
  // selection on this path, so T is searched among them: 4096 bins over [LB, the largest key], then ranks in T's bin.
  if (g.pub_m > 0) {
    static_assert(kIsPer == 1, "one position per thread");
    DSV41_PX(10);
    const int pp = ch * kIsChunk + t;
    const bool valid = pp < c;
    const uint32_t kk = valid ? score_key(sc[t]) : 0u;
    const int nvalid = min(max(c - ch * kIsChunk, 0), kIsChunk);
    bool pubd = valid;
    if (nvalid > g.pub_m) {
      uint32_t mx = 0u, nmn = 0u;  // the largest key and the complement of the smallest (the scoring loop's)
#pragma unroll
      for (int w = 0; w < 8; ++w) mx = max(mx, ured[w]), nmn = max(nmn, ured[8 + w]);
      const int sh = bin_shift(mx - ~nmn);
      DSV41_PX(11);
      if (valid) atomicAdd(&lhist[(mx - kk) >> sh], 1);  // bin 0: the chunk's largest key (lhist is zero here)
      __syncthreads();
      bins_reach(lhist, g.pub_m, tmp, s_ro);
      DSV41_PX(12);
      pubd = valid && (int)((mx - kk) >> sh) <= s_ro[0];
    }
    const unsigned long long bal = __ballot(pubd);
    const int wo = __popcll(bal & ((1ull << lane) - 1));
    if (lane == 0) wcnt[wave][0] = __popcll(bal);
    uint32_t out_max = valid && !pubd ? kk : 0u, unused = 0u;
    block_umax2<kIsThreads>(out_max, unused, ured);  // (its barrier also publishes wcnt)
    int wbase = 0, npub = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      wbase += w < wave ? wcnt[w][0] : 0;
      npub += wcnt[w][0];
    }
    uint32_t* const lrow = g.lst + (long)r * ns * kIsLst;
    uint32_t* const mine = lrow + (long)ch * kIsLst;
    if (pubd) __hip_atomic_store(mine + 1 + wbase + wo, kk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == 0) __hip_atomic_store(mine, out_max, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    DSV41_PX(13);
    // the flag goes out after this workgroup's list has landed: a reader that sees this epoch finds the list
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned long long* const frow = g.fl + (long)r * ns * kIsWordStride;
    if (t == 0)
      __hip_atomic_store(frow + ch * kIsWordStride, (unsigned long long)epoch << 32 | (uint32_t)npub, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    DSV41_PH(2);
    DSV41_PX(14);
    if (FUSED && late) {  // (while the row's other chunks publish)
      is_late_appends(ap, r, slot, ppos, late, redf);
      late = 0;
    }
#pragma unroll
    for (int j = 0; j < kHistBins / kIsThreads; ++j) lhist[t + j * kIsThreads] = 0;  // (read after the barriers below)
    if (t == 0) s_m1 = 0, s_tie = 1;
    {  // the row barrier: every chunk's flag carries this epoch
      unsigned long long fv = 0ull;
#pragma unroll 1
      for (int spins = 0;; ++spins) {
        if (t < ns) fv = __hip_atomic_load(frow + t * kIsWordStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__syncthreads_and(t >= ns || (uint32_t)(fv >> 32) == epoch)) break;
        if (spins >= kIsSpinLimit) {
          if (t == 0) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (t < ns) na_q[t] = (int)(fv & 0xffffu);
    }
    DSV41_PH(3);
    DSV41_PX(15);
    const int nq = t < ns ? na_q[t] : 0;
    uint32_t nmax = (uint32_t)nq, unused2 = 0u;
    block_umax2<kIsThreads>(nmax, unused2, ured + 2 * kIsThreads / 64);  // (its barrier also publishes na_q)
    const int per = ((int)nmax + 4) & ~3, slots = ns * per;  // list slots read per chunk: entry 0 + nmax keys
    bool fast = slots <= kIsRd * kIsThreads;
    uint32_t T = 0u;
    uint32_t v[kIsRd];
    int vq[kIsRd / 4];  // chunk of v[4u .. 4u+3] (-1: none); list entry 0 is the chunk's largest left-out key
    int ve[kIsRd / 4];  // list entry of v[4u]
    bool key[kIsRd];    // v[u] is a published key above the largest left-out key
    if (fast) {
      // every published list, 16-byte device-scope loads all in flight together
      const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(lrow, 0, 0x7fffffff, 0x00020000);
#pragma unroll
      for (int u = 0; u < kIsRd / 4; ++u) {
        const int id = 4 * (u * kIsThreads + t), q = id / per, e = id - q * per;
        const is_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(lrs, id < slots ? (q * kIsLst + e) * 4 : 0, 0,
                                                                  kIsCpolDevice);
        v[4 * u] = x[0], v[4 * u + 1] = x[1], v[4 * u + 2] = x[2], v[4 * u + 3] = x[3];
        vq[u] = id < slots && e <= na_q[q] ? q : -1;
        ve[u] = e;
      }
      uint32_t lb = 0u, ux = 0u;
#pragma unroll
      for (int u = 0; u < kIsRd; ++u) {
        const int q = vq[u / 4], e = ve[u / 4] + (u & 3);
        key[u] = q >= 0 && e > 0 && e <= na_q[q];  // (above lb: refined below)
        if (q >= 0 && e == 0) lb = max(lb, v[u]);
        if (key[u]) ux = max(ux, v[u]);
      }
      block_umax2<kIsThreads>(lb, ux, ured);
      DSV41_PH(4);
      DSV41_PX(16);
      // T: the k-th largest key above lb
      const int sh = bin_shift(ux > lb ? ux - lb - 1 : 0u);
#pragma unroll
      for (int u = 0; u < kIsRd; ++u) {
        key[u] = key[u] && v[u] > lb;
        if (key[u]) atomicAdd(&lhist[(ux - v[u]) >> sh], 1);
      }
      __syncthreads();
      DSV41_PX(17);
      int above_lb;
      {
        int hv[8], local = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) hv[i] = lhist[8 * t + i], local += hv[i];
        int before = block_scan_dpp<kIsThreads>(local, tmp, &above_lb);
        if (before < k && k <= before + local) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (before < k && k <= before + hv[i]) {
              s_ro[0] = 8 * t + i;
              s_ro[1] = before;
            }
            before += hv[i];
          }
        }
      }
      fast = above_lb >= k;  // (uniform: the block total)
      __syncthreads();
      DSV41_PX(18);
      if (fast) {
        const int B = s_ro[0], need = k - s_ro[1], m1 = lhist[B];
        uint32_t* const lcu = (uint32_t*)lc;
#pragma unroll
        for (int u = 0; u < kIsRd; ++u)
          if (key[u] && (int)((ux - v[u]) >> sh) == B) lcu[atomicAdd(&s_m1, 1)] = v[u];
        __syncthreads();
        DSV41_PX(19);
#pragma unroll 1
        for (int i = t; i < m1; i += kIsThreads) {
          const uint32_t x = lcu[i];
          int gt = 0, ge = 0;
#pragma unroll 4
          for (int j = 0; j < m1; ++j) {
            const uint32_t y = lcu[j];
            gt += y > x;
            ge += y >= x;
          }
          if (gt < need && need <= ge) {  // (threads holding equal keys write the same values)
            s_T = x;
            s_tie = ge != need;
          }
        }
        __syncthreads();
        DSV41_PX(20);
        T = s_T;
        fast = !s_tie;
      }
    }
    DSV41_PH(5);
    if (fast) {
      // ---- ordered emission: this chunk's keys >= T after the earlier chunks' (their published keys >= T)
      int sb = 0;  // (T > lb: the keys >= T are published keys above lb)
#pragma unroll
      for (int u = 0; u < kIsRd; ++u) sb += key[u] && vq[u / 4] < ch && v[u] >= T;
      const bool take = valid && kk >= T;
      int2 tot2;
      const int2 ex2 = block_scan2_dpp<kIsThreads>(sb, (int)take, (int2*)ured, &tot2);
      DSV41_PX(21);
      if (take) oidx[tot2.x + ex2.y] = pp + g.offset;
      if (t == 0)  // (the next launch's epoch)
        __hip_atomic_store(rcnt + ch * kIsWordStride, (unsigned long long)epoch << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      DSV41_PH(7);
#ifdef DSV41_TIMING
      if (t == 0 && blockIdx.x < 1024) g_is_spins[blockIdx.x][1] = -1;  // took the one-exchange path
#endif
      return;
    }
    // fall back: this chunk's histogram of all its valid keys (a new key included), then the two exchanges
#pragma unroll
    for (int j = 0; j < kHistBins / kIsThreads; ++j) lhist[t + j * kIsThreads] = 0;
    __syncthreads();
    if (valid) atomicAdd(&lhist[kk >> 20], 1);
    __syncthreads();
  }
#pragma unroll 1
  for (int i = t; i < kHistBins / 2; i += kIsThreads) {  // bins in pairs: one 64-bit add (no carry out of a bin)
    const uint32_t lo = (uint32_t)lhist[2 * i], hi = (uint32_t)lhist[2 * i + 1];
    if (lo | hi) atomicAdd((unsigned long long*)(gh + 2 * i), ((unsigned long long)hi << 32) | lo);
  }
  if (FUSED && late) is_late_appends(ap, r, slot, ppos, late, redf);  // (while the row's other chunks add theirs)
  // ---- B. the row histogram once it holds all c valid positions (row barrier and data in one read), threshold bin
  DSV41_PH(2);
  if (t == 0) {
    s_bin = 0;  // (a histogram holding fewer than k entries is a caller error)
    s_need = k;
    s_cnt = 0;
  }
  {
    constexpr int BP = kHistBins / kIsThreads;  // bins per thread: 4095 - BP*t (h[0]) down to 4096 - BP*(t+1)
    int h[BP];
    int local, total, above, spins = 0;
#pragma unroll 1
    while (true) {
#pragma unroll
      for (int u = 0; u < BP / 2; ++u) {
        const unsigned long long v = __hip_atomic_load(
            (unsigned long long*)(gh + kHistBins - BP * (t + 1) + 2 * u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        h[BP - 1 - 2 * u] = (int)(v & 0xffffffffu);
        h[BP - 2 - 2 * u] = (int)(v >> 32);
      }
      local = 0;
#pragma unroll
      for (int i = 0; i < BP; ++i) local += h[i];
      above = block_scan_dpp<kIsThreads>(local, tmp, &total);  // (total is uniform over the workgroup)
      if (total == c) break;
      if (++spins >= kIsSpinLimit) {
        if (t == 0) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    DSV41_PH(3);
#ifdef DSV41_TIMING
    if (t == 0 && blockIdx.x < 1024) g_is_spins[blockIdx.x][0] = spins;
#endif
    if (above < k && k <= above + local) {
#pragma unroll 1
      for (int i = 0; i < BP; ++i) {
        if (k <= above + h[i]) {
          s_bin = kHistBins - 1 - BP * t - i;
          s_need = k - above;
          s_cnt = h[i];
          break;
        }
        above += h[i];
      }
    }
    __syncthreads();
  }
  const uint32_t lo = (uint32_t)s_bin << 20, hi = (uint32_t)(s_bin + 1) << 20;  // bin B = [lo, hi)
  const int need = s_need;
  // ---- C. classify this thread's positions
  const int p0 = ch * kIsChunk + kIsPer * t;
  uint32_t key[kIsPer];
  int na = 0, nc = 0;
#pragma unroll
  for (int e = 0; e < kIsPer; ++e) {
    key[e] = score_key(sc[kIsPer * t + e]);
    const bool ok = p0 + e < c;
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
  for (int w = 0; w < 8; ++w) cbase += w < wave ? wcnt[w][1] : 0;
  unsigned long long* crow = g.cand + (long)r * ns * kIsChunk;
  if (nc > 0) {
    int o = ch * kIsChunk + cbase + ic - nc;
#pragma unroll
    for (int e = 0; e < kIsPer; ++e)
      if (p0 + e < c && key[e] >= lo && key[e] < hi)
        __hip_atomic_store(crow + o++, is_cand_value(key[e], p0 + e, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // the counts go out after this workgroup's candidates have landed: a reader that sees this epoch in the count word
  // finds the candidates in place
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    unsigned ta = 0, tc = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) ta += wcnt[w][0], tc += wcnt[w][1];
    __hip_atomic_store(rcnt + ch * kIsWordStride, (unsigned long long)epoch << 32 | tc << 16 | ta, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- D. counts of all chunks + speculative candidate prefixes, read until every count word carries this epoch
  // and every speculative candidate below its chunk's count carries this epoch's tag (row barrier and gather in one)
  DSV41_PH(4);
  constexpr int kIsSpec = is_spec<MAXC>();
  constexpr int kSpecPer = MAXC * kIsSpec / kIsThreads;
  unsigned long long sv[kSpecPer];
  {
    int spins = 0;
#pragma unroll 1
    while (true) {
      unsigned long long cv = 0ull;
      if (t < ns) cv = __hip_atomic_load(rcnt + t * kIsWordStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < kSpecPer; ++u) {
        const int id = u * kIsThreads + t, q = id / kIsSpec, e = id % kIsSpec;
        sv[u] = q < ns ? __hip_atomic_load(crow + q * kIsChunk + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
      }
      if (t < ns) {
        na_q[t] = (int)(cv & 0xffffu);
        nc_q[t] = (int)((cv >> 16) & 0xffffu);
      }
      bool ok = t >= ns || (uint32_t)(cv >> 32) == epoch;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kSpecPer; ++u) {
        const int id = u * kIsThreads + t, q = id / kIsSpec, e = id % kIsSpec;
        if (q < ns && e < nc_q[q]) ok = ok && (uint32_t)(sv[u] >> kIsTagShift & ((1u << (32 - kIsTagShift)) - 1)) == tag;
      }
      if (__syncthreads_and(ok)) {
#ifdef DSV41_TIMING
        if (t == 0 && blockIdx.x < 1024) g_is_spins[blockIdx.x][1] = spins;
#endif
        break;
      }
      if (++spins >= kIsSpinLimit) {
        if (t == 0) __hip_atomic_store(g.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  DSV41_PH(5);
  {  // every chunk has read the histogram (its count word is out): clear this chunk's slice for the next launch
    const int zb = (kHistBins + ns - 1) / ns, z0 = ch * zb, z1 = min(kHistBins, z0 + zb);
#pragma unroll 1
    for (int i = z0 + t; i < z1; i += kIsThreads) gh[i] = 0;
  }
  if constexpr (MAXC <= 128) {
    if (wave < 2) {  // prefix of the candidate counts (2 x 64 chunks); entries above B in earlier chunks
      const int q = wave * 64 + lane;
      const int x = q < ns ? nc_q[q] : 0;
      const int ix = wave_incl_scan(x);
      pc[q + 1] = ix;  // (wave 1 adds wave 0's total below)
      const int y = q < ch ? na_q[q] : 0;
      const int iy = wave_incl_scan(y);
      if (lane == 63) wcnt[wave][0] = iy, wcnt[wave][1] = ix;
      const bool over = __ballot(x > kIsSpec) != 0;
      if (lane == 0) tmp[wave] = over;
    }
    __syncthreads();
    if (t >= 64 && t < 128) pc[t + 1] += wcnt[0][1];
    if (t == 0) {
      pc[0] = 0;
      s_selb = wcnt[0][0] + wcnt[1][0];
      s_over = tmp[0] | tmp[1];
    }
    __syncthreads();
  } else {  // one chunk per thread: workgroup scans
    const int x = t < ns ? nc_q[t] : 0;
    const int y = t < ch ? na_q[t] : 0;
    const int over = __syncthreads_or(x > kIsSpec);
    int tx, ty;
    const int ex = block_scan_dpp<kIsThreads>(x, tmp, &tx);
    block_scan_dpp<kIsThreads>(y, tmp, &ty);
    if (t < ns) pc[t + 1] = ex + x;
    if (t == 0) {
      pc[0] = 0;
      s_selb = ty;
      s_over = over;
    }
    __syncthreads();
  }
  const int m = pc[ns];
  const bool staged = m <= kIsCand;
  if (t == 0 && staged) lc[m] = 0ull;  // pad for pairwise reads
#pragma unroll
  for (int u = 0; u < kSpecPer; ++u) {
    const int id = u * kIsThreads + t, q = id / kIsSpec, e = id % kIsSpec;
    if (staged && q < ns && e < nc_q[q]) lc[pc[q] + e] = sv[u];
  }
  if (staged && s_over) {  // chunks with more than kIsSpec candidates: the rest, one candidate per thread
#pragma unroll 1
    for (int i = t; i < m; i += kIsThreads) {
      int lo = 0, hi = ns;  // the chunk q with pc[q] <= i < pc[q + 1]: the largest q with pc[q] <= i
#pragma unroll 1
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pc[mid] <= i) lo = mid;
        else hi = mid;
      }
      const int e = i - pc[lo];
      if (e >= kIsSpec)
        lc[i] = __hip_atomic_load(crow + lo * kIsChunk + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  auto cand_at = [&](int i) -> unsigned long long {
    if (staged) return lc[i];
    int q = 0;
    while (pc[q + 1] <= i) ++q;
    return __hip_atomic_load(crow + q * kIsChunk + (i - pc[q]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  DSV41_PH(6);
  const unsigned long long T = threshold_candidate<kIsThreads>(cand_at, lc, staged, m, need, lo, rs);
  int sb = 0;  // taken candidates of earlier chunks
#pragma unroll 1
  for (int i = t; i < pc[ch]; i += kIsThreads) sb += cand_at(i) >= T;
  int tot;
  block_scan_dpp<kIsThreads>(sb, tmp, &tot);
  const int base = s_selb + tot;
  // ---- F. ordered emission of this chunk
  bool take[kIsPer];
  int nt = 0;
#pragma unroll
  for (int e = 0; e < kIsPer; ++e) {
    const bool ok = p0 + e < c;
    take[e] = ok && (key[e] >= hi ||
                     (key[e] >= lo && is_cand_value(key[e], p0 + e, tag) >= T));
    nt += take[e];
  }
  int o = base + block_scan_dpp<kIsThreads>(nt, tmp, &tot);
#pragma unroll
  for (int e = 0; e < kIsPer; ++e)
    if (take[e]) oidx[o++] = p0 + e + g.offset;
  DSV41_PH(7);
}

int is_slots(int n_pos) { return (n_pos + kIsChunk - 1) / kIsChunk; }


// ------------------------------------------------------------------------------------------------ appends + scores
// The decode step's appends and the indexer scores with the row histogram in one launch, for rows longer than the
// one-launch selection takes (the selection follows as its own launches, dsv41_select_topk).  Score grid: chunks of
// 1024 positions, 16 waves x 64 keys (the layout of the long-row score kernel: chunk x of row r runs on XCD x mod 8),
// the row's e4m3 queries prepared in every workgroup (the first 512 threads, into LDS) while its keys are in flight.
// Before the score grid (dispatched first: a score workgroup holds a CU alone, so workgroups placed after a full
// score grid would wait for one to finish), 3 append-only workgroups per row: the ring row, the compressed row and
// the index key; for a
// row whose step closes a group the last one also scores the new key (position cl - 1: the same MFMA tile as the
// chunks', one valid column) and adds it to the row's histogram, and the chunk holding that position skips it (its
// table row is read before it is written).  The launch boundary orders all of it before the selection.
constexpr int kDsWaves = 16;  // (8-wave workgroups, two per CU: 21.2 against 16.8 us at C4)
constexpr int kDsThreads = 64 * kDsWaves;
constexpr int kDsChunk = kDsWaves * kKeysPerWave;

struct DsArgs {
  ScoreArgs s;  // e4m3 keys (ap.k8 / ap.ks), seq, cl, n_pos, out, hist, cand; q / w unused (prepared here)
  IsAppend app;
  int nx;       // score chunks per row
};

__global__ void __launch_bounds__(kDsThreads) decode_score_kernel(const DsArgs d) {
  const ScoreArgs& a = d.s;
  const IsAppend& ap = d.app;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int app_wgs = (3 * a.R + kXcds - 1) / kXcds * kXcds;  // (a multiple of 8: the score grid keeps its XCDs)
  __shared__ int lhist[kHistBins];
  __shared__ __align__(16) uint8_t qs[64 * 128];
  __shared__ float wfl[64];
  __shared__ __align__(16) uint8_t knew[128];
  __shared__ float ksnew, redf[kDsWaves];
  const int nht = (a.HI + 15) / 16;
  auto stage_queries = [&](int r, Qprep512& qp, bool load) {  // (threads < 512: head t / 8)
    if (t >= 512) return;
    if (load)
      qprep512_load(ap.q_idx + (long)r * a.HI * 128, ap.w_idx + (long)r * a.HI, a.HI, qp);
    else
      qprep512_store(qp, a.HI, qs, wfl);
  };
  auto read_queries = [&](i32x8_t (&qa8)[kHT], float (&wr)[kHT][4]) {
    float wl[kHT];
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      const int h = ht * 16 + l16;
      const int hc = ht < nht && h < a.HI ? h : 0;
      const uint4 u0 = *(const uint4*)(qs + hc * 128 + g * 32), u1 = *(const uint4*)(qs + hc * 128 + g * 32 + 16);
      qa8[ht] = i32x8_t{(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
      wl[ht] = ht < nht && h < a.HI ? wfl[h] : 0.0f;
    }
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[ht][i] = __shfl(wl[ht], 4 * g + i, 64);
  };
  uint4 qa16[kHT][4];  // (unused: e4m3 keys)
  if ((int)blockIdx.x < app_wgs) {  // ---- append-only workgroups: (row, which) = (e / 3, e % 3)
    const int e = (int)blockIdx.x, r = e / 3, which = e % 3;
    if (e >= 3 * a.R) return;
    DSV41_PH(6);
    const long slot = a.seq ? a.seq[r] : (long)(r / a.rows_per_slot);
    const long ppos = ap.pos[r];
    const bool closes = ((ppos + 1) % ap.ratio) == 0;
    if (which == 1 && !(ap.latent && ap.ckv)) return;
    if (which == 0) {  // (constant operation indices: the row operation's fields stay in registers)
      row_op<kDsThreads>(is_app_op(ap, r, slot, ppos, 0, nullptr, nullptr), redf);
      DSV41_PH(7);
      return;
    }
    if (which == 1) {
      row_op<kDsThreads>(is_app_op(ap, r, slot, ppos, 1, nullptr, nullptr), redf);
      DSV41_PH(7);
      return;
    }
    if (!closes) {
      row_op<kDsThreads>(is_app_op(ap, r, slot, ppos, 2, nullptr, nullptr), redf);
      DSV41_PH(7);
      return;
    }
    Qprep512 qp;
    stage_queries(r, qp, true);
    row_op<kDsThreads>(is_app_op(ap, r, slot, ppos, 2, knew, &ksnew), redf);  // the key, table and LDS copy
    stage_queries(r, qp, false);
    __syncthreads();
    if (wave == 0) {
      i32x8_t qa8[kHT];
      float wr[kHT][4];
      read_queries(qa8, wr);
      // column 0 of the tile holds the key (lanes with l16 = 0: bytes 32 g .. +32), the others zero
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 k0 = l16 == 0 ? *(const uint4*)(knew + g * 32) : z;
      const uint4 k1 = l16 == 0 ? *(const uint4*)(knew + g * 32 + 16) : z;
      const float sum = score_tile<1>(qa8, qa16, wr, nht, k0, k1, nullptr);
      long cl = row_cl(a, r);
      if (cl > a.n_pos) cl = a.n_pos;
      const long knew_row = (ppos + 1) / ap.ratio - 1;
      if (lane == 0 && knew_row >= 0 && knew_row < cl) {
        const float v = is_cand(a, r, knew_row) ? sum * ksnew : -__builtin_inff();
        a.out[(long)r * a.out_rstride + knew_row] = v;
        atomicAdd(a.hist + (long)r * kHistBins + (score_key(v) >> 20), 1);
      }
    }
    DSV41_PH(7);
    return;
  }
  // ---- score grid (block b on XCD b % 8; chunk x of every row on XCD x % 8)
  const int bxcd = (blockIdx.x - app_wgs) % kXcds, bj = (blockIdx.x - app_wgs) / kXcds;
  const int r = bj % a.R, bx = (bj / a.R) * kXcds + bxcd;
  if (bx >= d.nx) return;
  Qprep512 qp;
  stage_queries(r, qp, true);  // (first: in flight with the row data)
  long cl = row_cl(a, r);
  if (cl > a.n_pos) cl = a.n_pos;
  // Positions: chunk bx (its 16 waves x 4 tiles of 16), and past the d.nx chunks of the row one more tile per wave
  // (tile 64 nx + 16 bx + wave), so that a grid capped at the free CUs still covers the row.
  const long x0 = (64L * d.nx + 16 * bx) * 16;  // first position of this workgroup's extra tiles
  if ((long)bx * kDsChunk >= cl && x0 >= cl) return;
  const long slot = a.seq ? a.seq[r] : (long)(r / a.rows_per_slot);
  const long ppos = ap.pos[r];
  const long knew_row = ((ppos + 1) % ap.ratio) == 0 ? (ppos + 1) / ap.ratio - 1 : -1;  // (-1: no new key)
  DSV41_PH(0);
  static_assert(kHistBins % kDsThreads == 0, "histogram clear");
#pragma unroll
  for (int j = 0; j < kHistBins / kDsThreads; ++j) lhist[t + j * kDsThreads] = 0;  // (no loop between the loads)
  const int lim = (int)cl;
  const int kt0 = bx * kDsChunk + wave * kKeysPerWave;
  constexpr int NT = 5;  // 4 tiles of the chunk, the extra tile
  const bool extra = x0 + 16 * wave < cl;  // (wave-uniform)
  auto tile_pos = [&](int nt) { return nt < 4 ? kt0 + nt * 16 + l16 : (int)x0 + 16 * wave + l16; };
  uint4 k0[NT], k1[NT];
  float ksc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    // positions past the row load row 0 (unconditional loads: a select on a loaded value would make the compiler
    // wait for it before the later tiles' loads are issued); their scores are not recorded
    const int p = tile_pos(nt), pl = p < lim ? p : 0;
    if (nt == 4 && !extra) break;
    const uint8_t* krow = (const uint8_t*)a.keys + slot * a.k_sstride + (long)pl * 128 + g * 32;
    k0[nt] = *(const uint4*)krow;
    k1[nt] = *(const uint4*)(krow + 16);
    ksc[nt] = a.kscale[slot * a.ks_sstride + pl];
  }
  stage_queries(r, qp, false);
#ifdef DSV41_TIMING
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
  DSV41_PH(1);
  __syncthreads();  // queries staged, histogram cleared
  DSV41_PH(2);
  i32x8_t qa8[kHT];
  float wr[kHT][4];
  read_queries(qa8, wr);
  float* orow = a.out + (long)r * a.out_rstride;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (nt == 4 && !extra) break;
    const int p = tile_pos(nt);
    const float sum = score_tile<1>(qa8, qa16, wr, nht, k0[nt], k1[nt], nullptr);
    if (g == 0 && p < lim && p != knew_row) {  // (the new key's position is its append workgroup's)
      const float v = is_cand(a, r, p) ? sum * ksc[nt] : -__builtin_inff();
      orow[p] = v;
      atomicAdd(&lhist[score_key(v) >> 20], 1);
    }
  }
  DSV41_PH(3);
  __syncthreads();
  DSV41_PH(4);
  int* gh = a.hist + (long)r * kHistBins;
#pragma unroll 1
  for (int i = t; i < kHistBins / 2; i += kDsThreads) {  // bins in pairs: one 64-bit add (no carry out of a bin)
    const uint32_t lo = (uint32_t)lhist[2 * i], hi = (uint32_t)lhist[2 * i + 1];
    if (lo | hi) atomicAdd((unsigned long long*)(gh + 2 * i), ((unsigned long long)hi << 32) | lo);
  }
#ifdef DSV41_TIMING
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
  DSV41_PH(5);
}

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_spins_is(int* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_is_spins), sizeof(g_is_spins)); }
int dsv41_read_px_is(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_px), sizeof(g_dsv41_px)); }
int dsv41_read_ph_is(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ph), sizeof(g_dsv41_ph)); }
int dsv41_read_ts_is(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ts), sizeof(g_dsv41_ts)); }
#endif

long dsv41_index_select_workspace_bytes(int R, int n_pos) {
  const long ns = is_slots(n_pos);
  return (long)R * kHistBins * 4 + (long)R * ns * 8 * kIsWordStride + (long)R * ns * kIsChunk * 8 +
         (long)R * ns * 8 + (long)R * ns * 8 * kIsWordStride + 16 + (long)R * ns * kIsLst * 4 + 16;
}

}  // extern "C"

namespace {

// Shared set-up of dsv41_index_select / dsv41_decode_select (q8 / wf: prepared queries, or null when FUSED).
int select_setup(IsArgs& g, const void* q8, long q_rstride, const float* wf, long w_rstride, int R, int HI,
                 const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                 const long* cl, int n_pos, int k, int offset, void* ws, long ws_bytes, float* score_out,
                 long score_rstride, int* out, long out_rstride, const void* cand, long cand_rstride) {
  const int ns = is_slots(n_pos);
  if (n_pos <= 0 || HI <= 0 || HI > 64 || !cl || !kscale || ns > kIsMaxChunks || (long)R * ns > kIsMaxWG)
    return (int)hipErrorInvalidValue;
  if (!ws || ws_bytes < dsv41_index_select_workspace_bytes(R, n_pos)) return (int)hipErrorInvalidValue;
  if (((uintptr_t)ws & 7) != 0) return (int)hipErrorInvalidValue;  // 64-bit histogram / count atomics
  ScoreArgs& a = g.s;
  a.q = (const uint16_t*)q8;
  a.q_rstride = q_rstride;
  a.w = wf;
  a.w_rstride = w_rstride;
  a.HI = HI;
  a.R = R;
  a.kfmt = 1;
  a.keys = keys;
  a.k_sstride = k_sstride;
  a.kscale = kscale;
  a.ks_sstride = ks_sstride;
  a.seq = seq;
  a.rows_per_slot = 1;
  a.cl = cl;
  a.n_pos = n_pos;
  a.write_masked = 1;
  a.out = score_out;
  a.out_rstride = score_rstride;
  a.cand = (const uint8_t*)cand;
  a.cand_rstride = cand_rstride;
  g.k = k;
  g.offset = offset;
  g.idx = out;
  g.idx_rstride = out_rstride;
  g.nslots = ns;
  char* w = (char*)ws;
  g.hist = (int*)w;
  g.cnt = (unsigned long long*)(w + (long)R * kHistBins * 4);
  g.cand = g.cnt + (long)R * ns * kIsWordStride;
  g.fl = g.cand + (long)R * ns * kIsChunk + (long)R * ns;  // (after a spare [R, nslots] u64 region)
  g.lst = (uint32_t*)(((uintptr_t)(g.fl + (long)R * ns * kIsWordStride) + 15) & ~(uintptr_t)15);  // (16-byte reads)
  g.err = (int*)(w + dsv41_index_select_workspace_bytes(R, n_pos) - 16);
  // published keys per chunk on the one-exchange path: 1.5 times a chunk's share of k, plus 8 (a chunk holding
  // more of the selection than it published sends the row to the two-exchange path); DSV41_IS_PUB_M overrides it
  // (0: the two-exchange path only)
  g.pub_m = (int)min((long)kIsChunk, 3L * ((k + ns - 1) / ns) / 2 + 8);
  if (const char* e = getenv("DSV41_IS_PUB_M")) g.pub_m = atoi(e) < 0 ? 0 : min(atoi(e), kIsChunk);
  return 0;
}

template <bool FUSED>
int select_launch(const IsArgs& g, hipStream_t st) {
  const int grid = g.s.R * g.nslots;
  if (g.nslots <= 128)
    index_select_kernel<128, FUSED><<<grid, kIsThreads, 0, st>>>(g);
  else
    index_select_kernel<kIsMaxChunks, FUSED><<<grid, kIsThreads, 0, st>>>(g);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // namespace

namespace {
// Compute units of the current device (queried once per device; 256 when the query fails).
int ds_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cached[dev];
}
}  // namespace

extern "C" {

int dsv41_index_select(const void* q8, long q_rstride, const float* wf, long w_rstride, int R, int HI,
                       const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                       const long* cl, int n_pos, int k, int offset, void* ws, long ws_bytes, float* score_out,
                       long score_rstride, int* out, long out_rstride, const void* cand, long cand_rstride,
                       void* stream) {
  if (R <= 0 || k <= 0) return 0;
  IsArgs g{};
  const int e = select_setup(g, q8, q_rstride, wf, w_rstride, R, HI, keys, k_sstride, kscale, ks_sstride, seq, cl,
                             n_pos, k, offset, ws, ws_bytes, score_out, score_rstride, out, out_rstride, cand,
                             cand_rstride);
  return e ? e : select_launch<false>(g, (hipStream_t)stream);
}

int dsv41_decode_select(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                        const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                        const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                        long ks_sstride, int kcap, const long* pos, const long* seq, const long* nw_tab, int R,
                        int ratio, const float* cos_t, const float* sin_t, int rd, float eps, const void* q_idx,
                        const void* w_idx, int HI, const long* cl, int n_pos, int k, int offset, void* ws,
                        long ws_bytes, float* score_out, long score_rstride, int* out, long out_rstride,
                        const void* cand, long cand_rstride, void* stream) {
  if (R <= 0 || k <= 0) return 0;
  if (!row_ok(Dw, 32) || ratio <= 0 || rd < 0 || rd % 2 != 0 || rd > Dw || rd > 128 || W <= 0 || !kv_raw ||
      !kv_norm || !ring || !k_raw || !k_norm || !k8 || !ks || !pos || !seq || !q_idx || !w_idx || kcap <= 0 ||
      (latent && (!ckv || cap <= 0)) || (rd > 0 && (!cos_t || !sin_t)))
    return (int)hipErrorInvalidValue;
  IsArgs g{};
  const int e = select_setup(g, nullptr, 0, nullptr, 0, R, HI, k8, k8_sstride, ks, ks_sstride, seq, cl, n_pos, k,
                             offset, ws, ws_bytes, score_out, score_rstride, out, out_rstride, cand, cand_rstride);
  if (e) return e;
  g.app = IsAppend{(const uint16_t*)kv_raw, (const uint16_t*)kv_norm, (uint16_t*)ring, ring_sstride, W, Dw,
                   (const uint16_t*)latent, (uint16_t*)ckv, ckv_sstride, cap, (const uint16_t*)k_raw,
                   (const uint16_t*)k_norm, (uint16_t*)kbf, kbf_sstride, (uint8_t*)k8, k8_sstride, ks, ks_sstride,
                   kcap, pos, nw_tab, ratio, rd, cos_t, sin_t, eps, (const uint16_t*)q_idx, (const uint16_t*)w_idx};
  return select_launch<true>(g, (hipStream_t)stream);
}


int dsv41_decode_score(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                       const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                       const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                       long ks_sstride, int kcap, const long* pos, const long* seq, const long* nw_tab, int R,
                       int ratio, const float* cos_t, const float* sin_t, int rd, float eps, const void* q_idx,
                       const void* w_idx, int HI, const long* cl, int n_pos, float* score, long score_rstride,
                       int* hist, const void* cand, long cand_rstride, void* stream) {
  if (R <= 0 || n_pos <= 0) return 0;
  if (!row_ok(Dw, 32) || ratio <= 0 || rd < 0 || rd % 2 != 0 || rd > Dw || rd > 128 || W <= 0 || !kv_raw ||
      !kv_norm || !ring || !k_raw || !k_norm || !k8 || !ks || !pos || !seq || !q_idx || !w_idx || kcap <= 0 ||
      (latent && (!ckv || cap <= 0)) || (rd > 0 && (!cos_t || !sin_t)) || !cl || !score || !hist || HI <= 0 ||
      HI > 64 || n_pos > kcap || ((uintptr_t)hist & 7) != 0)
    return (int)hipErrorInvalidValue;
  DsArgs d{};
  ScoreArgs& a = d.s;
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
  a.out = score;
  a.out_rstride = score_rstride;
  a.hist = hist;
  a.cand = (const uint8_t*)cand;
  a.cand_rstride = cand_rstride;
  d.app = IsAppend{(const uint16_t*)kv_raw, (const uint16_t*)kv_norm, (uint16_t*)ring, ring_sstride, W, Dw,
                   (const uint16_t*)latent, (uint16_t*)ckv, ckv_sstride, cap, (const uint16_t*)k_raw,
                   (const uint16_t*)k_norm, (uint16_t*)kbf, kbf_sstride, (uint8_t*)k8, k8_sstride, ks, ks_sstride,
                   kcap, pos, nw_tab, ratio, rd, cos_t, sin_t, eps, (const uint16_t*)q_idx, (const uint16_t*)w_idx};
  // chunks per row: the row's chunks rounded up to a multiple of 8, or, when that overfills the CUs the append
  // workgroups leave, as many as fit (a multiple of 8 again) provided one extra tile per wave covers the rest
  const int app_wgs = (3 * R + kXcds - 1) / kXcds * kXcds;
  int nx = (n_pos + kDsChunk - 1) / kDsChunk;
  nx = (nx + kXcds - 1) / kXcds * kXcds;
  const int fit = (ds_cus() - app_wgs) / R / kXcds * kXcds;
  if (fit >= kXcds && nx > fit && (64L * fit + 16L * fit) * 16 >= n_pos) nx = fit;
  d.nx = nx;
  const int grid = app_wgs + nx * R;
  decode_score_kernel<<<grid, kDsThreads, 0, (hipStream_t)stream>>>(d);
  DSV41_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
