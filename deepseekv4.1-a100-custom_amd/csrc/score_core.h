// Score tile of the lightning indexer (shared by the score kernels): arguments, the per-row valid count and one
// 16-key column tile against all head tiles.  See indexer.hip for the kernels.
#pragma once
#include "common.h"

namespace {

struct ScoreArgs {
  const uint16_t* q;  // bf16 [R, HI, 128] (bf16 keys) or prepared e4m3 [R, 64, 128] bytes (e4m3 keys)
  long q_rstride;     // elements (bf16) or bytes (e4m3) between rows
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
  int* hist;  // optional [R, kHistBins]: counts of score_key(score) >> 20 over t < cl (decode selection)
  const uint8_t* cand;  // optional candidate mask [R, >= n_pos] (nonzero = candidate): other t < cl score -inf
  long cand_rstride;
};

// Candidate mask of position t of row r (true when no mask is given).
DSV41_DEV bool is_cand(const ScoreArgs& a, int r, long t) { return !a.cand || a.cand[(long)r * a.cand_rstride + t]; }

DSV41_DEV long row_cl(const ScoreArgs& a, int r) {
  if (a.cl) return a.cl[r];
  return (a.cl_start + (long)(r % a.rows_per_slot) + 1) / a.cl_ratio;
}

constexpr int kHT = 4;            // head tiles of 16 (up to 64 indexer heads)
constexpr int kHistBins = 4096;   // top 12 bits of the order-preserving score key (8 bins per octave)
constexpr int kKeysPerWave = 64;   // 4 column tiles of 16 keys (two or more waves per SIMD)
constexpr int kKeysPerWG = 4 * kKeysPerWave;

// One column tile (16 keys) against all head tiles; returns this lane's partial weighted relu sum for key l16.
// Every head tile is computed (unused ones carry weight 0), so the MFMAs issue back to back.
template <int KFMT>
DSV41_DEV float score_tile(const i32x8_t (&qa8)[kHT], const uint4 (&qa16)[kHT][4], const float (&wr)[kHT][4],
                           int nht, uint4 k0, uint4 k1, const uint4* kb16) {
  f32x4_t acc[kHT];
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) acc[ht] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (KFMT == 1) {
    const i32x8_t kb = i32x8_t{(int)k0.x, (int)k0.y, (int)k0.z, (int)k0.w, (int)k1.x, (int)k1.y, (int)k1.z, (int)k1.w};
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) acc[ht] = mfma_fp8_16x16x128(qa8[ht], kb, acc[ht]);
  } else {
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc[ht] = mfma_bf16_16x16x32(qa16[ht][ks], kb16[ks], acc[ht]);
  }
  (void)nht;  // head tiles past the head count hold a valid query row with weight 0: no branches around the MFMAs
  float part[kHT];  // one chain per head tile (four short dependent chains instead of one of 16)
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    part[ht] = wr[ht][0] * relu(acc[ht][0]);
#pragma unroll
    for (int i = 1; i < 4; ++i) part[ht] += wr[ht][i] * relu(acc[ht][i]);
  }
  static_assert(kHT == 4, "head tiles");
  float sum = (part[0] + part[1]) + (part[2] + part[3]);
  sum = row_sum4(sum);
  return sum;
}

}  // namespace
