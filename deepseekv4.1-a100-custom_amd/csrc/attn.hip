// Sparse latent attention over gathered KV rows, with a per-head sink in the softmax denominator.
//
// One kernel family serves every attention entry point of the path:
//   dsv41_sparse_attn   kernels.sparse_attn / fused.sparse_attn_decode  (explicit index list into one KV tensor)
//   dsv41_sparse_attn2  fused.sparse_attn_decode2 / _split              (index < n1 -> kv1, else kv2[index - n1])
//   dsv41_sattn2        fused2.sattn2                                    (SWA ring with position validity, then
//                                                                         compressed rows by index; inverse rope)
//
// Work decomposition (gfx950, wave64): a workgroup of 4 waves owns one query row, 64 heads (wave w: heads
// 16w..16w+15) and a contiguous chunk of that row's key list ("split").  Key rows are gathered 32 at a time into
// LDS with 16-byte loads (invalid rows are zero-filled), shared by the 4 waves.  Per wave and tile:
//   S^T[32 rows x 16 heads] = K * Q^T  -- 16x16x32 bf16 MFMA, A = K from LDS, B = Q held in VGPRs for the whole loop
//   online softmax per head (fp32; max/sum across the 4 lane groups by shuffles)
//   O[16 heads x DV] += P * V          -- the S^T accumulator of a lane already is the P operand (head = lane & 15,
//                                         8 key rows), so P never leaves registers; V is read from the same LDS tile.
// Several splits per row write fp32 partials (m, l, acc); a combine kernel merges them with the sink and applies
// the inverse rope (dsv41/fused2.py:381-403).  A single split writes the final bf16 output directly.
#include <mutex>
#include <type_traits>

#include "attn_core.h"

namespace {



template <int DQK, int DV>
__global__ void __launch_bounds__(256) attn_split_kernel(const AttnArgs a) {
  constexpr int KS = DQK / 32;   // MFMA k-steps over the QK width
  constexpr int CT = DV / 16;    // 16-wide output column tiles
  constexpr int RSTR = DQK + 8;  // LDS row stride in elements (16 B pad)
  constexpr int U = DQK / 8;     // 16-byte units per row
  __shared__ __align__(16) uint16_t ktile[32 * RSTR];
  __shared__ const uint16_t* rptr[32];

  const int sp = blockIdx.x, hb = blockIdx.y, r = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int h0 = hb * 64 + wave * 16;
  const int H = a.H;

  uint4 qf[KS];
  {
    const int h = h0 + l16;
    const uint16_t* qrow = a.q + (long)r * a.q_rstride + (long)h * DQK;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[ks] = h < H ? *(const uint4*)(qrow + ks * 32 + g * 8) : make_uint4(0, 0, 0, 0);
  }

  long slot, pos = 0, pmax = 0, plim = 0;
  const int W = a.n1;
  if (a.mode == 1) {
    slot = a.seq[r];
    pos = a.pos[r];
    pmax = a.pmax[r];
    plim = a.plim ? a.plim[r] : pos;
  } else {
    slot = r / a.rows_per_slot;
  }
  const uint16_t* base1 = a.kv1 + slot * a.kv1_sstride;
  const uint16_t* base2 = a.kv2 ? a.kv2 + slot * a.kv2_sstride : nullptr;
  const int* irow = a.t > 0 ? a.idx + (long)r * a.idx_rstride : nullptr;

  float m_run = -1e30f, l_run = 0.0f;
  f32x4_t o[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) o[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int j0 = sp * a.chunk;
  const int j1 = min(a.L, j0 + a.chunk);
  for (int jt = j0; jt < j1; jt += 32) {
    if (tid < 32) {
      const int j = jt + tid;
      const uint16_t* p = nullptr;
      if (j < j1) {
        if (a.mode == 1 && j < W) {
          int m = (int)(pmax - j) % W;  // positions fit in 31 bits
          m = m < 0 ? m + W : m;
          const long held = pmax - m;
          if (held >= 0 && held <= plim && pos - held < W) p = base1 + (long)j * DQK;
        } else {
          const int ix = irow[a.mode == 1 ? j - W : j];
          if (a.mode == 1) {
            if (ix >= 0 && ix < a.n2) p = base2 + (long)ix * DQK;
          } else if (ix >= 0 && ix < a.n1 + a.n2) {
            p = ix < a.n1 ? base1 + (long)ix * DQK : base2 + (long)(ix - a.n1) * DQK;
          }
        }
      }
      rptr[tid] = p;
    }
    __syncthreads();
    for (int e = tid; e < 32 * U; e += 256) {
      const int row = e / U, c = e - row * U;
      const uint16_t* p = rptr[row];
      const uint4 v = p ? *(const uint4*)(p + c * 8) : make_uint4(0, 0, 0, 0);
      *(uint4*)(ktile + row * RSTR + c * 8) = v;
    }
    __syncthreads();

    f32x4_t s[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      s[rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      const uint16_t* krow = ktile + (rt * 16 + l16) * RSTR + g * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s[rt] = mfma_bf16_16x16x32(*(const uint4*)(krow + ks * 32), qf[ks], s[rt]);
    }
    // s[rt][i] = score of key row rt*16 + 4g + i for head h0 + l16
    float p[8];
    float tmax = -1e30f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = (e >> 2) * 16 + 4 * g + (e & 3);
      const float x = rptr[row] ? s[e >> 2][e & 3] * a.scale : -1e30f;
      p[e] = x;
      tmax = fmaxf(tmax, x);
    }
    tmax = row_max4(tmax);
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f((m_run - m_new) * kLog2e);
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = (e >> 2) * 16 + 4 * g + (e & 3);
      p[e] = rptr[row] ? exp2f((p[e] - m_new) * kLog2e) : 0.0f;
      psum += p[e];
    }
    psum = row_sum4(psum);
    l_run = alpha * l_run + psum;
    m_run = m_new;

    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
    const uint4 pa = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                pack_bf16x2(p[6], p[7]));
    const uint16_t* vrow[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vrow[e] = ktile + ((e >> 2) * 16 + 4 * g + (e & 3)) * RSTR + l16;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[ct][i] *= al[i];
      const uint4 vb = make_uint4((uint32_t)vrow[0][ct * 16] | ((uint32_t)vrow[1][ct * 16] << 16),
                                  (uint32_t)vrow[2][ct * 16] | ((uint32_t)vrow[3][ct * 16] << 16),
                                  (uint32_t)vrow[4][ct * 16] | ((uint32_t)vrow[5][ct * 16] << 16),
                                  (uint32_t)vrow[6][ct * 16] | ((uint32_t)vrow[7][ct * 16] << 16));
      o[ct] = mfma_bf16_16x16x32(pa, vb, o[ct]);
    }
    __syncthreads();
  }

  if (a.nsplit == 1) {
    const int hl = h0 + l16;
    const float den = l_run + exp2f(((hl < H ? a.sink[hl] : 0.0f) - m_run) * kLog2e);
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) inv[i] = 1.0f / __shfl(den, 4 * g + i, 64);
    long pr = pos < 0 ? 0 : pos;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c = ct * 16 + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = round_bf16(o[ct][i] * inv[i]);
        const float partner = dpp_mov<0xB1>(v);  // lane ^ 1
        if (a.rd > 0 && c >= DV - a.rd) {
          const int jj = (c - (DV - a.rd)) >> 1;
          const float cs = a.cos_t[pr * (a.rd / 2) + jj];
          const float sn = -a.sin_t[pr * (a.rd / 2) + jj];
          v = (c & 1) ? (partner * sn + v * cs) : (v * cs - partner * sn);
        }
        const int h = h0 + 4 * g + i;
        if (h < H) a.out[(long)r * a.out_rstride + (long)h * DV + c] = f2bf(v);
      }
    }
  } else {
    const int hl = h0 + l16;
    if (g == 0 && hl < H) {
      const long pi = ((long)r * H + hl) * a.nsplit + sp;
      a.pm[pi] = m_run;
      a.pl[pi] = l_run;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = h0 + 4 * g + i;
      if (h >= H) continue;
      float* dst = a.pacc + (((long)r * H + h) * a.nsplit + sp) * DV;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) dst[ct * 16 + l16] = o[ct][i];
    }
  }
}

// Merge the splits of one (row, head): LSE combine + sink, bf16 round, inverse rope on the last rd columns.
template <int DV>
__global__ void __launch_bounds__(256) attn_combine_kernel(const AttnArgs a) {
  const int h = blockIdx.x, r = blockIdx.y;
  const int H = a.H, ns = a.nsplit;
  const long base = ((long)r * H + h) * ns;
  float mx = -1e30f;
  for (int s = 0; s < ns; ++s) mx = fmaxf(mx, a.pm[base + s]);
  float den = exp2f((a.sink[h] - mx) * kLog2e);
  for (int s = 0; s < ns; ++s) den += a.pl[base + s] * exp2f((a.pm[base + s] - mx) * kLog2e);
  const long pr = (a.mode == 1 && a.pos) ? (a.pos[r] < 0 ? 0 : a.pos[r]) : 0;
  for (int c = 2 * threadIdx.x; c < DV; c += 512) {
    float n0 = 0.0f, n1 = 0.0f;
    for (int s = 0; s < ns; ++s) {
      const float w = exp2f((a.pm[base + s] - mx) * kLog2e);
      const float2 v = *(const float2*)(a.pacc + (base + s) * DV + c);
      n0 += v.x * w;
      n1 += v.y * w;
    }
    float re = round_bf16(n0 / den), im = round_bf16(n1 / den);
    if (a.rd > 0 && c >= DV - a.rd) {
      const int jj = (c - (DV - a.rd)) >> 1;
      const float cs = a.cos_t[pr * (a.rd / 2) + jj];
      const float sn = -a.sin_t[pr * (a.rd / 2) + jj];
      const float yr = re * cs - im * sn, yi = re * sn + im * cs;
      re = yr;
      im = yi;
    }
    uint16_t* dst = a.out + (long)r * a.out_rstride + (long)h * DV + c;
    dst[0] = f2bf(re);
    dst[1] = f2bf(im);
  }
}

// ------------------------------------------------------------------------------------------------ decode kernel
// Few query rows (decode): the key list of a row is split across many workgroups, so each workgroup owns only 16
// heads (its partial output is 16 x DV) and the 4 waves of a workgroup split every 64-key tile 16 rows each.  Each
// wave keeps its own online-softmax state; the 4 states are merged through LDS at the end.  Partials are stored
// normalised (acc / l) in bf16 next to fp32 (m, l), which halves the partial traffic at an error far below bf16
// output rounding.



// Merge the split partials of heads h0..h0+15 of row r (512 threads, nsplit <= 32): weights w_s = l_s e^(m_s - M)
// normalised by sum_s w_s + e^(sink - M), then out = sum_s w_s o_s (o_s bf16-normalised), bf16 round, inverse rope
// on the last rd columns.
template <int DV>
DSV41_DEV void merge_splits(const AttnArgs& a, int r, int h0, long pr, float (*wts)[33]) {
  const int tid = threadIdx.x, H = a.H, ns = a.nsplit;
  {
    const int hh = tid >> 5, sp = tid & 31, h = h0 + hh;
    const bool ok = h < H && sp < ns;
    const long pi = ((long)r * H + h) * ns + sp;
    // pm/pl lines can hold entries of other units: agent-scope loads do not use the CU cache
    const float m = ok ? __hip_atomic_load(a.pm + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -1e30f;
    const float l = ok ? __hip_atomic_load(a.pl + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    const float M = group_max(m, 32);  // over the head's 32 split lanes (DPP moves and a row swap)
    const float w = ok ? l * exp2f((m - M) * kLog2e) : 0.0f;
    const float w16 = row16_sum(w);
    const auto hs = __builtin_amdgcn_permlane16_swap(__float_as_uint(w16), __float_as_uint(w16), false, false);
    float den = __uint_as_float(hs[0]) + __uint_as_float(hs[1]);  // the 32-lane sum
    den += exp2f((a.sink[h < H ? h : H - 1] - M) * kLog2e);
    wts[hh][sp] = w / den;
  }
  __syncthreads();
  const uint16_t* pb = (const uint16_t*)a.pacc;
  constexpr int CG = DV / 8;  // 8-column groups per head
#pragma unroll 1
  for (int e = tid; e < 16 * CG; e += 512) {
    const int hh = e / CG, c = (e - hh * CG) * 8, h = h0 + hh;
    if (h >= H) continue;
    const long base = ((long)r * H + h) * ns;
    float num[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll 1
    for (int s0 = 0; s0 < ns; s0 += 8) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *(const uint4*)(pb + (base + min(s0 + u, ns - 1)) * DV + c);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float wg = s0 + u < ns ? wts[hh][s0 + u] : 0.0f;
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          num[2 * q] += wg * __uint_as_float(vv[q] << 16);
          num[2 * q + 1] += wg * __uint_as_float(vv[q] & 0xffff0000u);
        }
      }
    }
    uint32_t pk[4];
#pragma unroll
    for (int q = 0; q < 8; q += 2) {
      float re = round_bf16(num[q]), im = round_bf16(num[q + 1]);
      const int cc = c + q;
      if (a.rd > 0 && cc >= DV - a.rd) {
        const int jj = (cc - (DV - a.rd)) >> 1;
        const float cs = a.cos_t[pr * (a.rd / 2) + jj];
        const float sn = -a.sin_t[pr * (a.rd / 2) + jj];
        const float yr = re * cs - im * sn, yi = re * sn + im * cs;
        re = yr;
        im = yi;
      }
      pk[q / 2] = pack_bf16x2(re, im);
    }
    *(uint4*)(a.out + (long)r * a.out_rstride + (long)h * DV + c) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
}


constexpr int kCoopSpinLimit = 1 << 20;
// The cooperative merge's arrival counters (u64) lie 128 bytes apart: device-scope atomics on one cache line
// serialise at the memory side (a unit's ~17 arrivals and polls then also wait for the other units').
constexpr int kCoopStride = 16;

// Decode attention, 8 waves per workgroup (2 per SIMD): wave w handles key rows 16*(w&3)..+15 of every 64-key tile
// and output columns [(w>>2)*DV/2, +DV/2) (QK^T and the softmax are computed by both column halves, identically).
// The softmax keeps a reference maximum per head and rescales the accumulators only when the tile maximum exceeds
// it by more than kRescale (log2 units): p = 2^(s*log2e - m_ref) <= 2^kRescale stays far from fp32/bf16 range
// limits, and the final normalisation uses the same reference, so the result is the exact softmax.
template <int DQK, int DV>
__global__ void __launch_bounds__(512) attn_decode_kernel(const AttnArgs a) {
  DSV41_WG_TS(0);
  constexpr int KS = DQK / 32;
  constexpr int CTH = DV / 32;  // 16-column output tiles per wave (half of DV)
  constexpr int U = DQK / 8;    // 16-byte chunks per row; chunk c of row j stored at j*U + (c ^ (j & 7))
  static_assert(U % 8 == 0, "row width must be a multiple of 64 elements");
  constexpr int TILE = 64;
  constexpr int TILE_ELEMS = TILE * DQK;
  constexpr int kLoadsPerTile = TILE * U / 512;  // 16-byte direct-to-LDS loads per wave per tile
  static_assert(kLoadsPerTile < 16, "vmcnt immediate");
  static_assert(16 * DQK / 8 % 64 == 0 && 16 * DQK <= TILE_ELEMS, "Q staging");
  constexpr float kRescale = 8.0f;
  constexpr int KT_ELEMS = 2 * TILE_ELEMS > 4 * 16 * (DV + 4) * 2 ? 2 * TILE_ELEMS : 4 * 16 * (DV + 4) * 2;
  __shared__ __align__(16) uint16_t ktile[KT_ELEMS];  // two tile buffers; the merge buffer aliases them
  __shared__ const uint16_t* rptr[3][TILE];            // resolved row pointers of tiles i, i+1, i+2 (null: invalid)
  __shared__ float wm[4][16], wl[4][16], wf[4][16], hM[16], hL[16];
  constexpr int kIxPre = 512;  // index entries prefetched (8 tiles); later tiles load theirs when resolved
  __shared__ int ixs[kIxPre];

  DSV41_TS(10);
  DSV41_PH(0);
  int sp, hg, r, home = -1;
  if (a.coop && a.hg_share) {
    // cooperative merge (device-scope, any placement): the head groups of one (row, split) share an XCD, so the
    // rows they all gather come from one L2
    const int HG = (a.H + 15) / 16;
    const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
    const int grp = x + kXcds * (j / HG);
    if (grp >= a.R * a.nsplit) return;
    hg = j % HG;
    r = grp / a.nsplit;
    sp = grp % a.nsplit;
    if (hg * 16 >= a.H) return;
  } else if (a.arrive) {  // the nsplit workgroups of a unit share XCD `home` and merge through its L2
    const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
    const int unit = x * a.upx + j / a.nsplit;
    if (unit >= a.units) return;
    const int HG = (a.H + 15) / 16;
    sp = j % a.nsplit;
    hg = unit % HG;
    r = unit / HG;
    home = x;
  } else {
    sp = blockIdx.x;
    hg = blockIdx.y;
    r = blockIdx.z;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rw = wave & 3, half = wave >> 2;
  const int l16 = lane & 15, g = lane >> 4;
  const int h0 = hg * 16;
  const int H = a.H;

  // the index rows of the first two tiles and Q are loaded before the row's position data (independent loads)
  const int W = a.n1;
  const int* irow = a.t > 0 ? a.idx + (long)r * a.idx_rstride : nullptr;
  const int all_tiles = (a.L + TILE - 1) / TILE;  // split sp takes tiles [sp*T/ns, (sp+1)*T/ns)
  const int j0 = (int)((long)sp * all_tiles / a.nsplit) * TILE;
  const int j1 = min(a.L, (int)((long)(sp + 1) * all_tiles / a.nsplit) * TILE);
  const int ntiles = (j1 - j0 + TILE - 1) / TILE;
  auto load_ix = [&](int jo) {  // index-list entry of key position j0 + jo (or -1)
    const int j = j0 + jo;
    const int jj = a.mode == 1 ? j - W : j;
    return j < j1 && jj >= 0 && irow ? irow[jj] : -1;
  };
  ixs[tid] = load_ix(tid);  // the first kIxPre entries of the split, kept in LDS
  // Q of the 16 heads (16 x DQK bf16, rows of missing heads repeat the last head and are never written) is staged
  // once through the second tile buffer with direct-to-LDS loads; every wave then reads its fragments from LDS (the
  // 8 waves each loading all of Q would pull 8x the bytes through the CU while every CU starts at once)
  uint16_t* const qlds = ktile + TILE_ELEMS;
  {
    constexpr int QCH = 16 * DQK / 8;  // 16-byte chunks
    constexpr int PR = DQK / 8;        // chunks per head row
#pragma unroll
    for (int u = 0; u < (QCH + 511) / 512; ++u) {
      const int cid = u * 512 + wave * 64 + lane;
      if (u * 512 + wave * 64 < QCH) {  // wave-uniform: a whole wave's chunks lie inside Q (QCH % 64 == 0)
        const int hh = cid / PR, part = cid - hh * PR;
        const int h = h0 + hh < H ? h0 + hh : H - 1;
        lds_dma16(a.q + (long)r * a.q_rstride + (long)h * DQK + part * 8, qlds + (u * 512 + wave * 64) * 8);
      }
    }
  }
  long slot, pos = 0, pmax = 0, plim = 0;
  if (a.mode == 1) {
    slot = a.seq[r];
    pos = a.pos[r];
    pmax = a.pmax[r];
    plim = a.plim ? a.plim[r] : pos;
  } else {
    slot = r / a.rows_per_slot;
  }
  const uint16_t* base1 = a.kv1 + slot * a.kv1_sstride;
  const uint16_t* base2 = a.kv2 ? a.kv2 + slot * a.kv2_sstride : nullptr;

  auto resolve = [&](int ti) {  // threads 0..63: row pointer of key position j0 + ti*TILE + tid
    if (tid < TILE) {
      const int jo = ti * TILE + tid;
      const int ix = jo < kIxPre ? ixs[jo] : load_ix(jo);
      const int j = j0 + jo;
      const uint16_t* p = nullptr;
      if (j < j1) {
        if (a.mode == 1 && j < W) {
          int m = (int)(pmax - j) % W;  // positions fit in 31 bits
          m = m < 0 ? m + W : m;
          const long held = pmax - m;
          if (held >= 0 && held <= plim && pos - held < W) p = base1 + (long)j * DQK;
        } else {
          if (a.mode == 1) {
            if (ix >= 0 && ix < a.n2) p = base2 + (long)ix * DQK;
          } else if (ix >= 0 && ix < a.n1 + a.n2) {
            p = ix < a.n1 ? base1 + (long)ix * DQK : base2 + (long)(ix - a.n1) * DQK;
          }
        }
      }
      rptr[ti % 3][tid] = p;
    }
  };
  auto issue = [&](int ti) {  // direct-to-LDS 16-byte loads (inline assembly: no compiler waits around them)
    uint16_t* buf = ktile + (ti & 1) * TILE_ELEMS;
    const uint16_t* const* rp = rptr[ti % 3];
    const uint16_t* src[kLoadsPerTile];  // all row pointers read before the first load (the loads clobber memory)
#pragma unroll
    for (int rd = 0; rd < kLoadsPerTile; ++rd) {
      const int q = rd * 512 + wave * 64 + lane;  // LDS chunk position
      const int j = q / U, cs = q - j * U;
      const int c = cs ^ (j & 7);
      const uint16_t* p = rp[j];
      src[rd] = p ? p + c * 8 : g_zero_row;
    }
#pragma unroll
    for (int rd = 0; rd < kLoadsPerTile; ++rd) lds_dma16(src[rd], buf + (rd * 512 + wave * 64) * 8);
  };

  __builtin_amdgcn_s_waitcnt(0);  // Q has arrived too: no wait for it is left inside the tile loop
  DSV41_PH(1);
  __syncthreads();
  uint4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const uint4*)(qlds + l16 * DQK + ks * 32 + g * 8);
  if (ntiles > 0) resolve(0);
  if (ntiles > 1) resolve(1);
  __syncthreads();  // (Q has been read: its buffer takes tile 1)
  DSV41_TS(11);
  DSV41_PH(2);
  if (ntiles > 0) issue(0);
  if (ntiles > 1) issue(1);

  float m_ref = -1e30f, l_run = 0.0f;  // per head (lane's head l16), log2 units
  f32x4_t o[CTH];
#pragma unroll
  for (int c = 0; c < CTH; ++c) o[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const float sl2 = a.scale * kLog2e;

  for (int ti = 0; ti < ntiles; ++ti) {
    // tile ti is complete once at most one tile's loads of this wave remain (loads complete in order)
    if (ti + 1 < ntiles)
      __builtin_amdgcn_s_waitcnt(kLoadsPerTile | (0x7 << 4) | (0xf << 8));  // vmcnt(kLoadsPerTile)
    else
      __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    DSV41_TS(12 + 2 * (ti & 3));
    const uint16_t* buf = ktile + (ti & 1) * TILE_ELEMS;
    const uint16_t* const* rp = rptr[ti % 3];
    const int rb = rw * 16;  // this wave's 16 key rows of the tile
    f32x4_t s = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    {
      const int j = rb + l16;
      const uint16_t* krow = buf + j * DQK;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        s = mfma_bf16_16x16x32(*(const uint4*)(krow + (((ks * 4 + g) ^ (j & 7)) * 8)), qf[ks], s);
    }
    // s[i] = score of key row rb + 4g + i for head h0 + l16
    float x[4];
    float tmax = -1e30f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = rp[rb + 4 * g + i] ? s[i] * sl2 : -1e30f;
      tmax = fmaxf(tmax, x[i]);
    }
    tmax = row_max4(tmax);
    const bool bump = tmax > m_ref + kRescale;
    if (__ballot(bump)) {  // wave-uniform: some head of this wave needs a new reference
      const float m_new = bump ? tmax : m_ref;
      const float alpha = exp2f(m_ref - m_new);
      l_run *= alpha;
      m_ref = m_new;
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[ct][i] *= al[i];
    }
    float psum = 0.0f;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = rp[rb + 4 * g + i] ? exp2f(x[i] - m_ref) : 0.0f;
      psum += p[i];
    }
    psum = row_sum4(psum);
    l_run += psum;
    const uint2 pa = make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
    // V operand: lane (column l16 of the 16-column tile, rows rb + 4g .. +3) via the transpose read: input lane
    // j of the 16-lane group reads row rb + 4g + j/4, columns 4*(j%4)..+3 of the tile
    const int vj = rb + 4 * g + (l16 >> 2);
    const uint16_t* vrow = buf + vj * DQK + ((l16 & 1) << 2);
    const int vsw = vj & 7;
#pragma unroll
    for (int ct = 0; ct < CTH; ++ct) {
      const int cch = ((half * (DV / 2) + ct * 16) >> 3) + ((l16 & 3) >> 1);  // chunk of column col0 + 4*(l16&3)
      const uint2 vb = lds_read_tr16(vrow + ((cch ^ vsw) << 3));
      o[ct] = mfma_bf16_16x16x16(pa, vb, o[ct]);
    }
    DSV41_TS(13 + 2 * (ti & 3));
    if (ti + 2 < ntiles) {
      resolve(ti + 2);
      lds_barrier();  // buffer ti & 1 is free, the pointers of tile ti + 2 are visible
      issue(ti + 2);
    }
  }
  __syncthreads();
  DSV41_TS(20);
  DSV41_PH(3);

  // ---- merge the 4 row-waves' states per head (both column halves hold identical m, l): per-head maximum M, sum L
  // and the waves' factors once, then the waves' accumulators scaled into LDS (row stride DVP: the 4 heads a
  // 16-lane row group writes fall on different banks) and summed
  constexpr int DVP = DV + 4;
  if (half == 0 && g == 0) {
    wm[rw][l16] = m_ref;
    wl[rw][l16] = l_run;
  }
  __syncthreads();
  if (tid < 16) {
    const float M = fmaxf(fmaxf(wm[0][tid], wm[1][tid]), fmaxf(wm[2][tid], wm[3][tid]));
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(wm[w][tid] - M);
      wf[w][tid] = f;
      L += wl[w][tid] * f;
    }
    hM[tid] = M;
    hL[tid] = L;
  }
  __syncthreads();
  {
    float* xw = (float*)ktile + rw * 16 * DVP + half * (DV / 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float fac = wf[rw][4 * g + i];
#pragma unroll
      for (int ct = 0; ct < CTH; ++ct) xw[(4 * g + i) * DVP + ct * 16 + l16] = o[ct][i] * fac;
    }
  }
  __syncthreads();
  DSV41_TS(21);
  DSV41_PH(4);
  const float* xb = (const float*)ktile;
  const bool final_out = a.nsplit == 1;
  const long pr = pos < 0 ? 0 : pos;
  const float ln2 = 0.6931471805599453f;
  constexpr int CG = DV / 8;  // 8-column groups per head: one 16-byte store each
#pragma unroll 1
  for (int e = tid; e < 16 * CG; e += 512) {
    const int hh = e / CG, c = (e - hh * CG) * 8;
    const int hout = h0 + hh;
    if (hout >= H) continue;
    const float M = hM[hh], L = hL[hh];
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 x0 = *(const float4*)(xb + (w * 16 + hh) * DVP + c);
      const float4 x1 = *(const float4*)(xb + (w * 16 + hh) * DVP + c + 4);
      v[0] += x0.x, v[1] += x0.y, v[2] += x0.z, v[3] += x0.w;
      v[4] += x1.x, v[5] += x1.y, v[6] += x1.z, v[7] += x1.w;
    }
    uint32_t pk[4];
    if (final_out) {
      const float inv = 1.0f / (L + exp2f(a.sink[hout] * kLog2e - M));
#pragma unroll
      for (int q = 0; q < 8; q += 2) {
        float re = round_bf16(v[q] * inv), im = round_bf16(v[q + 1] * inv);
        const int cc = c + q;
        if (a.rd > 0 && cc >= DV - a.rd) {
          const int jj = (cc - (DV - a.rd)) >> 1;
          const float cs = a.cos_t[pr * (a.rd / 2) + jj];
          const float sn = -a.sin_t[pr * (a.rd / 2) + jj];
          const float yr = re * cs - im * sn, yi = re * sn + im * cs;
          re = yr;
          im = yi;
        }
        pk[q / 2] = pack_bf16x2(re, im);
      }
      *(uint4*)(a.out + (long)r * a.out_rstride + (long)hout * DV + c) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
      for (int q = 0; q < 8; q += 2) pk[q / 2] = pack_bf16x2(v[q] * inv, v[q + 1] * inv);
      const long pi = ((long)r * H + hout) * a.nsplit + sp;
      if (a.coop) {  // device-scope stores: read by the unit's other workgroups, possibly on other XCDs
        __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{pk[0], pk[1], pk[2], pk[3]}, pacc_rsrc(a.pacc),
                                               (int)((pi * DV + c) * 2), 0, kCpolDevice);
        if (c == 0) {
          __hip_atomic_store(a.pm + pi, M * ln2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.pl + pi, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        *(uint4*)((uint16_t*)a.pacc + pi * DV + c) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        if (c == 0) {
          a.pm[pi] = M * ln2;  // natural-log units, as the merge expects
          a.pl[pi] = L;
        }
      }
    }
  }
  DSV41_TS(22);
  DSV41_PH(5);
  if (final_out || !a.arrive) {
    DSV41_WG_TS(1);
    return;
  }
  if (a.coop) {
    // ---- every split workgroup of the unit merges a slice once all have published.  Counter = epoch * 256 +
    // arrivals: the last arrival of a launch moves it to the next epoch (any nsplit <= 255, any history)
    unsigned long long* cnt = a.coop + ((long)r * ((H + 15) / 16) + hg) * kCoopStride;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
    __syncthreads();
    if (tid == 0) {
      const unsigned long long old = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long base = old & ~255ull;
      if ((int)(old & 255) + 1 == a.nsplit) {
        __hip_atomic_fetch_add(cnt, 256ull - a.nsplit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        int spins = 0;
#pragma unroll 1
        while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < base + a.nsplit &&
               ++spins < kCoopSpinLimit)
          __builtin_amdgcn_s_sleep(1);
        // gave up waiting (the unit's workgroups were not co-resident): the merge below may read unpublished
        // partials, so the launch reports it through the workspace's error word
        if (spins >= kCoopSpinLimit) __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    DSV41_PH(6);
    merge_slice<DV>(a, r, h0, pr, sp);
    DSV41_PH(7);
    DSV41_WG_TS(1);
    return;
  }
  // ---- the last split workgroup of the unit to finish merges all splits' partials
  __shared__ int s_slot;
  __shared__ float wts[16][33];
  int* cnt = a.arrive + (long)r * ((H + 15) / 16) + hg;
  const int old = group_arrive(cnt, home, &s_slot);
  if ((old & (kMisplaced - 1)) != a.nsplit - 1) {
    DSV41_WG_TS(1);
    return;
  }
  DSV41_PH(6);
  group_acquire(old, home);
  // a merger off the home XCD cannot see the home members' partials (plain stores, still in the home L2): the launch
  // reports it (the dispatch order that places workgroup b on XCD b % 8 did not hold)
  if (tid == 0 && xcd_id() != home) __hip_atomic_store(a.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  merge_splits<DV>(a, r, h0, pr, wts);
  DSV41_PH(7);
  DSV41_WG_TS(1);
}

// ------------------------------------------------------------------------------------------------ decode kernel, 32 heads
// Few query rows (decode), one gather round trip per workgroup: a workgroup owns one query row, 32 heads and a split
// of at most 128 key positions, all gathered into LDS at once (two 64-key halves in flight; the QK of the first half
// runs while the second lands).  Against attn_decode_kernel the rows of a split are gathered by two workgroups
// instead of four, in one round trip instead of one per 64-key tile.  8 waves:
//   QK  wave w = (hb = w & 1: heads 16hb..16hb+15 of the group, kp = w >> 1: keys 16kp..16kp+15 of each half):
//       S^T for its 32 keys (16x16x32 bf16 MFMA, A = K from LDS, B = Q in VGPRs); one maximum per head over the whole
//       split (exchanged through LDS: no online rescale), p = 2^(s - M), the bf16 probabilities into LDS in the PV
//       MFMA's operand order (k = 8g + j: key 16kp + 4g + j of half 0 for j < 4, of half 1 for j >= 4), the partial
//       sums into LDS;
//   PV  wave w: O[32 heads x columns w*DV/8 ..] = P V over the split (4 k-steps of the 16x16x32 bf16 MFMA, each V
//       fragment -- the LDS transpose read of both halves -- used for both head blocks).
// The partial (bf16, normalised by the split's sum, in the MFMA's register layout) and (m, l) are stored with
// device-scope stores; the splits of a (row, 32-head) unit then merge cooperatively in the same launch, as in
// attn_decode_kernel (every workgroup of the launch is resident at once: the host plans it so).  The head groups of
// a (row, split) are placed on one XCD, so the rows they both gather come through one L2.
// Cooperative merge of the 32-head kernel's partials (register-layout tiles): split workgroup sp of unit (r, hg)
// merges tiles [sp*NT/ns, (sp+1)*NT/ns) of the unit's NT = 8 * DV / 64 tiles, one wave per tile (the host keeps
// NT / ns <= 8).  Each wave issues its tile's partial loads first (device-scope, 8 bytes per lane and split), while
// the workgroup turns the unit's (m, l) into per-(split, head) weights in LDS (wts: >= 64 * 32 floats):
// w_s = l_s e^(m_s - M) / (sum_s l_s e^(m_s - M) + e^(sink - M)).  Output: bf16 round, inverse rope on the last rd
// columns (the partner column of a pair is the neighbouring lane).
template <int DV>
DSV41_DEV void merge_tiles32(const AttnArgs& a, int r, int hg, int HG, long pr, int sp, float* wts) {
  constexpr int CW = DV / 128, NT = 16 * CW, MS = 32;
  const int ns = a.nsplit, H = a.H, h0 = hg * 32;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int ti = (int)((long)sp * NT / ns) + wave;
  const bool act = ti < (int)((long)(sp + 1) * NT / ns);  // wave-uniform
  const __amdgpu_buffer_rsrc_t rs = pacc_rsrc(a.pacc);
  const long ub0 = ((long)r * HG + hg) * ns * (32L * DV) + ((long)ti * 64 + lane) * 4;  // split 0's entry of the lane
  auto load_batch = [&](int s0, uint2 (&v)[MS]) {  // (only the batch's splits: each load costs issue time)
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      if (s0 + u < ns) {  // wave-uniform
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)((ub0 + (long)(s0 + u) * (32L * DV)) * 2), 0,
                                                            kCpolDevice);
        v[u] = make_uint2(x[0], x[1]);
      }
    }
  };
  // this lane's output column and, for the last rd columns, its inverse-rope cos / sin: loaded once, before the
  // partials and unconditionally (the zero row when there is no rope), so that they share the partials' round trip
  // instead of each head's rotation waiting for its own load
  const int c = ((ti / CW) & 7) * (DV / 8) + (ti % CW) * 16 + l16;
  const bool rope = a.rd > 0 && c >= DV - a.rd;
  const long cidx = rope ? pr * (a.rd / 2) + ((c - (DV - a.rd)) >> 1) : 0;
  const float rcos = (a.rd > 0 ? a.cos_t : (const float*)g_zero_row)[cidx];
  const float rsin = (a.rd > 0 ? a.sin_t : (const float*)g_zero_row)[cidx];
  uint2 v[MS];
  if (act) load_batch(0, v);
  // weights: thread (head hh = tid >> 4, q = tid & 15) takes splits q, q + 16, q + 32, q + 48 (one batch of loads);
  // the head's maximum and sum over its 16 lanes
  {
    const int hh = tid >> 4, q = tid & 15, h = h0 + hh;
    float m[4], l[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sq = q + 16 * u;
      const bool ok = sq < ns && h < H;
      const long pi = ((long)r * H + (ok ? h : 0)) * ns + (ok ? sq : 0);
      m[u] = ok ? __hip_atomic_load(a.pm + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -1e30f;
      l[u] = ok ? __hip_atomic_load(a.pl + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    }
    const float M = group_max(fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3])), 16);
    float w[4], den = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      w[u] = l[u] * exp2f((m[u] - M) * kLog2e);
      den += w[u];
    }
    den = row16_sum(den) + exp2f((a.sink[h < H ? h : H - 1] - M) * kLog2e);
    const float inv = 1.0f / den;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (q + 16 * u < ns) wts[(q + 16 * u) * 32 + hh] = w[u] * inv;
  }
  lds_barrier();
  if (!act) return;
  const int hb = ti / (8 * CW), w = (ti / CW) & 7, ct = ti % CW;
  const int hl = hb * 16 + 4 * g;  // heads hl .. hl + 3 of the unit
  float num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int s0 = 0; s0 < ns; s0 += MS) {
    if (s0 > 0) load_batch(s0, v);
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      if (s0 + u < ns) {
        const float4 w = *(const float4*)(wts + (s0 + u) * 32 + hl);
        num[0] += w.x * __uint_as_float(v[u].x << 16);
        num[1] += w.y * __uint_as_float(v[u].x & 0xffff0000u);
        num[2] += w.z * __uint_as_float(v[u].y << 16);
        num[3] += w.w * __uint_as_float(v[u].y & 0xffff0000u);
      }
    }
  }
  (void)w;
  (void)ct;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float val = round_bf16(num[i]);
    const float partner = dpp_mov<0xB1>(val);  // lane ^ 1: column c ^ 1 of the same head
    if (rope) {
      const float cs = rcos, sn = -rsin;
      val = (c & 1) ? (partner * sn + val * cs) : (val * cs - partner * sn);
    }
    const int h = h0 + hl + i;
    if (h < H) a.out[(long)r * a.out_rstride + (long)h * DV + c] = f2bf(val);
  }
}

template <int DQK, int DV>
__global__ void __launch_bounds__(512) attn_decode32_kernel(const AttnArgs a) {
  DSV41_WG_TS(0);
  constexpr int KS = DQK / 32;
  constexpr int U = DQK / 8;           // 16-byte chunks per row; chunk c of row j stored at j*U + (c ^ (j & 7))
  constexpr int HALF = 64;             // keys per half
  constexpr int HALF_ELEMS = HALF * DQK;
  constexpr int kLd = HALF * U / 512;  // 16-byte direct-to-LDS loads per lane per half
  constexpr int CW = DV / 128;         // 16-column output tiles per wave and head block (an eighth of DV)
  static_assert(U % 8 == 0 && HALF * U % 512 == 0 && kLd < 16, "row width");
  static_assert(32 * DQK <= HALF_ELEMS && 32 * U % 64 == 0, "Q staging fits one half, whole waves");
  static_assert(CW >= 1, "DV a multiple of 128");
  __shared__ __align__(16) uint16_t kbuf[2 * HALF_ELEMS];  // keys (half 0 | half 1); Q staging, then the output
  __shared__ const uint16_t* rptr[2 * HALF];              // row of each key of the split (null: invalid)
  __shared__ uint4 pex[2][4][64];                          // [hb][kp][lane]: probabilities, PV operand order
  __shared__ float smax[2][4][16], ssum[2][4][16];         // [hb][kp][head]: partial maxima (log2 units) and sums
  __shared__ int ixs[2 * HALF];                             // index entries of the split

  const int HG = (a.H + 31) / 32;
  const int x = blockIdx.x % kXcds, jx = blockIdx.x / kXcds;
  const int grp = x + kXcds * (jx / HG);  // (row, split) pair; its HG head groups share XCD x
  if (grp >= a.R * a.nsplit) return;
  const int hg = jx % HG, r = grp / a.nsplit, sp = grp % a.nsplit;
  if (hg * 32 >= a.H) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hb = wave & 1, kp = wave >> 1;
  const int l16 = lane & 15, g = lane >> 4;
  const int H = a.H, h0 = hg * 32;
  DSV41_PH(0);

  // the row's position data first: scalar loads, before any inline-assembly load clobbers memory
  long slot, pos = 0, pmax = 0, plim = 0;
  if (a.mode == 1) {
    slot = a.seq[r];
    pos = a.pos[r];
    pmax = a.pmax[r];
    plim = a.plim ? a.plim[r] : pos;
  } else {
    slot = r / a.rows_per_slot;
  }
  // ---- index entries (waves 0-1, direct to LDS) and Q of the 32 heads staged into half 1, issued before any wait (the compiler's waits cannot tell these loads apart, so the waits are explicit)
  const int W = a.n1;
  const int* irow = a.t > 0 ? a.idx + (long)r * a.idx_rstride : nullptr;
  const int j0 = sp * a.chunk, j1 = min(a.L, j0 + a.chunk);
  const bool two = j1 - j0 > HALF;  // workgroup-uniform: the second half holds keys
  constexpr int QCH = 32 * U;
  constexpr int NQ01 = (QCH + 511) / 512;  // Q loads of waves 0 and 1 (QCH is a multiple of 256)
  if (wave < 2) {
    const int j = j0 + tid, jj = a.mode == 1 ? j - W : j;
    const bool ok = j < j1 && jj >= 0 && irow;  // (other entries read a valid word and are ignored)
    lds_dma4_at(ok ? (const void*)(irow + jj) : (const void*)g_zero_row, lds_addr_of(ixs) + (uint32_t)(wave * 256));
  }
  uint16_t* const qlds = kbuf + HALF_ELEMS;
#pragma unroll
  for (int u = 0; u < NQ01; ++u) {
    const int cid = u * 512 + wave * 64 + lane;
    if (u * 512 + wave * 64 < QCH) {  // wave-uniform (QCH % 64 == 0)
      const int hh = cid / U, part = cid - hh * U;
      const int h = h0 + hh < H ? h0 + hh : H - 1;  // rows of missing heads repeat the last head (never stored)
      lds_dma16(a.q + (long)r * a.q_rstride + (long)h * DQK + part * 8, qlds + (u * 512 + wave * 64) * 8);
    }
  }
  if (wave < 2) {  // row pointer of key j0 + tid (the same validity rules as attn_decode_kernel)
    __builtin_amdgcn_s_waitcnt(NQ01 | (0x7 << 4) | (0xf << 8));  // vmcnt(NQ01): this wave's index entries landed
    const int jj = a.mode == 1 ? j0 + tid - W : j0 + tid;
    const int ix = j0 + tid < j1 && jj >= 0 && irow ? ixs[tid] : -1;
    const uint16_t* base1 = a.kv1 + slot * a.kv1_sstride;
    const uint16_t* base2 = a.kv2 ? a.kv2 + slot * a.kv2_sstride : nullptr;
    const int j = j0 + tid;
    const uint16_t* p = nullptr;
    if (j < j1) {
      if (a.mode == 1 && j < W) {
        int m = (int)(pmax - j) % W;
        m = m < 0 ? m + W : m;
        const long held = pmax - m;
        if (held >= 0 && held <= plim && pos - held < W) p = base1 + (long)j * DQK;
      } else if (a.mode == 1) {
        if (ix >= 0 && ix < a.n2) p = base2 + (long)ix * DQK;
      } else if (ix >= 0 && ix < a.n1 + a.n2) {
        p = ix < a.n1 ? base1 + (long)ix * DQK : base2 + (long)(ix - a.n1) * DQK;
      }
    }
    rptr[tid] = p;
  }
  lds_barrier();  // (an LDS-only barrier: __syncthreads would wait for the Q loads in flight)
  // direct-to-LDS loads of rounds [rd0, rd1) of half hf (inline assembly: no compiler waits around them)
  auto issue = [&](int hf, auto rd0c, auto rd1c) {
    constexpr int rd0 = decltype(rd0c)::value, rd1 = decltype(rd1c)::value;
    uint16_t* buf = kbuf + hf * HALF_ELEMS;
    const uint16_t* src[rd1 > rd0 ? rd1 - rd0 : 1];  // row pointers read before the first load (the loads clobber
#pragma unroll                                        // memory)
    for (int rd = rd0; rd < rd1; ++rd) {
      const int q = rd * 512 + wave * 64 + lane;  // LDS chunk position
      const int jr = q / U, cs = q - jr * U;
      const uint16_t* p = rptr[hf * HALF + jr];
      src[rd - rd0] = p ? p + (cs ^ (jr & 7)) * 8 : g_zero_row;
    }
#pragma unroll
    for (int rd = rd0; rd < rd1; ++rd) lds_dma16(src[rd - rd0], buf + (rd * 512 + wave * 64) * 8);
  };
  using C0 = std::integral_constant<int, 0>;
  using CQ = std::integral_constant<int, NQ01>;  // rounds from NQ01 on lie past the Q staging (LDS chunks < QCH)
  using CL = std::integral_constant<int, kLd>;
  static_assert(NQ01 <= kLd, "Q staging within half 1");
  issue(0, C0{}, CL{});
  if (two) issue(1, CQ{}, CL{});
  // Q has landed once at most the key loads issued after it remain (loads complete in order)
  if (two)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kLd - NQ01));
  else
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kLd));
  lds_barrier();  // every wave's Q chunks have landed (the key loads stay in flight)
  DSV41_PH(1);
  uint4 qf[KS];  // B operand: Q of head 16hb + l16, k = 32 ks + 8g ..
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const uint4*)(qlds + (hb * 16 + l16) * DQK + ks * 32 + g * 8);
  lds_barrier();  // (Q has been read: the rest of half 1 takes its chunks)
  if (two) issue(1, C0{}, CQ{});
  DSV41_PH(2);

  // ---- S^T of this wave's 16 keys of each half (key row 16kp + l16 of the half as the A operand)
  auto qk = [&](int hf) {
    const int jr = kp * 16 + l16;
    const uint16_t* krow = kbuf + hf * HALF_ELEMS + jr * DQK;
    f32x4_t acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      acc = mfma_bf16_16x16x32(*(const uint4*)(krow + (((ks * 4 + g) ^ (jr & 7)) * 8)), qf[ks], acc);
    return acc;  // acc[i] = score of key 16kp + 4g + i of the half, head 16hb + l16
  };
  if (two)
    __builtin_amdgcn_s_waitcnt(kLd | (0x7 << 4) | (0xf << 8));  // vmcnt(kLd): half 0 has landed
  else
    __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  const f32x4_t s0 = qk(0);
  f32x4_t s1 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if (two) {
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    s1 = qk(1);
  }
  DSV41_PH(3);

  // ---- softmax over the split: one maximum per head (log2 units), probabilities and partial sums
  const float sl2 = a.scale * kLog2e;
  float xv[8];
  float mx = -1e30f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int kk = (e >> 2) * HALF + kp * 16 + 4 * g + (e & 3);
    xv[e] = rptr[kk] ? (e < 4 ? s0[e & 3] : s1[e & 3]) * sl2 : -1e30f;
    mx = fmaxf(mx, xv[e]);
  }
  mx = row_max4(mx);
  if (g == 0) smax[hb][kp][l16] = mx;
  lds_barrier();
  const float M = fmaxf(fmaxf(smax[hb][0][l16], smax[hb][1][l16]), fmaxf(smax[hb][2][l16], smax[hb][3][l16]));
  float pv[8];
  float ps = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int kk = (e >> 2) * HALF + kp * 16 + 4 * g + (e & 3);
    pv[e] = rptr[kk] ? exp2f(xv[e] - M) : 0.0f;
    ps += pv[e];
  }
  ps = row_sum4(ps);
  if (g == 0) ssum[hb][kp][l16] = ps;
  pex[hb][kp][lane] = make_uint4(pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                                 pack_bf16x2(pv[6], pv[7]));
  lds_barrier();  // probabilities and sums visible

  // ---- PV: O[heads 16b + 4g + i][columns w*DV/8 + 16ct + l16] for both head blocks b (each V fragment read once)
  f32x4_t o[2][CW];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int ct = 0; ct < CW; ++ct) o[b][ct] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int vj = 4 * g + (l16 >> 2);
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) {
    const uint4 pa0 = pex[0][k4][lane], pa1 = pex[1][k4][lane];
    const int jr = k4 * 16 + vj;  // V rows jr (half 0) and jr of half 1: (jr + 64) & 7 = jr & 7
    const uint16_t* vrow = kbuf + jr * DQK + ((l16 & 1) << 2);
    const int vsw = jr & 7;
#pragma unroll
    for (int ct = 0; ct < CW; ++ct) {
      const int cch = ((wave * (DV / 8) + ct * 16) >> 3) + ((l16 & 3) >> 1);  // chunk of column col0 + 4*(l16&3)
      const uint16_t* pp = vrow + ((cch ^ vsw) << 3);
      const uint2 v0 = lds_read_tr16(pp);
      const uint2 v1 = two ? lds_read_tr16(pp + HALF_ELEMS) : make_uint2(0u, 0u);
      const uint4 vb = make_uint4(v0.x, v0.y, v1.x, v1.y);
      o[0][ct] = mfma_bf16_16x16x32(pa0, vb, o[0][ct]);
      o[1][ct] = mfma_bf16_16x16x32(pa1, vb, o[1][ct]);
    }
  }
  DSV41_PH(4);

  // ---- the split's partial: O / l in bf16 in the MFMA's register layout (tile (b, w, ct): 64 lanes x 4 heads, one
  // 8-byte device-scope store per lane and tile), m (natural-log units) and l per head
  const long pr = pos < 0 ? 0 : pos;
  {
    const long ub = (((long)r * HG + hg) * a.nsplit + sp) * (32L * DV);  // this split's partial (bf16 elements)
    const __amdgpu_buffer_rsrc_t rs = pacc_rsrc(a.pacc);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float invl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hl = 4 * g + i;
        const float l = ssum[b][0][hl] + ssum[b][1][hl] + ssum[b][2][hl] + ssum[b][3][hl];
        invl[i] = l > 0.0f ? 1.0f / l : 0.0f;
      }
#pragma unroll
      for (int ct = 0; ct < CW; ++ct) {
        const long off = ub + ((long)((b * 8 + wave) * CW + ct) * 64 + lane) * 4;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{pack_bf16x2(o[b][ct][0] * invl[0], o[b][ct][1] * invl[1]),
                                                      pack_bf16x2(o[b][ct][2] * invl[2], o[b][ct][3] * invl[3])},
                                              rs, (int)(off * 2), 0, kCpolDevice);
      }
    }
  }
  if (tid < 32 && h0 + tid < H) {
    const int hb2 = tid >> 4, hl = tid & 15;
    const float Mh = fmaxf(fmaxf(smax[hb2][0][hl], smax[hb2][1][hl]), fmaxf(smax[hb2][2][hl], smax[hb2][3][hl]));
    const float Lh = ssum[hb2][0][hl] + ssum[hb2][1][hl] + ssum[hb2][2][hl] + ssum[hb2][3][hl];
    const long pi = ((long)r * H + h0 + tid) * a.nsplit + sp;
    __hip_atomic_store(a.pm + pi, Mh * 0.6931471805599453f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.pl + pi, Lh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  DSV41_PH(5);

  // ---- every split workgroup of the unit merges a slice once all have published.  Counter = epoch * 256 +
  // arrivals: the last arrival of a launch moves it to the next epoch (any nsplit <= 255, any history)
  unsigned long long* cnt = a.coop + ((long)r * HG + hg) * kCoopStride;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  if (tid == 0) {
    const unsigned long long old = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long base = old & ~255ull;
    if ((int)(old & 255) + 1 == a.nsplit) {
      __hip_atomic_fetch_add(cnt, 256ull - a.nsplit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      int spins = 0;
#pragma unroll 1
      while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < base + a.nsplit &&
             ++spins < kCoopSpinLimit)
        __builtin_amdgcn_s_sleep(1);
      // gave up waiting (the unit's workgroups were not co-resident): the merge below may read unpublished
      // partials, so the launch reports it through the workspace's error word
      if (spins >= kCoopSpinLimit) __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  DSV41_PH(6);
  merge_tiles32<DV>(a, r, hg, HG, pr, sp, (float*)kbuf);
  DSV41_PH(7);
  DSV41_WG_TS(1);
}

// ------------------------------------------------------------------------------------------------ prefill kernel
// Many query rows, pipelined roles: one workgroup per (query row, 64 heads), whole key list, 32-key tiles, three
// stages in flight across the waves (iteration t, one workgroup barrier B0 each):
//   QK waves 0..3, hq = w: heads 16hq..16hq+15 over all 32 keys of the tile: the MFMAs of S for tile t (16x16x32
//       bf16; Q of 16 heads in VGPRs leaves room for the K fragments of both 16-key blocks, read six k steps ahead
//       of their MFMAs -- the QK wave's K reads set the tile's pace), then the softmax of tile t - 1, whose maximum
//       per head was taken in iteration t - 1 inside the wave (the four lane groups by row swaps; no exchange).
//       The probabilities (bf16, MFMA operand order) and the per-head rescale factor of tile t - 1 go to LDS.
//       Wave 0 also loads the index entries and resolves the row pointers three tiles ahead.
//   PV waves 4..7, cq = w - 4: O[64 heads x columns cq*DV/4 ..] += P V for tile t - 2 (16x16x32 bf16 MFMA over the
//       tile's 32 keys, each transposed V fragment used for four head blocks; the V fragments were read into VGPRs
//       in iteration t - 1), interleaved with the direct-to-LDS gathers of tile t + 2 (counted vmcnt waits), then
//       the V fragments of tile t - 1.
// Four tile buffers: tile t (QK), t - 1 (V read by the PV waves), t + 1 and t + 2 (in flight; tile t + 2 goes into
// tile t - 2's buffer, whose last read ended before B0).  B0: tile t has landed; P / rescale of tile t - 2 and the
// row pointers of tile t + 2 are visible.  Keep the PV waves free of register
// spills: a scratch reload waits for every outstanding load (vmcnt(0)), the in-flight gathers included.
template <int DQK, int DV>
__global__ void __launch_bounds__(512) attn_prefill_ws_kernel(const AttnArgs a) {
  constexpr int KS = DQK / 32;  // 32-deep k steps of QK^T
  constexpr int CT = DV / 64;   // 16-column output tiles per PV wave (a quarter of DV)
  constexpr int U = DQK / 8;    // 16-byte chunks per row; chunk c of row j at j*U + (c ^ (j & 7))
  static_assert(U % 8 == 0 && CT >= 1 && KS >= 2, "row widths");
  constexpr int TILE = 32, NBUF = 4;
  constexpr int TILE_ELEMS = TILE * DQK;
  constexpr int kLd = TILE * U / 256;  // loads per PV-wave lane per tile
  static_assert(TILE * U % 256 == 0 && kLd < 16, "vmcnt immediate");
  static_assert(64 * DV * 4 <= NBUF * TILE_ELEMS * 2, "output staging fits the tile buffers");
  constexpr float kRescale = 8.0f;
  __shared__ __align__(16) uint16_t ktile[NBUF * TILE_ELEMS];
  __shared__ const uint16_t* rptr[NBUF][TILE];  // row of each key (the zero row when invalid: no test per gather)
  __shared__ uint32_t rvalid[NBUF];            // bit j: key j of the tile is valid
  __shared__ int ixring[8][64];  // index entries of tile T in slot T & 7 (entries 0..31; 32..63 unused)
  __shared__ uint2 pex[2][4][2][64];  // [tile parity][head block][key block][lane]
  __shared__ __align__(16) float salpha[2][64];  // [tile parity][head]: rescale factor (1 when the reference stays)
  __shared__ __align__(16) int srescale[2][4];    // [tile parity][head block]: some factor differs from 1
  __shared__ float hfac[64];

  const int hg64 = blockIdx.y;
  const int per_xcd = (a.R + kXcds - 1) / kXcds, zb = blockIdx.z;
  const int r = (zb % kXcds) * per_xcd + zb / kXcds;  // contiguous row ranges per XCD: shared rows hit its L2
  if (r >= a.R) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool qk = wave < 4;
  const int cq = wave & 3;  // PV role
  const int l16 = lane & 15, g = lane >> 4;
  const int H = a.H;

  const int W = a.n1;
  const int* irow = a.t > 0 ? a.idx + (long)r * a.idx_rstride : nullptr;
  // key split sp = blockIdx.x takes tiles [sp * T / ns, (sp + 1) * T / ns) of the row's T tiles (keys jb .. jend)
  const int sp = blockIdx.x, all_tiles = (a.L + TILE - 1) / TILE;
  const int tb = (int)((long)sp * all_tiles / a.nsplit), te = (int)((long)(sp + 1) * all_tiles / a.nsplit);
  const int jb = tb * TILE, jend = min(a.L, te * TILE);
  const int ntiles = te - tb;
  // wave 0 loads index entries for two tiles at a time (tile 2u + (lane >> 5), key lane & 31) ...
  // wave 0 brings the index entries of tile T into ring slot T & 7 by direct-to-LDS loads (entries outside the list
  // read the zero row; resolve() applies the validity).  A register load would not do: the compiler waited for it
  // where the branch that hands it on joined -- a memory round trip on the critical wave every other tile.
  auto ix_dma = [&](int T) {
    const int j = jb + T * TILE + (lane & 31);
    const int jj = a.mode == 1 ? j - W : j;
    const bool ok = lane < 32 && j < jend && jj >= 0 && irow;
    lds_dma4_at(ok ? (const void*)(irow + jj) : (const void*)g_zero_row, lds_addr_of(&ixring[T & 7][0]));
  };
  long slot, pos = 0, pmax = 0, plim = 0;
  if (a.mode == 1) {
    slot = a.seq[r];
    pos = a.pos[r];
    pmax = a.pmax[r];
    plim = a.plim ? a.plim[r] : pos;
  } else {
    slot = r / a.rows_per_slot;
  }
  const uint16_t* base1 = a.kv1 + slot * a.kv1_sstride;
  const uint16_t* base2 = a.kv2 ? a.kv2 + slot * a.kv2_sstride : nullptr;
  // ... and the lanes holding tile ti (half ti & 1 of the wave) resolve its row pointers
  auto resolve = [&](int ti) {
    if (wave == 0 && (lane >> 5) == (ti & 1)) {
      const int j = jb + ti * TILE + (lane & 31);
      const int ix = irow ? ixring[ti & 7][lane & 31] : -1;
      const uint16_t* p = nullptr;
      if (j < jend) {
        if (a.mode == 1 && j < W) {
          int m = (int)(pmax - j) % W;
          m = m < 0 ? m + W : m;
          const long held = pmax - m;
          if (held >= 0 && held <= plim && pos - held < W) p = base1 + (long)j * DQK;
        } else if (a.mode == 1) {
          if (ix >= 0 && ix < a.n2) p = base2 + (long)ix * DQK;
        } else if (ix >= 0 && ix < a.n1 + a.n2) {
          p = ix < a.n1 ? base1 + (long)ix * DQK : base2 + (long)(ix - a.n1) * DQK;
        }
      }
      rptr[ti % NBUF][lane & 31] = p ? p : g_zero_row;
      const uint32_t bits = (uint32_t)(__ballot(p != nullptr) >> (32 * (ti & 1)));
      if ((lane & 31) == 0) rvalid[ti % NBUF] = bits;
    }
  };

  {
    if (wave == 0) {
#pragma unroll
      for (int T = 0; T < 5; ++T) ix_dma(T);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    resolve(0);
    resolve(1);
    resolve(2);
    resolve(3);  // (every slot holds valid pointers: the gathers past the row read through stale slots)
  }
  // zero probabilities and rescale words "of tiles -2 and -1": the PV waves' first two iterations multiply zeros
  // instead of branching around their MFMAs
#pragma unroll
  for (int u = 0; u < 4; ++u) ((uint32_t*)&pex[0][0][0][0])[u * 512 + tid] = 0u;
  if (tid < 8) (&srescale[0][0])[tid] = 0;
  float* stg = (float*)ktile;  // output staging [64 heads][DV] once the tiles are done
#ifndef DSV41_QKT
#define DSV41_QKT 0
#endif
#define PF_TS(k, thr) \
  if (t >= 30 && t < 34) DSV41_TST(16 * (t - 30) + (k), thr)
  // The two roles run separate loops (so Q and the O accumulators never share registers) with the same barrier
  // sequence: one after the prologue, B0 per iteration t = 0..ntiles, two in the epilogue.
  if (qk) {
    const int hq = wave;  // heads 16 hq .. 16 hq + 15, all 32 keys of each tile
    uint4 qf[KS];
    {
      const int h = hg64 * 64 + 16 * hq + l16;
      const uint16_t* qrow = a.q + (long)r * a.q_rstride + (long)(h < H ? h : H - 1) * DQK + g * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const uint4*)(qrow + ks * 32);
    }
    float m_ref = -1e30f, l_run = 0.0f, tmax_prev = -1e30f;
    const float sl2 = a.scale * kLog2e;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float scp[2][4];  // scaled, masked scores of the previous tile (key 16 kbk + 4 g + i, head 16 hq + l16)
#pragma unroll
    for (int kbk = 0; kbk < 2; ++kbk)
#pragma unroll
      for (int i = 0; i < 4; ++i) scp[kbk][i] = -1e30f;
    for (int t = 0; t <= ntiles + 1; ++t) {
      PF_TS(0, DSV41_QKT);
      lds_barrier();  // B0
      PF_TS(1, DSV41_QKT);
      if (t > ntiles) break;
      if (t + 3 < ntiles && wave == 0) {  // pointers of tile t + 3 (its slot last served tile t - 1, now done)
        ix_dma(t + 5);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(2));  // tile t + 3's entries (two loads were issued after them)
        resolve(t + 3);
      }
      PF_TS(4, DSV41_QKT);
      const int tp = t - 1;
      const uint16_t* buf = ktile + (t % NBUF) * TILE_ELEMS;
      const uint32_t vall = rvalid[t % NBUF];
      uint4 kf[2][KS];
      const uint16_t* kbase[2][2];  // [key block][k-step parity]
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk) {
        const int jr = 16 * kbk + l16;
        kbase[kbk][0] = buf + jr * DQK + ((g ^ (jr & 3)) + (jr & 4)) * 8;
        kbase[kbk][1] = kbase[kbk][0] - (jr & 4) * 16;
      }
      f32x4_t s[2][2];  // [key block][k-step parity]
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk) s[kbk][0] = s[kbk][1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      // K fragments read KD k steps ahead of their MFMAs, each k step's group pinned by a scheduling barrier (the
      // compiler's own schedule kept two or three reads in flight).  KD = 6 keeps at most ~14 LDS operations of the
      // wave outstanding; the same loop with every read issued up front (36 outstanding) gave wrong results.
      constexpr int KD = KS < 6 ? KS : 6;
#pragma unroll
      for (int ks = 0; ks < KD; ++ks)
#pragma unroll
        for (int kbk = 0; kbk < 2; ++kbk) kf[kbk][ks] = *(const uint4*)(kbase[kbk][ks & 1] + ks * 32);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s[0][ks & 1] = mfma_bf16_16x16x32(kf[0][ks], qf[ks], s[0][ks & 1]);
        s[1][ks & 1] = mfma_bf16_16x16x32(kf[1][ks], qf[ks], s[1][ks & 1]);
        if (ks + KD < KS) {
#pragma unroll
          for (int kbk = 0; kbk < 2; ++kbk)
            kf[kbk][ks + KD] = *(const uint4*)(kbase[kbk][(ks + KD) & 1] + (ks + KD) * 32);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // softmax of tile t - 1 (at t == 0 the maximum and the scores of "tile -1" are -1e30: its probabilities meet
      // zero V fragments in the PV waves, and the first valid tile's factor 2^(-1e30 - m) = 0 clears the sum)
      {
        const float m_new = tmax_prev > m_ref + kRescale ? tmax_prev : m_ref;
        const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
        m_ref = m_new;
        if (g == 0) salpha[tp & 1][16 * hq + l16] = alpha;
        const unsigned long long moved = __ballot(alpha != 1.0f);
        if (lane == 0) srescale[tp & 1][hq] = moved != 0;
        float psum = 0.0f;
#pragma unroll
        for (int kbk = 0; kbk < 2; ++kbk) {
          float p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[i] = __builtin_amdgcn_exp2f(scp[kbk][i] - m_new);
            psum += p[i];
          }
          pex[tp & 1][hq][kbk][lane] = make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]));
        }
        l_run += psum;
      }
      PF_TS(2, DSV41_QKT);
      float tm = -1e30f;
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk) {
        const uint32_t vb = vall >> (16 * kbk + 4 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          scp[kbk][i] = (vb >> i) & 1u ? (s[kbk][0][i] + s[kbk][1][i]) * sl2 : -1e30f;
          tm = fmaxf(tm, scp[kbk][i]);
        }
      }
      tmax_prev = row_max4(tm);
      PF_TS(3, DSV41_QKT);
    }
    __syncthreads();  // E1
    const float lsum = row_sum4(l_run);
    lds_barrier();  // (the barrier sequence of the other form)
    if (g == 0) {
      const int hl = 16 * hq + l16, h = hg64 * 64 + hl;
      const float l = lsum;
      if (a.nsplit > 1) {
        hfac[hl] = l > 0.0f ? 1.0f / l : 0.0f;
        if (h < H) {
          const long pi = ((long)r * H + h) * a.nsplit + sp;
          a.pm[pi] = m_ref * 0.6931471805599453f;
          a.pl[pi] = l;
        }
      } else {
        hfac[hl] = 1.0f / (l + exp2f(a.sink[h < H ? h : H - 1] * kLog2e - m_ref));
      }
    }
    __syncthreads();  // E3
  } else {
    // gathers: LDS chunk position cc = rd*256 + cq*64 + lane holds chunk (cc % U) ^ (row & 7) of row cc / U
    const uint16_t* src[kLd];  // gather sources of a tile, read before the first load (the loads clobber memory)
    auto sources = [&](int ti) {
      const uint16_t* const* rp = rptr[ti % NBUF];
#pragma unroll
      for (int rd = 0; rd < kLd; ++rd) {
        const int cc = rd * 256 + cq * 64 + lane;
        const int j = cc / U, cs = cc - j * U;
        src[rd] = rp[j] + (cs ^ (j & 7)) * 8;  // (invalid keys: the zero row, read whole)
      }
    };
    // LDS byte address of this wave's first chunk in buffer 0 (wave-uniform, computed once)
    const uint32_t wlds = lds_addr_of(ktile) + (uint32_t)(cq * 64 * 16);
    auto dma = [&](int ti, int rd) {  // direct-to-LDS 16-byte load (inline assembly: no compiler waits around it)
      lds_dma16_at(src[rd], wlds + (uint32_t)(((ti % NBUF) * TILE_ELEMS + rd * 256 * 8) * 2));
    };
    // O of heads 16b + 4g + i, columns cq*DV/4 + 16 ct + l16
    f32x4_t o[4][CT];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int c = 0; c < CT; ++c) o[b][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();
    if (ntiles > 0) {
      sources(0);
#pragma unroll
      for (int rd = 0; rd < kLd; ++rd) dma(0, rd);
    }
    if (ntiles > 1) {
      sources(1);
#pragma unroll
      for (int rd = 0; rd < kLd; ++rd) dma(1, rd);
    }
    const int vj = 4 * g + (l16 >> 2);  // key rows vj (first half) and vj + 16 (second half); (vj + 16) & 7 = vj & 7
    const int vsw = vj & 7;
    uint4 vb[CT];  // V fragments of tile t - 2, read in iteration t - 1 (zero before the first)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) vb[ct] = make_uint4(0, 0, 0, 0);
    // element offsets in a V row of column tiles ct = c4 and c4 + 4: chunk (cq DV/32 + 2 ct + h01) ^ vsw with
    // h01 = (l16 & 3) >> 1; the swizzle only permutes the low three chunk bits, so tile c4 + 4 lies 8 chunks (64
    // elements) after tile c4
    int voff[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) voff[c4] = ((cq * (DV / 32) + 2 * c4 + ((l16 & 3) >> 1)) ^ vsw) * 8;
    for (int t = 0; t <= ntiles + 1; ++t) {
      PF_TS(8, 256);
      if (t < ntiles) {
        if (t + 1 < ntiles)
          __builtin_amdgcn_s_waitcnt(kLd | (0x7 << 4) | (0xf << 8));  // vmcnt(kLd): tile t has landed
        else
          __builtin_amdgcn_s_waitcnt(0);
      }
      PF_TS(9, 256);
      lds_barrier();  // B0
      PF_TS(10, 256);
      // PV of tile t - 2 (P written in iteration t - 1, V read into registers in iteration t - 1), interleaved with
      // the gathers of tile t + 2 into buffer (t + 2) % NBUF (tile t - 2's: every read of it ended before B0; its
      // pointers were resolved in iteration t - 1); then the V fragments of tile t - 1
      // (near the end the gathers of tiles past the row land in buffers no wave reads again, from row pointers
      // left by earlier tiles: no branch per load; E1 waits for them before the buffers take the output)
      const int tp = t - 2;
      sources(t + 2);
      const uint16_t* vrow = ktile + ((t + NBUF - 1) % NBUF) * TILE_ELEMS + vj * DQK + ((l16 & 1) << 2);
      auto vread = [&](int ct) {  // column tile ct: chunk 2 ct + h01 (+ the wave's quarter), swizzled
        const uint16_t* p = vrow + voff[ct & 3] + (ct >> 2) * 64;
        const uint2 v0 = lds_read_tr16(p);
        const uint2 v1 = lds_read_tr16(p + 16 * DQK);
        return make_uint4(v0.x, v0.y, v1.x, v1.y);
      };
      // the LDS reads of the iteration first (the head blocks' rescale words, P fragments), before the gathers
      // (which clobber memory)
      uint4 pa[4];
      int4 resc;
      {
        resc = *(const int4*)srescale[tp & 1];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          // 16x16x32 MFMA over the tile's 32 keys in the k order (4g + i, then 16 + 4g + i): the A operand of
          // head block b is its two 16-key probability fragments side by side, the B operand two transposed V reads
          const uint2 p0 = pex[tp & 1][b][0][lane], p1 = pex[tp & 1][b][1][lane];
          pa[b] = make_uint4(p0.x, p0.y, p1.x, p1.y);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
      if (resc.x | resc.y | resc.z | resc.w) {  // rescale by the factors of tile t - 2 (rarely needed)
        const int rb[4] = {resc.x, resc.y, resc.z, resc.w};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (rb[b]) {
            const float4 al = *(const float4*)&salpha[tp & 1][16 * b + 4 * g];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
              o[b][ct][0] *= al.x;
              o[b][ct][1] *= al.y;
              o[b][ct][2] *= al.z;
              o[b][ct][3] *= al.w;
            }
          }
        }
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int rd = ct * kLd / CT; rd < (ct + 1) * kLd / CT; ++rd) dma(t + 2, rd);
#pragma unroll
        for (int b = 0; b < 4; ++b) o[b][ct] = mfma_bf16_16x16x32(pa[b], vb[ct], o[b][ct]);
      }
      __builtin_amdgcn_sched_barrier(0);  // (after the MFMAs: the fragments are overwritten)
      if (t >= 1 && t <= ntiles) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) vb[ct] = vread(ct);
      }
      PF_TS(11, 256);
    }
    __syncthreads();  // E1: every PV wave is past its last V read, so the tile buffers can take the output
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) stg[(16 * b + 4 * g + i) * DV + cq * (DV / 4) + ct * 16 + l16] = o[b][ct][i];
    lds_barrier();    // E2
    __syncthreads();  // E3
  }
#undef PF_TS
  constexpr int CG = DV / 8;
#pragma unroll 1
  for (int e = tid; e < 64 * CG; e += 512) {
    const int hl = e / CG, c = (e - hl * CG) * 8, h = hg64 * 64 + hl;
    if (h >= H) continue;
    const float f = hfac[hl];
    const float4 x0 = *(const float4*)(stg + hl * DV + c), x1 = *(const float4*)(stg + hl * DV + c + 4);
    const uint4 v = make_uint4(pack_bf16x2(x0.x * f, x0.y * f), pack_bf16x2(x0.z * f, x0.w * f),
                               pack_bf16x2(x1.x * f, x1.y * f), pack_bf16x2(x1.z * f, x1.w * f));
    if (a.nsplit > 1)  // bf16 partial [R, H, nsplit, DV] (merged by attn_decode_combine_kernel)
      *(uint4*)((uint16_t*)a.pacc + (((long)r * H + h) * a.nsplit + sp) * DV + c) = v;
    else
      *(uint4*)(a.out + (long)r * a.out_rstride + (long)h * DV + c) = v;
  }
}

// Merge bf16-normalised partials: out = sum_s w_s l_s o_s / (sum_s w_s l_s + exp(sink - M)), w_s = exp(m_s - M).
// One workgroup per (row, 4 heads); thread -> (head, 8 consecutive columns); all split loads are independent.
template <int DV>
__global__ void __launch_bounds__(256) attn_decode_combine_kernel(const AttnArgs a) {
  constexpr int MAXS = 32;  // splits held in registers; more are merged in further rounds
  constexpr int B = 8;      // partial rows loaded per batch
  const int r = blockIdx.y;
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int H = a.H, ns = a.nsplit;
  if (h >= H) return;
  const long base = ((long)r * H + h) * ns;
  const long pr = (a.mode == 1 && a.pos) ? (a.pos[r] < 0 ? 0 : a.pos[r]) : 0;
  const uint16_t* pb = (const uint16_t*)a.pacc;
  // the inverse rope's cos / sin of the 4 column pairs at c (the last rd columns), issued with the partials'
  // loads and unconditionally (the zero row when there is no rope): one round trip instead of one per pair
  auto rope_load = [&](int c, float (&rc)[4], float (&rs)[4]) {
    const float* cb = a.rd > 0 ? a.cos_t : (const float*)g_zero_row;
    const float* sb = a.rd > 0 ? a.sin_t : (const float*)g_zero_row;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int cc = c + 2 * e;
      const long idx = a.rd > 0 && cc >= DV - a.rd ? pr * (a.rd / 2) + ((cc - (DV - a.rd)) >> 1) : 0;
      rc[e] = cb[idx];
      rs[e] = sb[idx];
    }
  };
  auto finish = [&](int c, const float (&num)[8], float den, const float (&rc)[4], const float (&rs)[4]) {
    const float inv = 1.0f / den;
    uint32_t pk[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float re = round_bf16(num[e] * inv), im = round_bf16(num[e + 1] * inv);
      const int cc = c + e;
      if (a.rd > 0 && cc >= DV - a.rd) {
        const float cs = rc[e / 2], sn = -rs[e / 2];
        const float yr = re * cs - im * sn, yi = re * sn + im * cs;
        re = yr;
        im = yi;
      }
      pk[e / 2] = pack_bf16x2(re, im);
    }
    *(uint4*)(a.out + (long)r * a.out_rstride + (long)h * DV + c) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  };
  if (ns <= B && DV == 512) {
    // one round trip: the splits' maxima, sums and partial rows are loaded together (none depends on another)
    const int c = (threadIdx.x & 63) * 8;
    uint4 v[B];
    float m[B], l[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int s = u < ns ? u : ns - 1;
      v[u] = *(const uint4*)(pb + (base + s) * DV + c);
      m[u] = u < ns ? a.pm[base + s] : -1e30f;
      l[u] = a.pl[base + s];
    }
    float rc[4], rs[4];
    rope_load(c, rc, rs);
    float mx = -1e30f;
#pragma unroll
    for (int u = 0; u < B; ++u) mx = fmaxf(mx, m[u]);
    float num[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float den = exp2f((a.sink[h] - mx) * kLog2e);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const float wg = u < ns ? l[u] * exp2f((m[u] - mx) * kLog2e) : 0.0f;
      den += wg;
      const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        num[2 * e] += wg * __uint_as_float(vv[e] << 16);
        num[2 * e + 1] += wg * __uint_as_float(vv[e] & 0xffff0000u);
      }
    }
    finish(c, num, den, rc, rs);
    return;
  }
  float mx = -1e30f;
  for (int s0 = 0; s0 < ns; s0 += MAXS) {
    float mv[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) mv[s] = s0 + s < ns ? a.pm[base + s0 + s] : -1e30f;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) mx = fmaxf(mx, mv[s]);
  }
  const float sink_term = exp2f((a.sink[h] - mx) * kLog2e);
  for (int c = (threadIdx.x & 63) * 8; c < DV; c += 512) {
    float rc[4], rs[4];
    rope_load(c, rc, rs);
    float num[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float den = sink_term;
    for (int s0 = 0; s0 < ns; s0 += B) {
      uint4 v[B];
      float wg[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int s = s0 + u < ns ? s0 + u : ns - 1;
        v[u] = *(const uint4*)(pb + (base + s) * DV + c);
        wg[u] = s0 + u < ns ? a.pl[base + s] * exp2f((a.pm[base + s] - mx) * kLog2e) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        den += wg[u];
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          num[2 * e] += wg[u] * __uint_as_float(vv[e] << 16);
          num[2 * e + 1] += wg[u] * __uint_as_float(vv[e] & 0xffff0000u);
        }
      }
    }
    finish(c, num, den, rc, rs);
  }
}

// Kernel choice: few (row, 64-head) pairs -> decode kernel (16-head workgroups, key splits merged in the launch);
// otherwise the 64-head kernel, with key splits (bf16 partials + the combine kernel) when the rows alone do not
// fill the chip.
// Measured (one layer-step, 576/512, 64 heads, 2176 keys per row): 1 row (C4) decode kernel 18.5 us vs 64-head
// kernel + splits 30.5 us; 4 rows (C2) 19.8 vs 32.5 us; 48 rows (C5) 85.2 vs 57.3 us (the decode kernel's four
// 16-head workgroups per row each gather every row: at many rows that redundancy dominates).
bool use_decode_kernel(int R, int H) { return (long)R * ((H + 63) / 64) < 16; }

template <int DQK, int DV>
int launch_attn(AttnArgs& a, hipStream_t st) {
  if constexpr (DV % 128 == 0) {
    if (use_decode_kernel(a.R, a.H) && a.dec32) {
      const int HG2 = (a.H + 31) / 32;
      attn_decode32_kernel<DQK, DV><<<dim3(kXcds * HG2 * ((a.R * a.nsplit + kXcds - 1) / kXcds)), 512, 0, st>>>(a);
      DSV41_CHECK_LAUNCH();
      return 0;
    }
  }
  if (use_decode_kernel(a.R, a.H)) {
    const int HG = (a.H + 15) / 16;
    const dim3 grid = a.coop && a.hg_share ? dim3(kXcds * HG * ((a.R * a.nsplit + kXcds - 1) / kXcds))
                      : a.arrive          ? dim3(kXcds * a.upx * a.nsplit)
                                          : dim3(a.nsplit, HG, a.R);
    attn_decode_kernel<DQK, DV><<<grid, 512, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
    if (a.nsplit > 1 && !a.arrive) {
      attn_decode_combine_kernel<DV><<<dim3((a.H + 3) / 4, a.R), 256, 0, st>>>(a);
      DSV41_CHECK_LAUNCH();
    }
    return 0;
  }
  dim3 grid(a.nsplit, (a.H + 63) / 64, a.R);
  if (a.rd == 0) {  // (rows padded to a multiple of 8: contiguous row ranges per XCD)
    attn_prefill_ws_kernel<DQK, DV><<<dim3(a.nsplit, grid.y, (a.R + kXcds - 1) / kXcds * kXcds), 512, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
    if (a.nsplit > 1) {  // bf16 partials merged with the sink
      attn_decode_combine_kernel<DV><<<dim3((a.H + 3) / 4, a.R), 256, 0, st>>>(a);
      DSV41_CHECK_LAUNCH();
    }
    return 0;
  }
  attn_split_kernel<DQK, DV><<<grid, 256, 0, st>>>(a);
  DSV41_CHECK_LAUNCH();
  if (a.nsplit > 1) {
    attn_combine_kernel<DV><<<dim3(a.H, a.R), 256, 0, st>>>(a);
    DSV41_CHECK_LAUNCH();
  }
  return 0;
}

int dispatch(AttnArgs& a, int dqk, int dv, hipStream_t st) {
  if (dqk == 576 && dv == 512) return launch_attn<576, 512>(a, st);
  if (dqk == 512 && dv == 512) return launch_attn<512, 512>(a, st);
  if (dqk == 256 && dv == 256) return launch_attn<256, 256>(a, st);
  if (dqk == 128 && dv == 128) return launch_attn<128, 128>(a, st);
  if (dqk == 64 && dv == 64) return launch_attn<64, 64>(a, st);
  // head widths: 512 (reference), 576/512 (absorbed MLA); 256/128/64 for reduced test geometries
  return (int)hipErrorInvalidValue;
}

// Compute units per XCD of the current device (queried once per device).
int cus_per_xcd() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n / kXcds;
  }
  return cached[dev];
}

constexpr int kFuseMaxSplits = 32;  // splits a decode launch merges itself
#ifndef DSV41_DEC_WG
#define DSV41_DEC_WG 192
#endif
constexpr int kDecWG = DSV41_DEC_WG;
  // decode-kernel workgroups the split plan aims at

// Split plan.  Decode kernel: <= 192 workgroups over (rows x 16-head groups x splits), >= 2 tiles of 64 keys per
// split.  64-head kernel: splits up to one workgroup per CU when rows are few, >= 2 tiles of 32 keys per split.
// The 32-head decode kernel's plan (automatic split count only, DV a multiple of 128): splits of 128 keys (64 when that leaves fewer than
// 96 workgroups), 8 to 64 of them, every workgroup resident at once (one per CU; the head groups of a (row, split) on one
// XCD).  DSV41_ATTN_DEC32=0 selects the 16-head kernel instead.  Returns false when it does not apply.
bool plan_dec32(int R, int H, int L, int dv, int* nsplit, int* chunk) {
  const char* env = getenv("DSV41_ATTN_DEC32");
  if ((env && atoi(env) == 0) || !use_decode_kernel(R, H) || dv % 128) return false;
  const int HG2 = (H + 31) / 32;
  int ch = 128;
  if ((long)R * HG2 * ((L + 127) / 128) < 96) ch = 64;
  const int ns = (L + ch - 1) / ch;
  if (ns < 8 || ns > 64) return false;  // (the merge: <= 8 of 64 output tiles per workgroup, <= 64 splits)
  if ((long)HG2 * (((long)R * ns + kXcds - 1) / kXcds) > cus_per_xcd()) return false;
  *nsplit = ns;
  *chunk = ch;
  return true;
}

void plan(int R, int H, int L, int want, int dv, int* nsplit, int* chunk) {
  if (want <= 0 && plan_dec32(R, H, L, dv, nsplit, chunk)) return;
  const bool dec = use_decode_kernel(R, H);
  const int tile = dec ? 64 : 32;
  const int tiles = (L + tile - 1) / tile < 1 ? 1 : (L + tile - 1) / tile;
  int per;
  if (want > 0) {
    per = (tiles + want - 1) / want;
  } else if (dec) {
    // <= 192 workgroups (three quarters of the CUs; each holds one), >= 2 tiles per split; the decode kernel balances
    // the tiles over the splits.  Measured at C2 (16 units, cooperative merge): 12 splits 19.5 us, 16 splits 20.2 us.
    const long wgs = (long)R * ((H + 15) / 16);
    const int cap = tiles / 2 < 1 ? 1 : tiles / 2;
    int ns = (int)(wgs >= kDecWG ? 1 : kDecWG / wgs);
    if (ns > cap) ns = cap;
    *nsplit = ns;
    *chunk = (tiles + ns - 1) / ns * tile;
    return;
  } else {
    const long wgs = (long)R * ((H + 63) / 64);
    // one workgroup per CU (the kernel holds a CU alone): splits up to one round of the grid, no second round
    const long cus = (long)cus_per_xcd() * kXcds > 0 ? (long)cus_per_xcd() * kXcds : 256;
    const long target = wgs >= cus ? 1 : cus / wgs;
    per = (int)((tiles + target - 1) / target);
    if (per < 2 && target > 1) per = 2;
  }
  if (per < 1) per = 1;
  if (per > tiles) per = tiles;
  *chunk = per * tile;
  *nsplit = (tiles + per - 1) / per;
}

// The decode kernel merges its own splits (XCD-local units): cooperatively when every workgroup is resident at
// once, else by the last arrival of each unit (any unit count; with fewer units than XCDs some XCDs idle).
bool fuse_merge(int R, int H, int ns) { (void)R; (void)H; return ns > 1 && ns <= kFuseMaxSplits; }

// Decode-kernel workspace: the error word (int at byte 0: 1 = a cooperative merge stopped waiting for its unit),
// then the split arrival counters from byte 256 (their size depends on R and H only, so calls with any split count
// find them where the previous call left them at rest), then m, l (fp32) and the bf16 partials.
constexpr long kCounterBase = 256;
long counter_bytes(int R, int H) {
  const long units = (long)R * ((H + 15) / 16);
  return kCounterBase + (units * 4 + 8 + units * 8 * kCoopStride + 255) / 256 * 256;  // int counters, pad, u64 counters
}

long workspace_bytes(int R, int H, int ns, int dv) {
  if (ns <= 1) return 0;
  // (the 32-head kernel's partials cover whole 32-head groups)
  if (use_decode_kernel(R, H)) return counter_bytes(R, H) + (long)R * H * ns * 8 + (long)R * ((H + 31) / 32 * 32) * ns * 2L * dv;
  return (long)R * H * ns * (2 + dv) * 4;
}

int finish_plan(AttnArgs& a, int want_nsplit, void* ws, long ws_bytes, int dv) {
  int ns, chunk;
  plan(a.R, a.H, a.L, want_nsplit, dv, &ns, &chunk);
  a.nsplit = ns;
  a.chunk = chunk;
  if (ns > 1) {
    const long need = workspace_bytes(a.R, a.H, ns, dv);
    if (!ws || ws_bytes < need) return (int)hipErrorInvalidValue;
    const bool dec = use_decode_kernel(a.R, a.H);
    float* f = (float*)((char*)ws + (dec ? counter_bytes(a.R, a.H) : 0));
    a.pm = f;
    a.pl = f + (long)a.R * a.H * ns;
    a.pacc = f + 2L * a.R * a.H * ns;
    if (dec && want_nsplit <= 0 && plan_dec32(a.R, a.H, a.L, dv, &ns, &chunk)) {
      a.dec32 = 1;
      a.err = (int*)ws;
      a.coop = (unsigned long long*)((char*)ws + kCounterBase + ((long)a.R * ((a.H + 15) / 16) * 4 + 7) / 8 * 8);
    } else if (dec && fuse_merge(a.R, a.H, ns)) {
      a.units = a.R * ((a.H + 15) / 16);
      a.upx = (a.units + kXcds - 1) / kXcds;
      a.err = (int*)ws;
      a.arrive = (int*)((char*)ws + kCounterBase);
      // cooperative merge when every workgroup of the launch can be resident at once (one per CU, the XCDs dealt
      // round-robin): early arrivals wait for the rest of their unit
      if ((long)a.upx * ns <= cus_per_xcd()) {
        a.coop = (unsigned long long*)((char*)ws + kCounterBase + ((long)a.units * 4 + 7) / 8 * 8);
        // head groups of a (row, split) on one XCD when that placement is also resident at once
        const long per_xcd = (long)((a.H + 15) / 16) * ((a.R * ns + kXcds - 1) / kXcds);
        a.hg_share = per_xcd <= cus_per_xcd();
      }
    }
  }
  return 0;
}

// Arguments of a sattn2 launch (dsv41_sattn2 and its no-allocation variant); returns 0 or a hipError_t.
int sattn2_args(AttnArgs& a, const void* q, const void* kv_win, long win_sstride, int win, const void* kv_c,
                long c_sstride, int n_c_rows, const int* idx, int t, const long* pos, const long* seq,
                const long* pmax, const long* plim, const float* sink, const float* cos_t, const float* sin_t, int rd,
                float scale, void* out, int B, int h, int dv) {
  if (win <= 0 || h <= 0 || t < 0 || rd < 0 || rd > dv || (rd & 1)) return (int)hipErrorInvalidValue;
  if (t > 0 && (!kv_c || !idx)) return (int)hipErrorInvalidValue;
  a = AttnArgs{};
  a.q = (const uint16_t*)q;
  a.H = h;
  a.R = B;
  a.mode = 1;
  a.kv1 = (const uint16_t*)kv_win;
  a.kv1_sstride = win_sstride;
  a.n1 = win;
  a.kv2 = (const uint16_t*)kv_c;
  a.kv2_sstride = c_sstride;
  a.n2 = n_c_rows;
  a.idx = idx;
  a.idx_rstride = t;
  a.t = t;
  a.rows_per_slot = 1;
  a.pos = pos;
  a.seq = seq;
  a.pmax = pmax;
  a.plim = plim;
  a.scale = scale;
  a.sink = sink;
  a.L = win + t;
  a.out = (uint16_t*)out;
  a.out_rstride = (long)h * dv;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.rd = rd;
  return 0;
}

// ---- the no-allocation variant's scratch: one static array per device (each GPU the library runs on holds its
// copy until the process ends), its device address taken once per device with hipGetSymbolAddress
__device__ __align__(256) unsigned char scratch[DSV41_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};

// Device address of `scratch` on the current device (null on failure; *rc gets the hipError_t).
void* scratch_ptr(int* rc) {
  int dev = 0;
  *rc = (int)hipGetDevice(&dev);
  if (*rc) return nullptr;
  if (dev < 0 || dev >= 64) {
    *rc = (int)hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    *rc = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*rc) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

__global__ void zero_words_kernel(unsigned int* p, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace

extern "C" {

#ifdef DSV41_TIMING
int dsv41_read_ts_attn(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ts), sizeof(g_dsv41_ts)); }
int dsv41_read_ph_attn(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_ph), sizeof(g_dsv41_ph)); }
int dsv41_read_wg_attn(long long* host) { return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dsv41_wg), sizeof(g_dsv41_wg)); }
#endif


long dsv41_attn_workspace_bytes(int R, int H, int L, int dv, int want_nsplit) {
  int ns, chunk;
  plan(R, H, L, want_nsplit, dv, &ns, &chunk);
  return workspace_bytes(R, H, ns, dv);
}

int dsv41_sparse_attn(const void* q, const void* kv, const float* sink, const int* idx, void* out, int b, int s, int h,
                      int dqk, int dv, int n_kv, long kv_bstride, int t, float scale, int want_nsplit, void* ws,
                      long ws_bytes, void* stream) {
  if (b <= 0 || s <= 0) return 0;
  if (n_kv <= 0 || t < 0 || h <= 0) return (int)hipErrorInvalidValue;
  AttnArgs a{};
  a.q = (const uint16_t*)q;
  a.q_rstride = (long)h * dqk;
  a.H = h;
  a.R = b * s;
  a.mode = 0;
  a.kv1 = (const uint16_t*)kv;
  a.kv1_sstride = kv_bstride;
  a.n1 = n_kv;
  a.kv2 = nullptr;
  a.n2 = 0;
  a.idx = idx;
  a.idx_rstride = t;
  a.t = t;
  a.rows_per_slot = s;
  a.scale = scale;
  a.sink = sink;
  a.L = t;
  a.out = (uint16_t*)out;
  a.out_rstride = (long)h * dv;
  a.rd = 0;
  int rc = finish_plan(a, want_nsplit, ws, ws_bytes, dv);
  if (rc) return rc;
  return dispatch(a, dqk, dv, (hipStream_t)stream);
}

int dsv41_sparse_attn_kv2(const void* q, const void* kv, const void* kv2, const float* sink, const int* idx, void* out,
                          int b, int s, int h, int dqk, int dv, int n_kv, long kv_bstride, int n2, long kv2_bstride,
                          int t, long idx_rstride, float scale, int want_nsplit, void* ws, long ws_bytes,
                          void* stream) {
  if (b <= 0 || s <= 0) return 0;
  if (n_kv <= 0 || n2 < 0 || (n2 > 0 && !kv2) || t < 0 || h <= 0 || idx_rstride < t) return (int)hipErrorInvalidValue;
  AttnArgs a{};
  a.q = (const uint16_t*)q;
  a.q_rstride = (long)h * dqk;
  a.H = h;
  a.R = b * s;
  a.mode = 0;
  a.kv1 = (const uint16_t*)kv;
  a.kv1_sstride = kv_bstride;
  a.n1 = n_kv;
  a.kv2 = n2 > 0 ? (const uint16_t*)kv2 : nullptr;
  a.kv2_sstride = kv2_bstride;
  a.n2 = n2;
  a.idx = idx;
  a.idx_rstride = idx_rstride;
  a.t = t;
  a.rows_per_slot = s;
  a.scale = scale;
  a.sink = sink;
  a.L = t;
  a.out = (uint16_t*)out;
  a.out_rstride = (long)h * dv;
  a.rd = 0;
  int rc = finish_plan(a, want_nsplit, ws, ws_bytes, dv);
  if (rc) return rc;
  return dispatch(a, dqk, dv, (hipStream_t)stream);
}

int dsv41_sparse_attn2(const void* q, const void* kv1, const void* kv2, const float* sink, const int* idx, void* out,
                       int b, int h, int d, int n1, long kv1_bstride, int n2, long kv2_bstride, int t, float scale,
                       int want_nsplit, void* ws, long ws_bytes, void* stream) {
  if (b <= 0) return 0;
  if (n1 <= 0 || t < 0 || h <= 0) return (int)hipErrorInvalidValue;
  AttnArgs a{};
  a.q = (const uint16_t*)q;
  a.q_rstride = (long)h * d;
  a.H = h;
  a.R = b;
  a.mode = 0;
  a.kv1 = (const uint16_t*)kv1;
  a.kv1_sstride = kv1_bstride;
  a.n1 = n1;
  a.kv2 = (const uint16_t*)kv2;
  a.kv2_sstride = kv2_bstride;
  a.n2 = kv2 ? n2 : 0;
  a.idx = idx;
  a.idx_rstride = t;
  a.t = t;
  a.rows_per_slot = 1;
  a.scale = scale;
  a.sink = sink;
  a.L = t;
  a.out = (uint16_t*)out;
  a.out_rstride = (long)h * d;
  a.rd = 0;
  int rc = finish_plan(a, want_nsplit, ws, ws_bytes, d);
  if (rc) return rc;
  return dispatch(a, d, d, (hipStream_t)stream);
}

int dsv41_sattn2(const void* q, const void* kv_win, long win_sstride, int win, const void* kv_c, long c_sstride,
                 int n_c_rows, const int* idx, int t, const long* pos, const long* seq, const long* pmax,
                 const long* plim, const float* sink, const float* cos_t, const float* sin_t, int rd, float scale,
                 void* out, int B, int h, int dqk, int dv, int want_nsplit, void* ws, long ws_bytes, void* stream) {
  if (B <= 0) return 0;
  AttnArgs a;
  int rc = sattn2_args(a, q, kv_win, win_sstride, win, kv_c, c_sstride, n_c_rows, idx, t, pos, seq, pmax, plim, sink,
                       cos_t, sin_t, rd, scale, out, B, h, dv);
  if (rc) return rc;
  a.q_rstride = (long)h * dqk;
  rc = finish_plan(a, want_nsplit, ws, ws_bytes, dv);
  if (rc) return rc;
  return dispatch(a, dqk, dv, (hipStream_t)stream);
}

int dsv41_sattn2_noalloc(const void* q, const void* kv_win, long win_sstride, int win, const void* kv_c,
                         long c_sstride, int n_c_rows, const int* idx, int t, const long* pos, const long* seq,
                         const long* pmax, const long* plim, const float* sink, const float* cos_t, const float* sin_t,
                         int rd, float scale, void* out, int B, int h, int dqk, int dv, int want_nsplit,
                         void* stream) {
  if (B <= 0) return 0;
  AttnArgs a;
  int rc = sattn2_args(a, q, kv_win, win_sstride, win, kv_c, c_sstride, n_c_rows, idx, t, pos, seq, pmax, plim, sink,
                       cos_t, sin_t, rd, scale, out, B, h, dv);
  if (rc) return rc;
  a.q_rstride = (long)h * dqk;
  const long need = dsv41_attn_workspace_bytes(B, h, win + t, dv, want_nsplit);
  if (need > DSV41_SCRATCH_BYTES) return (int)hipErrorOutOfMemory;  // past the static scratch: pass fewer splits
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_ptr(&rc);
    if (!ws) return rc ? rc : (int)hipErrorInvalidValue;
  }
  rc = finish_plan(a, want_nsplit, ws, DSV41_SCRATCH_BYTES, dv);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (a.arrive || a.dec32) {  // the split counters (and error word) start at zero: a previous call may have used another layout
    const long words = counter_bytes(a.R, a.H) / 4;
    zero_words_kernel<<<(int)((words + 255) / 256 < 64 ? (words + 255) / 256 : 64), 256, 0, st>>>(
        (unsigned int*)ws, words);
    DSV41_CHECK_LAUNCH();
  }
  return dispatch(a, dqk, dv, st);
}

}  // extern "C"
