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
#include "common.h"

namespace {

struct AttnArgs {
  const uint16_t* q;  // [R, H, DQK]
  long q_rstride;     // elements between query rows
  int H, R;
  int mode;  // 0: explicit index list over [kv1 | kv2]; 1: ring (kv1, W = n1 rows) then compressed rows kv2[idx]
  const uint16_t* kv1;
  long kv1_sstride;  // elements between slots
  int n1;
  const uint16_t* kv2;
  long kv2_sstride;
  int n2;
  const int* idx;
  long idx_rstride;
  int t;
  int rows_per_slot;  // explicit mode: slot = r / rows_per_slot
  const long* pos;
  const long* seq;
  const long* pmax;
  const long* plim;
  float scale;
  const float* sink;
  int L;      // key positions per query row
  int chunk;  // key positions per split (multiple of 32)
  int nsplit;
  uint16_t* out;  // [R, H, DV] when nsplit == 1
  long out_rstride;
  float* pm;  // [R, H, nsplit]
  float* pl;
  float* pacc;  // [R, H, nsplit, DV]
  const float* cos_t;
  const float* sin_t;
  int rd;
};

DSV41_DEV uint32_t pack_bf16x2(float a, float b) { return (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16); }

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
          const long held = pmax - (((pmax - j) % W + W) % W);
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
    tmax = fmaxf(tmax, wave_shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, wave_shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f((m_run - m_new) * kLog2e);
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = (e >> 2) * 16 + 4 * g + (e & 3);
      p[e] = rptr[row] ? exp2f((p[e] - m_new) * kLog2e) : 0.0f;
      psum += p[e];
    }
    psum += wave_shfl_xor(psum, 16);
    psum += wave_shfl_xor(psum, 32);
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
        const float partner = wave_shfl_xor(v, 1);
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

template <int DQK, int DV>
int launch_attn(AttnArgs& a, hipStream_t st) {
  dim3 grid(a.nsplit, (a.H + 63) / 64, a.R);
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
  return (int)hipErrorInvalidValue;
}

// Split plan: enough workgroups to cover the chip (>= 512) when there are few query rows; chunks of >= 64 keys.
void plan(int R, int H, int L, int want, int* nsplit, int* chunk) {
  const int hblocks = (H + 63) / 64;
  const int tiles = (L + 31) / 32;
  int ns = want;
  if (ns <= 0) {
    const long wgs = (long)R * hblocks;
    ns = wgs >= 512 ? 1 : (int)((512 + wgs - 1) / wgs);
  }
  const int max_ns = tiles < 1 ? 1 : (tiles + 1) / 2;  // >= 2 tiles per split
  if (want <= 0 && ns > max_ns) ns = max_ns;
  if (ns > tiles) ns = tiles < 1 ? 1 : tiles;
  if (ns < 1) ns = 1;
  const int per = (tiles + ns - 1) / ns;
  *chunk = per * 32;
  *nsplit = (tiles + per - 1) / per;
  if (*nsplit < 1) *nsplit = 1;
}

int finish_plan(AttnArgs& a, int want_nsplit, void* ws, long ws_bytes, int dv) {
  int ns, chunk;
  plan(a.R, a.H, a.L, want_nsplit, &ns, &chunk);
  a.nsplit = ns;
  a.chunk = chunk;
  if (ns > 1) {
    const long need = (long)a.R * a.H * ns * (2 + dv) * 4;
    if (!ws || ws_bytes < need) return (int)hipErrorInvalidValue;
    float* f = (float*)ws;
    a.pm = f;
    a.pl = f + (long)a.R * a.H * ns;
    a.pacc = f + 2L * a.R * a.H * ns;
  }
  return 0;
}

}  // namespace

extern "C" {

long dsv41_attn_workspace_bytes(int R, int H, int L, int dv, int want_nsplit) {
  int ns, chunk;
  plan(R, H, L, want_nsplit, &ns, &chunk);
  return ns > 1 ? (long)R * H * ns * (2 + dv) * 4 : 0;
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
  if (win <= 0 || h <= 0 || t < 0 || rd < 0 || rd > dv || (rd & 1)) return (int)hipErrorInvalidValue;
  if (t > 0 && (!kv_c || !idx)) return (int)hipErrorInvalidValue;
  AttnArgs a{};
  a.q = (const uint16_t*)q;
  a.q_rstride = (long)h * dqk;
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
  int rc = finish_plan(a, want_nsplit, ws, ws_bytes, dv);
  if (rc) return rc;
  return dispatch(a, dqk, dv, (hipStream_t)stream);
}

}  // extern "C"
