/*
 * dsv41_hip.h -- C ABI of the MI355X (gfx950) sparse-attention path of DeepSeek-V4.1 as the dsv41 runtime runs it.
 *
 * Conventions (every entry point):
 *   - plain device pointers, element counts / strides in ELEMENTS of the pointed-to type unless stated (bytes for
 *     e4m3 key tables), bf16 tensors passed as raw 16-bit storage;
 *   - `stream` is a hipStream_t (the caller's current stream); nothing synchronises, nothing allocates: scratch
 *     memory is a caller-provided workspace sized by the matching *_workspace_bytes query;
 *   - every call is legal under stream capture;
 *   - return value: 0 on success, otherwise a hipError_t code (hipErrorInvalidValue = 1 for rejected shapes).
 * The Python shims in dsv41_amd/ keep the reference's call signatures and raise RuntimeError on a non-zero code
 * (the reference's launch helper does the same, dsv41/cukern.py:19-21, :34-57).
 */
#ifndef DSV41_HIP_H
#define DSV41_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------------ attention */

/* Workspace bytes for R query rows x H heads over L key positions with output width dv (0 when one split covers
 * a row).  want_nsplit <= 0 lets the library choose the split count; pass the same value to the launch.  The
 * workspace opens with split arrival counters (placed by R and H only): allocate it zeroed once per (R, H); every
 * launch leaves the counters ready for the next, whatever its split count (launches sharing it must be
 * stream-ordered).  Its first int32 is an error word: a decode-kernel launch whose in-launch split merge stopped
 * waiting for the other workgroups of its unit (they were not resident at once) sets it to 1, one whose
 * last-arrival merge ran off its unit's XCD (workgroups not dealt to the XCDs round-robin) sets it to 2 -- that
 * launch's output is then unreliable; the caller polls and clears it (the Python shims do with
 * DSV41_CHECK_ERRORS=1).  DSV41_ATTN_DEC32=0 in the environment selects the 16-head decode kernel over the 32-head
 * one (query the workspace size under the same setting: a launch given too small a workspace returns an error). */
long dsv41_attn_workspace_bytes(int R, int H, int L, int dv, int want_nsplit);

/* kernels.sparse_attn (dsv41/kernels.py:172-256) and fused.sparse_attn_decode (dsv41/fused.py:269-280).
 * q [b, s, h, dqk] bf16; kv [b, n_kv, dqk] bf16 (slot stride kv_bstride); idx [b, s, t] int32, -1 or >= n_kv =
 * empty; sink [h] fp32; out [b, s, h, dv] bf16 (V = the first dv columns of each kv row). */
int dsv41_sparse_attn(const void* q, const void* kv, const float* sink, const int* idx, void* out, int b, int s, int h,
                      int dqk, int dv, int n_kv, long kv_bstride, int t, float scale, int want_nsplit, void* ws,
                      long ws_bytes, void* stream);

/* dsv41_sparse_attn over two KV sources without concatenating them: index i < n_kv reads kv[i], n_kv <= i < n_kv + n2
 * reads kv2[i - n_kv] (the reference's torch.cat of the window and compressed rows and of their index lists before
 * kernels.sparse_attn, dsv41/model.py:1442-1443); idx rows have stride idx_rstride >= t. */
int dsv41_sparse_attn_kv2(const void* q, const void* kv, const void* kv2, const float* sink, const int* idx, void* out,
                          int b, int s, int h, int dqk, int dv, int n_kv, long kv_bstride, int n2, long kv2_bstride,
                          int t, long idx_rstride, float scale, int want_nsplit, void* ws, long ws_bytes,
                          void* stream);

/* fused.sparse_attn_decode2 / sparse_attn_decode_split (dsv41/fused.py:352-403, :406-472): one query per batch
 * row; index < n1 reads kv1[b, index], otherwise kv2[b, index - n1]. */
int dsv41_sparse_attn2(const void* q, const void* kv1, const void* kv2, const float* sink, const int* idx, void* out,
                       int b, int h, int d, int n1, long kv1_bstride, int n2, long kv2_bstride, int t, float scale,
                       int want_nsplit, void* ws, long ws_bytes, void* stream);

/* fused2.sattn2 (dsv41/fused2.py:334-446): query row b at position pos[b] of sequence seq[b] over that sequence's
 * SWA ring kv_win[seq, 0..win) (slot validity from pos/pmax/plim, dsv41/fused2.py:355-360) and the compressed rows
 * kv_c[seq, idx[b, :]]; LSE combine with the sink, bf16 round, inverse rope on the last rd output columns (rd = 0:
 * none).  dqk = 512 with dv = 512 is the reference geometry (K = V = the row); dqk = 576, dv = 512 is absorbed MLA
 * (V = the 512 latent columns).  plim may be null (= pos). */
int dsv41_sattn2(const void* q, const void* kv_win, long win_sstride, int win, const void* kv_c, long c_sstride,
                 int n_c_rows, const int* idx, int t, const long* pos, const long* seq, const long* pmax,
                 const long* plim, const float* sink, const float* cos_t, const float* sin_t, int rd, float scale,
                 void* out, int B, int h, int dqk, int dv, int want_nsplit, void* ws, long ws_bytes, void* stream);

/* Size of the static device scratch of dsv41_sattn2_noalloc (bytes, per device). */
#define DSV41_SCRATCH_BYTES (16L << 20)

/* No counterpart in the reference: dsv41_sattn2 for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and results as dsv41_sattn2 without the
 * workspace: the split partials and counters live in a static __device__ array of DSV41_SCRATCH_BYTES per device
 * (held until the process ends; its address is taken with hipGetSymbolAddress on the first call on each device).
 * Calls whose workspace (dsv41_attn_workspace_bytes for the same R, H, L, dv, want_nsplit) exceeds
 * DSV41_SCRATCH_BYTES return hipErrorOutOfMemory: pass a smaller want_nsplit (1 needs none).  Every call on a device
 * shares that device's array: calls that overlap on one device (different streams, or several threads without
 * stream order) race.  The split counters are cleared by a fill kernel at the start of every call that uses them;
 * the cooperative-merge error word of dsv41_attn_workspace_bytes' layout is not reported by this variant.
 * Allocates nothing (no hipMalloc / hipFree). */
int dsv41_sattn2_noalloc(const void* q, const void* kv_win, long win_sstride, int win, const void* kv_c,
                         long c_sstride, int n_c_rows, const int* idx, int t, const long* pos, const long* seq,
                         const long* pmax, const long* plim, const float* sink, const float* cos_t, const float* sin_t,
                         int rd, float scale, void* out, int B, int h, int dqk, int dv, int want_nsplit,
                         void* stream);

/* ------------------------------------------------------------------------------------------------ compressor */

/* Compressor pooling of the decode step, DecodeRuntime.compressor2 (dsv41/decode.py:243-265) after the wkv / wgate
 * projections: row r (position pos[r] of sequence seq[r]) writes kv[r], score[r] (fp32 [B, D], row stride x_rstride)
 * to ring slot pos % ring of ring_kv / ring_sc ([S, ring, D] fp32, sequence stride ring_sstride; initialise kv 0 and
 * score -inf), then pools the group of the `ratio` positions ending at pos[r] from the ring: per channel
 * sum_q kv[q] softmax_q(score[q]), cast to bf16, rmsnorm(norm_w bf16 [D], eps) -> latent[r] bf16; should[r] (bytes)
 * = (pos + 1) % ratio == 0.  Two launches (all ring writes before any pooling: drafts of one sequence see each other).
 * D <= 1024, 1 <= ratio <= min(16, ring). */
int dsv41_compress_pool_decode(const float* kv, const float* score, long x_rstride, float* ring_kv, float* ring_sc,
                               long ring_sstride, int ring, const long* pos, const long* seq, int B, int D, int ratio,
                               const void* norm_w, float eps, void* latent, long lat_rstride, void* should,
                               void* stream);

/* Compressor pooling of a prefill chunk, Compressor.__call__ (dsv41/model.py:593-660) after the projections, for one
 * sequence: positions start_pos .. start_pos + n_rows - 1 with kv / score fp32 [n_rows, D]; every group of `ratio`
 * positions that closes inside the chunk (n_groups of them, checked) is pooled as above into latent[g] (members before
 * start_pos from the ring: the continuation's partial group, :600-606); then the chunk's last min(n_rows, ring)
 * positions go to the ring ([ring, D] fp32 each). */
int dsv41_compress_pool_prefill(const float* kv, const float* score, long x_rstride, float* ring_kv, float* ring_sc,
                                int ring, long start_pos, int n_rows, int D, int ratio, const void* norm_w, float eps,
                                void* latent, long lat_rstride, int n_groups, void* stream);

/* ------------------------------------------------------------------------------------------------ indexer */

/* fused3.index_score (dsv41/fused3.py:20-62) and the score half of Indexer.__call__ (dsv41/model.py:766-893):
 * out[r, t] = sum_h w[r,h] * relu(q[r,h,:] . key[slot(r), t, :]) for t < cl(r), -inf for cl(r) <= t < n_pos when
 * write_masked.  kfmt 0: keys bf16 [S, rows, 128] (k_sstride in elements), q bf16 [R, HI, 128] (q_rstride in
 * elements), w fp32 [R, HI].  kfmt 1: keys e4m3 [S, rows, 128] (k_sstride in bytes) times kscale [S, rows] fp32;
 * q and w are the prepared e4m3 queries [R, 64, 128] (q_rstride in bytes) and folded weights [R, 64] of
 * dsv41_index_qprep / dsv41_decode_appends.  HI <= 64.
 * slot(r) = seq[r] (or r / rows_per_slot when seq is null); cl(r) = cl[r] (or (cl_start + r % rows_per_slot + 1) /
 * cl_ratio, the causal compressed length of a prefill chunk, dsv41/model.py:819-830, when cl is null).
 * hist (may be null): [R, 4096] int32 histogram of the top 12 bits of the order-preserving key of every score
 * written (t < cl), accumulated atomically -- the input of dsv41_select_topk; it must be zero on entry.
 * cand (may be null): candidate mask [R, >= n_pos] bytes (row stride cand_rstride; nonzero = candidate), the CAND
 * argument of dsv41/fused3.py:20-41 and the consumer mask of dsv41/model.py:854-866: t < cl(r) that is not a
 * candidate scores -inf (and is still a valid position for the top-k). */
int dsv41_index_score(const void* q, long q_rstride, const float* w, long w_rstride, int R, int HI, int D, int kfmt,
                      const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                      int rows_per_slot, const long* cl, long cl_start, int cl_ratio, int n_pos, int write_masked,
                      float* out, long out_rstride, int* hist, const void* cand, long cand_rstride, void* stream);

/* Index-query preparation for the e4m3 score path (the query side of dsv41/decode.py:284-288 after the reference's
 * FP4 rounding): per (row, head) a power-of-two scale 2^e = 2^ceil(log2(amax/448)), q8 = e4m3(q / 2^e) and
 * wf = w * 2^e.  q bf16 [R, HI, 128], w fp32 [R, HI] -> q8 [R, 64, 128] bytes, wf [R, 64] (heads >= HI: weight 0). */
int dsv41_index_qprep(const void* q, const float* w, int R, int HI, void* q8, float* wf, void* stream);

/* Workspace of dsv41_select_topk for R rows of n positions; its first R*4096 int32 are the histogram that
 * dsv41_index_score fills.  Allocate it zeroed once: every dsv41_select_topk call leaves the histogram zeroed. */
long dsv41_select_workspace_bytes(int R, int n);

/* Decode top-k (the topk_indices of dsv41/fused3.py:65-75 after fused3.index_score, dsv41/decode.py:289-294) from
 * the scores and the histogram built by dsv41_index_score: per row the k largest of score[r, 0..cl[r]), ascending,
 * + offset, -1 padding when cl[r] < k; ties lowest index first (the same set as dsv41_topk_indices).  Two launches
 * (per-chunk compaction over many workgroups, then one workgroup per row); n <= 262144, k <= n. */
int dsv41_select_topk(const float* score, long ld, int R, int n, int k, const long* cl, int offset, void* ws,
                      long ws_bytes, int* out, long out_rstride, void* stream);

/* Workspace of dsv41_index_select for R rows of n_pos positions (8-byte aligned: the histogram and count words take
 * 64-bit atomics; a misaligned workspace is rejected).  Allocate it zeroed once per (R, n_pos): every
 * call leaves its histogram zeroed and its per-chunk count words (which carry the launch epoch) consistent for the
 * next call (calls sharing it must be stream-ordered). */
long dsv41_index_select_workspace_bytes(int R, int n_pos);

/* The decode indexer in one launch: fused3.index_score followed by fused3.topk_indices (dsv41/decode.py:284-294;
 * scores as dsv41/fused3.py:20-62, selection as dsv41/fused3.py:65-75).  q8/wf: the prepared e4m3 queries and folded
 * weights of dsv41_index_qprep; keys: e4m3 [S, n_pos, 128] with fp32 per-row scales; row r uses slot seq[r] and
 * positions 0..cl[r).  out [R, k]: the k largest scores' positions, ascending, + offset, -1 padding when cl[r] < k;
 * ties lowest index first (the set of dsv41_topk_indices on the same scores).  score_out (may be null): the scores,
 * -inf for cl[r] <= t < n_pos.  Needs R * ceil(n_pos / 512) <= 512 workgroups (resident together: the rows'
 * workgroups meet at two barriers) and n_pos <= 262144; otherwise hipErrorInvalidValue (use dsv41_index_score +
 * dsv41_select_topk).  n_pos may be less than the key table's rows (the decode tables' spare last row is never
 * valid); a cl[r] > n_pos is clamped to n_pos and sets the workspace's last-but-three int32 to 2.  A barrier wait
 * that gives up (a workgroup never arrived) sets it to 1.  cand (may be null): candidate mask as in
 * dsv41_index_score (dsv41/decode.py:311-315). */
int dsv41_index_select(const void* q8, long q_rstride, const float* wf, long w_rstride, int R, int HI,
                       const void* keys, long k_sstride, const float* kscale, long ks_sstride, const long* seq,
                       const long* cl, int n_pos, int k, int offset, void* ws, long ws_bytes, float* score_out,
                       long score_rstride, int* out, long out_rstride, const void* cand, long cand_rstride,
                       void* stream);

/* The decode step's cache appends and the one-launch indexer in one launch: the operations of dsv41_decode_appends
 * (the SWA ring row, the compressed row and the index-key row of every row, dsv41/decode.py:129-164, :270-282; the
 * e4m3 preparation of the index queries q_idx [R, HI, 128] / w_idx [R, HI] bf16) followed by dsv41_index_select over
 * the e4m3 key table k8 / ks, the new key of a row whose step closes a group included (it is scored from the
 * values this launch computes).  Same results as dsv41_decode_appends followed by dsv41_index_select.  Every row
 * must belong to a different sequence (seq distinct: a row's new key is not visible to other rows of the launch);
 * the index-key width is 128; nw_tab (may be null) as in dsv41_decode_appends; limits and workspace as
 * dsv41_index_select. */
int dsv41_decode_select(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                        const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                        const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                        long ks_sstride, int kcap, const long* pos, const long* seq, const long* nw_tab, int R,
                        int ratio, const float* cos_t, const float* sin_t, int rd, float eps, const void* q_idx,
                        const void* w_idx, int HI, const long* cl, int n_pos, int k, int offset, void* ws,
                        long ws_bytes, float* score_out, long score_rstride, int* out, long out_rstride,
                        const void* cand, long cand_rstride, void* stream);

/* The decode step's cache appends and the indexer scores with their histogram in one launch, for rows longer than
 * dsv41_decode_select's one launch takes (the multi-launch decode indexer, dsv41/decode.py:106-174 with :284-294):
 * the operations of dsv41_decode_appends (ring row, compressed row, index-key row; the e4m3 query preparation in
 * the launch) followed by dsv41_index_score over the e4m3 key table k8 / ks with the row histogram hist [R, 4096]
 * (zero on entry; dsv41_select_topk leaves it zero), scores into score [R, n_pos] for positions < cl[r]; the new key
 * of a row whose step closes a group is scored from the values this launch computes.  Same results as
 * dsv41_decode_appends followed by dsv41_index_score (e4m3 keys, with the histogram).  Rows must belong to distinct
 * sequences (a row's new key is not visible to other rows of the launch); index-key width 128, HI <= 64; nw_tab
 * (may be null) as in dsv41_decode_appends. */
int dsv41_decode_score(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                       const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                       const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                       long ks_sstride, int kcap, const long* pos, const long* seq, const long* nw_tab, int R,
                       int ratio, const float* cos_t, const float* sin_t, int rd, float eps, const void* q_idx,
                       const void* w_idx, int HI, const long* cl, int n_pos, float* score, long score_rstride,
                       int* hist, const void* cand, long cand_rstride, void* stream);

/* Workspace of dsv41_candidate_blocks (block maxima and the selected blocks of every row). */
long dsv41_candidate_blocks_workspace_bytes(int R, int n, int topk_blocks, int block_size);

/* select_candidate_blocks (dsv41/model.py:256-265) on the masked scores of the candidate source layer
 * (dsv41/model.py:838-852, dsv41/decode.py:309-313): per row r the maxima of score[r, b*bs .. (b+1)*bs) over
 * positions < cl(r) (others count as -inf), the block of position cl(r) - 1 forced to +inf, the topk_blocks largest
 * blocks kept when their value is finite (ties: lowest block first; the reference leaves them unspecified), expanded
 * to mask[r, 0 .. width) bytes (1 = candidate) -- the block covering t, also past n.  cl(r) = cl[r], or
 * (cl_start + r % rows_per_seq + 1) / cl_ratio when cl is null.  score: fp32 [R, >= n] (row stride ld), n <= width. */
int dsv41_candidate_blocks(const float* score, long ld, int R, int n, int width, const long* cl, long cl_start,
                           int cl_ratio, int rows_per_seq, int topk_blocks, int block_size, void* mask,
                           long mask_rstride, void* ws, long ws_bytes, void* stream);

/* fused3.topk_indices + cuda/topk_select.cu (dsv41/fused3.py:65-75, dsv41/cuda/topk_select.cu:94-168), also the
 * selection of Indexer.__call__ (dsv41/model.py:868-893): per row the k largest of score[r, 0..c) with c =
 * min(cl(r), n), ascending, + offset; positions past the selection (c < k) are -1.  Ties: lower index first. */
int dsv41_topk_indices(const float* score, long ld, int R, int n, int k, const long* cl, long cl_start, int cl_ratio,
                       int rows_per_seq, int offset, int* out, long out_rstride, void* stream);

/* ------------------------------------------------------------------------------------------------ appends */

/* fused2.kv_write (dsv41/fused2.py:276-330) and the ring commit of Attention._window_kv (dsv41/model.py:1057-1298):
 * row r of x -> rmsnorm(w) -> bf16 -> rope(last rd, position p) -> bf16 -> fq8/32 -> cache[s, p % W] (rows r >=
 * commit_from only) and tmp[r] (when tmp != null).  p = pos[r] or pos0 + (r % rows_per_seq) * pos_stride; s = seq[r] or
 * r / rows_per_seq. */
int dsv41_kv_write(const void* x, long x_rstride, const void* w, const float* cos_t, const float* sin_t,
                   const long* pos, const long* seq, long pos0, long pos_stride, int rows_per_seq, void* cache,
                   long cache_sstride, int W, void* tmp, int n_rows, int D, int rd, float eps, int commit_from,
                   void* stream);

/* Attention._window_kv for a prefill chunk of one sequence (dsv41/model.py:1057-1298, the continuation copy
 * :1170-1298): out = [history | chunk] with history = ring rows of positions start_pos - hist .. start_pos - 1
 * (copied out before the commit), chunk row r = fq8(rope(rmsnorm(x[r]))) at position start_pos + r; the last
 * min(n_rows, W) chunk rows are committed to ring[(start_pos + r) % W].  ring is the sequence's [W, D] block, out
 * [hist + n_rows, D]; 0 <= hist <= min(start_pos, W - 1). */
int dsv41_window_kv(const void* x, long x_rstride, const void* w, const float* cos_t, const float* sin_t,
                    long start_pos, int n_rows, void* ring, int W, void* out, int hist, int D, int rd, float eps,
                    void* stream);

/* Compressed-KV append (dsv41/decode.py:157-164, dsv41/model.py:1320-1348, SharedAttn.write_compress_kv :508-541)
 * and index-key append (dsv41/decode.py:270-282, dsv41/model.py:696-732, SharedAttn.write_index_k :543-574):
 * row r of x -> [rmsnorm(norm_w)] -> [rope(last rd) at (pos[r] or pos0 + (r % rows_per_seq)*pos_stride) + pos_add] -> fake quant
 * (qmode 0 fp8 pow2, 1 fp4 pow2, 2 fp4 e4m3-scale; group 16/32; -1 none) -> bf16 cache[s, row] with s = seq[r] or
 * r / rows_per_seq and row = row[r] or row0 + r % rows_per_seq (row < 0: no write).  When k8 != null also writes
 * the e4m3 encoding with a per-row power-of-two scale: k8[s, row, :] (bytes) and ks[s, row]. */
int dsv41_append_rows(const void* x, long x_rstride, const void* norm_w, float eps, const float* cos_t,
                      const float* sin_t, int rd, const long* pos, long pos0, long pos_stride, long pos_add,
                      const long* seq, int rows_per_seq, const long* row, long row0, void* cache, long cache_sstride,
                      int qmode, int group, void* k8, long k8_sstride, float* ks, long ks_sstride, int n_rows, int D,
                      void* stream);

/* All cache writes of one decode step in one launch (dsv41/decode.py:129-164 kv_write + compressed append,
 * :270-282 index-key append, :176-181 spare row), plus the index-query preparation: per query row r at position
 * pos[r] of sequence seq[r]
 *   ring[seq, pos % W]        <- fq8(rope(rmsnorm(kv_raw[r], kv_norm)))                       (Dw wide)
 *   ckv[seq, row]             <- fq4/16-e4m3(rope(latent[r], pos + 1 - ratio))                (latent may be null)
 *   kbf[seq, row], k8/ks      <- fq4/32(rope(rmsnorm(k_raw[r], k_norm), pos + 1 - ratio))     (Dk = 128; k_raw may be
 *                                                                                               null; kbf or k8 may be null)
 *   q8[r], wf[r]              <- dsv41_index_qprep(q_idx[r], w_idx[r] (bf16))                  (q_idx may be null)
 * with row = (pos + 1) / ratio - 1 when (pos + 1) % ratio == 0, else the no-write row of the sequence: nw_tab[seq]
 * when nw_tab (int64 [S]) is given -- the reference's per-slot table under DSV41_SLOT_CAPS, the last row of each
 * slot's own capacity (dsv41/decode.py:62-68, :176-181), needed when the tables are as_strided views whose slot
 * stride is smaller than their row count (dsv41/slots.py:1-11) -- else the table's spare last row (cap - 1 /
 * kcap - 1).  Both tables take the same row (the reference passes one row to both appends, :157-164, :270-282). */
int dsv41_decode_appends(const void* kv_raw, const void* kv_norm, void* ring, long ring_sstride, int W, int Dw,
                         const void* latent, void* ckv, long ckv_sstride, int cap, const void* k_raw,
                         const void* k_norm, void* kbf, long kbf_sstride, void* k8, long k8_sstride, float* ks,
                         long ks_sstride, int kcap, int Dk, const long* pos, const long* seq,
                         const long* nw_tab, int ratio, const float* cos_t, const float* sin_t, int rd, float eps,
                         const void* q_idx, const void* w_idx, int HI, void* q8, float* wf, int B, void* stream);

/* Index-key table conversion for cache snapshots (dsv41/engine.py:1072-1230 copies the cache tensors as they are;
 * the reference's index_k is bf16 [.., 128], this build's e4m3 + fp32 per-row power-of-two scale): encode rows of
 * 128 bf16 (the key appends' encoding: scale 2^ceil(log2(amax / 448)), amax >= 1e-30, exponent >= -126) and decode
 * (e4m3 x scale, rounded to bf16).  decode(encode(k)) == k for the FP4-grid rows the reference stores. */
int dsv41_index_keys_encode(const void* kbf, long n_rows, void* k8, float* ks, void* stream);
int dsv41_index_keys_decode(const void* k8, const float* ks, long n_rows, void* kbf, void* stream);

/* ------------------------------------------------------------------------------------------------ projections */

/* Workspace bytes of dsv41_fp8_gemm for M rows, N columns, K (0 when no K split is planned).  Allocate it zeroed
 * once per shape: every launch leaves its arrival counters at zero (launches sharing it must be stream-ordered). */
long dsv41_fp8_gemm_workspace_bytes(int M, int N, int K);

/* fp8_gemm_tc / fp8_gemv_m1 (dsv41/cukern.py:116-200; weight format dsv41/w8.py:19-60): out[m, n] =
 * sum_k x[row(m, n), k] * e4m3(w8[n, k]) * 2^(s8[n / 32, k / 32] - 127), bf16 x (row stride ldx), fp32
 * accumulation, bf16 out [M, ldo] (and fp32 out_f32 [M, ldo] when not null).  w8: e4m3 bits [N, K] with every 16-k
 * group in the PERM_K byte order; s8: E8M0 [ceil(N / 32), Kc], Kc >= K / 32.  row(m, n) = m, or with group_cols > 0
 * (block-diagonal, dsv41/w8.py oproj_a) m * (N / group_cols) + n / group_cols.  K % 64 == 0; group_cols % 64 == 0;
 * x 4-byte and w8 16-byte aligned.  The weights stream once per 64 rows of M.  With x 16-byte aligned and ldx % 8 ==
 * 0, up to 16 rows over 1024-4096 columns (up to 4 rows over at most 4096 columns) run without a K split (faster for
 * the decode GEMVs; the workspace is then unused). */
int dsv41_fp8_gemm(const void* x, long ldx, const void* w8, const void* s8, int M, int N, int K, int Kc,
                   int group_cols, void* out, long ldo, float* out_f32, void* ws, long ws_bytes, void* stream);

/* fp8_gemv_m1_pre (dsv41/cukern.py:137-158): one launch, the activation prologue fused into the x staging of the
 * 64-column kernel: x = fake_quant_fp8(bf16(rmsnorm(x_raw) * norm_w), 32) (mode 1) or fake_quant_fp8(x_raw, 32)
 * (mode 2; norm_w unused), then out[0, n] as dsv41_fp8_gemm for one row.  x_raw bf16 [K] and norm_w 16-byte
 * aligned, K % 64 == 0, K <= 16384; the same results as dsv41_norm_quant followed by dsv41_fp8_gemm on the 64-column
 * kernel.  Workspace: dsv41_fp8_gemm_workspace_bytes(1, N, K). */
int dsv41_fp8_gemv_m1_pre(const void* x_raw, const void* norm_w, float eps, int mode, const void* w8, const void* s8,
                          int N, int K, int Kc, void* out, void* ws, long ws_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------ numerics */

/* norm_quant (dsv41/fused2.py:251-272): per row of D bf16 values (D % 32 == 0, D <= 16384; x and y 16-byte aligned,
 * rows contiguous) y = fake_quant_fp8(bf16(rmsnorm(x) * w), 32); with w null the fake quantisation alone
 * (dsv41/fused.py:83-84 at any such D).  The activation prologue of fp8_gemv_m1_pre (dsv41/cukern.py:137-158). */
int dsv41_norm_quant(const void* x, const void* w, float eps, void* y, long n_rows, int D, void* stream);

/* fake_quant_fp8 / fake_quant_fp4 (dsv41/fused.py:46-87, dsv41/quant.py:45-87) on rows of D bf16 values. */
int dsv41_fake_quant(const void* x, void* y, long n_rows, int D, int group, int mode, void* stream);

/* rope_ / rope_dev_ (dsv41/fused.py:203-234, :319-349): in place on the last rd of each row of x [n_rows, D]
 * (rows ordered (b, s, h)); position = (pos ? pos[b] + add : pos0) + s * pos_stride. */
int dsv41_rope(void* x, const float* cos_t, const float* sin_t, const long* pos, long pos0, long add, long pos_stride,
               long n_rows, int H, int S, int D, int rd, int inverse, void* stream);

/* rmsnorm (dsv41/fused.py:91-109): y = x / sqrt(mean(x^2) + eps) * w, bf16 rows of D <= 1024, or of D <= 16384 with
 * D % 32 == 0 and x, y 16-byte aligned. */
int dsv41_rmsnorm(const void* x, const void* w, void* y, long n_rows, int D, float eps, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DSV41_HIP_H */
