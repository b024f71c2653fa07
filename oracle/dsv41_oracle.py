"""CPU oracle for the DeepSeek-V4.1 sparse-attention hot path (numpy, float32).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module: only tests/, the smoke() check of
__graft_entry__.py and the cpu_baseline leg of bench.py use it, and only as the checker (or, in bench.py, as the
CPU baseline that is timed beside the GPU).  The product path raises when the HIP library is missing.

Every function restates one piece of the reference's arithmetic and cites the reference file:line it follows
(paths relative to the reference repository root).  How each function is pinned (known answers, closed forms,
brute force, library routines) is listed in PINNING below and exercised in tests/test_oracle.py.

Precision conventions follow the reference:
  * bf16 storage is emulated with round-to-nearest-even on float32 bit patterns (bf16()).
  * decode kernels (Triton, fused.py / fused2.py) keep QK and PV in fp32;
  * kernels.sparse_attn (prefill, torch) rounds the QK einsum and the PV einsum to bf16 (its einsums run in bf16).
"""
from __future__ import annotations

import numpy as np

PINNING = {
    "bf16": "bit pattern identity vs torch.bfloat16 cast (library routine), tests/test_oracle.py",
    "round_e4m3": "every e4m3 value is a fixed point; vs torch.float8_e4m3fn cast on 65536 random values",
    "round_e2m1": "known answers dsv41/test_kernels.py:51-55 (0.75,1.25,1.75,2.5,3.5,5)->(1,1,2,2,4,4); grid fixed points",
    "fake_quant_fp8": "closed form of dsv41/quant.py:45-53 vs torch float8 cast composition; idempotence",
    "fake_quant_fp4": "closed form of dsv41/quant.py:75-87 vs torch composition; idempotence; grid membership",
    "rope": "rope(inverse) o rope = id; vs complex rotation (apply_rotary_emb, dsv41/model.py:118-129)",
    "window_idx": "ring closed form == brute-force enumeration of positions (dsv41/model.py:132-254, fused2.py:359-360)",
    "sparse_attn": "dense masked softmax with the sink as an extra logit dropped after softmax (dsv41/test_kernels.py:33-49)",
    "sattn2": "split/online merge == single pass; == sparse_attn_decode over [ring | compressed] + inverse rope "
              "(dsv41/test_fused2_units.py:50-68)",
    "index_score": "brute-force per-head loop; chunked == full exactly (dsv41/test_long_prefill.py:66-96)",
    "topk": "brute force: sorted(range(n), key=(-score, index))[:k] on small n; ascending + -1 mask",
    "kv_write": "composition rmsnorm -> bf16 -> rope -> bf16 -> fq8 (dsv41/test_fused2_units.py:39-49)",
    "fp8_key_encode": "exact round trip of FP4-grid rows through e4m3 + per-row pow2 scale (closed-form argument)",
    "window_kv": "brute force: histories == the last rows produced before each chunk; ring == the last W rows",
    "compress_pool": "fed as any mix of prefill chunks and single decode rows, every closed group's latent equals the "
                     "one-call start_pos 0 result; equal gate scores give the group mean, one dominant score gives that "
                     "member; vs torch.softmax composition (library routine)",
    "e4m3_decode": "all 256 codes vs torch.float8_e4m3fn -> float32 cast (library routine)",
    "AttentionLayer": "composition of the pinned functions above; chunk invariance: a sequence fed as one chunk or as "
                      "several continuation chunks gives the same outputs and caches (the reference's procedure, "
                      "dsv41/test_long_prefill.py:66-96), tests/test_oracle.py",
    "indexer_query": "composition of fake_quant_fp8, rope and fake_quant_fp4 (pinned above); the query side of "
                     "AttentionLayer's chunk-invariance check",
    "linear_fp8": "composition of fake_quant_fp8 (pinned) and a library matmul",
    "fp8_gemm": "vs torch matmul of the dequantised weight (library routine, exact products); PERM_K round trip "
                "(known list dsv41/w8.py:23); block-diagonal == the dense product with the off-group blocks zeroed",
    "select_candidate_blocks": "properties of the top blocks (forced last block, count, every kept block max >= every "
                               "dropped finite one, whole blocks); indexer with candidates chunked == full exactly "
                               "(dsv41/test_long_prefill.py:66-96)",
}


# ----------------------------------------------------------------------------------------------- scalar formats
def bf16(x) -> np.ndarray:
    """Round float32 to bfloat16 (RNE), returned as float32.  torch's bf16 cast (library routine)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)  # wraps only for NaN patterns, which are restored below
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, a, out)
    return out.reshape(a.shape)


def ceil_log2(a: np.ndarray) -> np.ndarray:
    """ceil(log2(a)) for a > 0, exact via the fp32 bit pattern (dsv41/fused.py:10-16, dsv41/quant.py:34-37)."""
    bits = np.asarray(a, np.float32).view(np.int32)
    e = ((bits >> 23) & 0xFF) - 127
    mant = bits & 0x7FFFFF
    return e + (mant != 0).astype(np.int32)


def pow2i(e: np.ndarray) -> np.ndarray:
    """2^e for integer e in the normal fp32 range (dsv41/fused.py:19-21)."""
    return ((np.asarray(e, np.int32) + 127) << 23).astype(np.int32).view(np.float32)


def round_e4m3(v: np.ndarray) -> np.ndarray:
    """Nearest float8_e4m3fn value, ties to even, |v| <= 448 (dsv41/fused.py:24-34)."""
    v = np.asarray(v, np.float32)
    a = np.abs(v)
    bits = a.view(np.int32)
    e = ((bits >> 23) & 0xFF) - 127
    e = np.maximum(e, -6)
    ulp = pow2i(e - 3)
    r = (np.rint(a / ulp) * ulp).astype(np.float32)
    r = np.minimum(r, np.float32(448.0))
    return np.where(v < 0, -r, r).astype(np.float32)


def round_e2m1(v: np.ndarray) -> np.ndarray:
    """Nearest E2M1 value {0,.5,1,1.5,2,3,4,6}, ties to even (dsv41/quant.py:67-71, dsv41/fused.py:37-43)."""
    v = np.asarray(v, np.float32)
    a = np.abs(v)
    r = np.where(a < 2.0, np.rint(a * 2.0) / 2.0, np.where(a < 4.0, np.rint(a), np.rint(a / 2.0) * 2.0))
    r = np.minimum(r, 6.0).astype(np.float32)
    return np.where(v < 0, -r, r).astype(np.float32)


def fake_quant_fp8(x: np.ndarray, block: int = 32) -> np.ndarray:
    """Per-`block` FP8 fake quant with a power-of-two scale (dsv41/quant.py:45-53; dsv41/fused2.py:26-32).
    Returns float32 values on the e4m3 grid times the scale (caller rounds to the storage dtype)."""
    x = np.asarray(x, np.float32)
    g = x.reshape(-1, block)
    amax = np.maximum(np.abs(g).max(axis=1, keepdims=True), np.float32(1e-4))
    s = pow2i(ceil_log2((amax / np.float32(448.0)).astype(np.float32)))
    q = round_e4m3(np.clip(g / s, -448.0, 448.0))
    return (q * s).astype(np.float32).reshape(x.shape)


def fake_quant_fp4(x: np.ndarray, block: int = 32, scale_e4m3: bool = False) -> np.ndarray:
    """E2M1 values with a pow2 (E8M0) or e4m3-rounded scale per group (dsv41/quant.py:75-87, dsv41/fused.py:53-70)."""
    x = np.asarray(x, np.float32)
    g = x.reshape(-1, block)
    amax = np.abs(g).max(axis=1, keepdims=True)
    if scale_e4m3:
        amax = np.maximum(amax, np.float32(6 * 2.0 ** -9))
        s = round_e4m3((amax / np.float32(6.0)).astype(np.float32))
    else:
        amax = np.maximum(amax, np.float32(6 * 2.0 ** -126))
        s = pow2i(ceil_log2((amax / np.float32(6.0)).astype(np.float32)))
    q = round_e2m1(np.clip((g / s).astype(np.float32), -6.0, 6.0))
    return (q * s).astype(np.float32).reshape(x.shape)


def key_encode_fp8(k: np.ndarray):
    """Per-row e4m3 + fp32 pow2 scale encoding of an index-key row (this build's storage format for the indexer keys;
    the reference stores FP4-grid values in bf16, dsv41/model.py:726).  scale = 2^ceil(log2(amax/448)), amax >= 1e-30.
    Returns (float32 e4m3-grid values, float32 scale[..., 1])."""
    k = np.asarray(k, np.float32)
    amax = np.maximum(np.abs(k).max(axis=-1, keepdims=True), np.float32(1e-30))
    s = pow2i(np.maximum(ceil_log2((amax / np.float32(448.0)).astype(np.float32)), -126))
    q = round_e4m3(np.clip(k / s, -448.0, 448.0))
    return q, s.astype(np.float32)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """y = x * (1/sqrt(mean(x^2) + eps)) * w in fp32 (dsv41/fused.py:91-100, dsv41/fused2.py:281-287)."""
    x = np.asarray(x, np.float32)
    var = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return (x * inv * np.asarray(w, np.float32)).astype(np.float32)


# ----------------------------------------------------------------------------------------------- rotary
def rope_tables(dim: int, seqlen: int, original_seq_len: int, base: float, factor: float, beta_fast: float,
                beta_slow: float):
    """cos/sin [seqlen, dim/2] fp32 (dsv41/model.py:62-74, 76-117), YaRN-corrected frequencies."""
    import math
    freqs = (1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float32) / dim))).astype(np.float32)
    if original_seq_len > 0:
        def corrected_dim(rot):
            return dim * math.log(original_seq_len / (rot * 2 * math.pi)) / (2 * math.log(base))
        low = max(math.floor(corrected_dim(beta_fast)), 0)
        high = min(math.ceil(corrected_dim(beta_slow)), dim - 1)
        ramp = np.clip((np.arange(dim // 2, dtype=np.float32) - low) / max(high - low, 1e-3), 0, 1)
        smooth = 1 - ramp
        freqs = (freqs / factor * (1 - smooth) + freqs * smooth).astype(np.float32)
    ang = np.outer(np.arange(seqlen, dtype=np.float32), freqs).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, pos: np.ndarray, rd: int, inverse: bool = False) -> np.ndarray:
    """Rotate the last rd elements of each row (interleaved re/im pairs) at integer position pos (broadcast over
    rows); result rounded to bf16 like the in-place bf16 store (dsv41/fused.py:203-220, 319-335)."""
    x = np.array(x, np.float32, copy=True)
    d = x.shape[-1]
    pos = np.maximum(np.asarray(pos, np.int64), 0)
    c = cos[pos]
    s = sin[pos]
    if inverse:
        s = -s
    xr = x[..., d - rd::2]
    xi = x[..., d - rd + 1::2]
    yr = (xr * c - xi * s).astype(np.float32)
    yi = (xr * s + xi * c).astype(np.float32)
    x[..., d - rd::2] = bf16(yr)
    x[..., d - rd + 1::2] = bf16(yi)
    return x


# ----------------------------------------------------------------------------------------------- window ring
def window_idx(window: int, seqlen: int, start_pos: int) -> np.ndarray:
    """get_window_topk_idxs (dsv41/model.py:132-254): [seqlen, width] int32 physical ring slots (start_pos > 0) or
    temporary-row positions (start_pos == 0), -1 = invalid."""
    if seqlen <= 0:
        return np.zeros((0, 0), np.int32)
    if start_pos == 0:
        q = np.arange(seqlen)[:, None]
        width = min(seqlen, window)
        a = np.maximum(q - window + 1, 0) + np.arange(width)[None, :]
        return np.where(a <= q, a, -1).astype(np.int32)
    q = start_pos + np.arange(seqlen)[:, None]
    a = q - window + 1 + np.arange(window)[None, :]
    valid = (a >= 0) & (a <= q)
    return np.where(valid, a % window, -1).astype(np.int32)


def prefill_window_idx(window: int, seqlen: int, start_pos: int) -> tuple[int, np.ndarray]:
    """Continuation-prefill window indices into the temporary [history | chunk] KV (dsv41/model.py:1170-1240):
    returns (hist_len, idx [seqlen, width])."""
    hist = min(start_pos, window - 1)
    width = min(window, hist + seqlen)
    q = hist + np.arange(seqlen)[:, None]
    first = np.maximum(q - window + 1, 0)
    idx = first + np.arange(width)[None, :]
    return hist, np.where(idx <= q, idx, -1).astype(np.int32)


def ring_valid(pos: int, pmax: int, plim: int, window: int) -> np.ndarray:
    """Validity of every ring slot for a query at pos (dsv41/fused2.py:355-360): held = pmax - ((pmax - slot) mod W),
    valid iff held >= 0, held <= plim and pos - held < W."""
    tt = np.arange(window)
    held = pmax - ((pmax - tt) % window)
    return (held >= 0) & (held <= plim) & (pos - held < window)


# ----------------------------------------------------------------------------------------------- attention
def _attn_rows(q: np.ndarray, rows: np.ndarray, valid: np.ndarray, sink: np.ndarray, scale: float, dv: int,
               prefill_rounding: bool) -> np.ndarray:
    """One query (q [H, Dqk]) against gathered rows [T, Dqk] (V = rows[:, :dv]) with a per-head sink in the
    denominator only.  prefill_rounding: bf16-rounded QK and PV einsums (dsv41/kernels.py:249-254); otherwise fp32
    accumulation as in the Triton decode kernels (dsv41/fused.py:238-266)."""
    H = q.shape[0]
    if rows.shape[0] == 0 or not valid.any():
        return np.zeros((H, dv), np.float32)
    qf = q.astype(np.float32)
    kf = rows.astype(np.float32)
    s = qf @ kf.T
    if prefill_rounding:
        s = bf16(s)
    s = (s * np.float32(scale)).astype(np.float32)
    s = np.where(valid[None, :], s, -np.inf)
    m = np.maximum(s.max(axis=1, keepdims=True), np.float32(-1e30))
    p = np.exp(s - m).astype(np.float32)
    den = p.sum(axis=1, dtype=np.float64).astype(np.float32) + np.exp(sink.astype(np.float32) - m[:, 0])
    num = bf16(p) @ kf[:, :dv]
    if prefill_rounding:
        num = bf16(num)
    return (num / den[:, None]).astype(np.float32)


def sparse_attn(q, kv, sink, idx, scale, dv=None, prefill_rounding=True) -> np.ndarray:
    """kernels.sparse_attn (dsv41/kernels.py:172-256): q [b,s,H,Dqk], kv [b,n,Dqk], idx [b,s,t] (-1 or >= n invalid)
    -> bf16-valued float32 [b,s,H,dv]."""
    q = np.asarray(q, np.float32)
    kv = np.asarray(kv, np.float32)
    b, s, H, d = q.shape
    dv = d if dv is None else dv
    n = kv.shape[1]
    if n <= 0 and s > 0:
        raise RuntimeError("sparse_attn received empty KV with non-empty queries")
    out = np.zeros((b, s, H, dv), np.float32)
    for bi in range(b):
        for si in range(s):
            ix = np.asarray(idx[bi, si]).astype(np.int64)
            valid = (ix >= 0) & (ix < n)
            rows = kv[bi, np.clip(ix, 0, n - 1)]
            out[bi, si] = _attn_rows(q[bi, si], rows, valid, np.asarray(sink), scale, dv, prefill_rounding)
    return bf16(out)


def sattn2(q, kv_win, kv_c, idx, pos, seq, pmax, plim, sink, cos, sin, rd, scale, dv=None) -> np.ndarray:
    """fused2.sattn2 (dsv41/fused2.py:334-446): per query row b, the ring of sequence seq[b] (validity from pos/pmax/
    plim) then the compressed rows idx[b] of kv_c[seq[b]]; LSE combine + sink; bf16 round; inverse rope on the
    last rd (rd = 0: none).  q [B,1,H,Dqk] -> [B,1,H,dv]."""
    q = np.asarray(q, np.float32)
    B, _, H, d = q.shape
    dv = d if dv is None else dv
    W = kv_win.shape[1]
    out = np.zeros((B, 1, H, dv), np.float32)
    for b in range(B):
        sq = int(seq[b])
        vw = ring_valid(int(pos[b]), int(pmax[b]), int(plim[b] if plim is not None else pos[b]), W)
        rows = [np.asarray(kv_win[sq], np.float32)]
        valid = [vw]
        if kv_c is not None and idx is not None:
            ix = np.asarray(idx[b]).reshape(-1).astype(np.int64)
            vc = ix >= 0
            rows.append(np.asarray(kv_c[sq][np.maximum(ix, 0)], np.float32))
            valid.append(vc)
        o = _attn_rows(q[b, 0], np.concatenate(rows), np.concatenate(valid), np.asarray(sink), scale, dv, False)
        o = bf16(o)
        if rd:
            o = rope(o, cos, sin, np.int64(pos[b]), rd, inverse=True)
        out[b, 0] = o
    return out


def sparse_attn_decode2(q, kv1, kv2, sink, idx, scale) -> np.ndarray:
    """fused.sparse_attn_decode2 / sparse_attn_decode_split (dsv41/fused.py:352-472): index < n1 reads kv1, else
    kv2[index - n1]; fp32 accumulation."""
    q = np.asarray(q, np.float32)
    b, _, H, d = q.shape
    n1 = kv1.shape[1]
    out = np.zeros((b, 1, H, d), np.float32)
    for bi in range(b):
        ix = np.asarray(idx[bi]).reshape(-1).astype(np.int64)
        valid = ix >= 0
        r1 = np.asarray(kv1[bi], np.float32)[np.clip(ix, 0, n1 - 1)]
        if kv2 is not None:
            n2 = kv2.shape[1]
            r2 = np.asarray(kv2[bi], np.float32)[np.clip(ix - n1, 0, n2 - 1)]
            rows = np.where((ix < n1)[:, None], r1, r2)
        else:
            rows = r1
        out[bi, 0] = _attn_rows(q[bi, 0], rows, valid, np.asarray(sink), scale, d, False)
    return bf16(out)


# ----------------------------------------------------------------------------------------------- indexer
def index_score(q, index_k, weights, seq, cl, k_scale=None) -> np.ndarray:
    """fused3.index_score (dsv41/fused3.py:20-62): score[b,t] = sum_h w[b,h] relu(q[b,h,:] . k[seq[b],t,:]) in fp32;
    -inf for t >= cl[b].  k_scale [S, n] multiplies each key (fp8 storage); None for bf16 keys."""
    q = np.asarray(q, np.float32).reshape(len(seq), -1, np.asarray(q).shape[-1])
    B, H, D = q.shape
    n = index_k.shape[1]
    w = np.asarray(weights, np.float32).reshape(B, H)
    out = np.empty((B, n), np.float32)
    for b in range(B):
        k = np.asarray(index_k[int(seq[b])], np.float32)
        if k_scale is not None:
            k = k * np.asarray(k_scale[int(seq[b])], np.float32).reshape(-1, 1)
        s = np.maximum(q[b] @ k.T, 0.0)
        sc = (w[b][:, None] * s).sum(axis=0, dtype=np.float64).astype(np.float32)
        sc[np.arange(n) >= int(cl[b])] = -np.inf
        out[b] = sc
    return out


def score_key(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of fp32 (larger float -> larger key; -0.0 folded onto +0.0), the radix-select key
    of dsv41/cuda/topk_select.cu:87-92 with the sign of the order reversed."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).copy()
    u[u == 0x80000000] = 0
    neg = (u & 0x80000000) != 0
    return np.where(neg, ~u, u | 0x80000000).astype(np.uint32)


def topk_indices(score, k: int, cl) -> np.ndarray:
    """fused3.topk_indices + topk_select.cu (dsv41/fused3.py:65-75, dsv41/cuda/topk_select.cu:94-168): the k
    largest per row, ties -> lower index first (this build's declared rule), sorted ascending, -1 where idx >= cl.
    Entries >= cl are never preferred over entries < cl (they carry -inf in the reference)."""
    score = np.asarray(score, np.float32)
    B, n = score.shape
    out = np.full((B, k), -1, np.int32)
    for b in range(B):
        c = int(min(int(cl[b]), n))
        key = score_key(score[b, :c]).astype(np.int64)
        order = np.argsort(-key, kind="stable")
        sel = np.sort(order[:k])
        out[b, :len(sel)] = sel
    return out


def select_candidate_blocks(score, cl, topk_blocks: int, block_size: int) -> np.ndarray:
    """select_candidate_blocks (dsv41/model.py:256-265) on score rows [R, T] whose positions >= cl[r] are masked:
    block maxima over block_size positions (positions >= cl count as -inf), the block of position cl - 1 forced to
    +inf, the min(topk_blocks, n_blocks) largest kept when finite (ties -> lower block, this build's rule), expanded
    to a bool mask [R, T]."""
    score = np.asarray(score, np.float32)
    R, T = score.shape
    nb = -(-T // block_size)
    out = np.zeros((R, T), bool)
    for r in range(R):
        c = int(min(max(int(cl[r]), 0), T))
        m = np.full(nb, -np.inf, np.float32)
        for blk in range(nb):
            seg = score[r, blk * block_size:min((blk + 1) * block_size, c)]
            if seg.size:
                m[blk] = seg.max()
        if c > 0:
            m[(c - 1) // block_size] = np.inf
        order = sorted(range(nb), key=lambda blk: (-m[blk], blk))
        for blk in order[:min(topk_blocks, nb)]:
            if m[blk] > -np.inf:
                out[r, blk * block_size:(blk + 1) * block_size] = True
    return out


def indexer_prefill(q, weights, index_k, start_pos: int, ratio: int, topk: int, offset: int, k_scale=None,
                    query_chunk: int = 64, candidates=None, candidate_source=None):
    """Indexer.__call__ for seqlen > 1 (dsv41/model.py:766-893): score = sum_h w relu(q_h . K^T) per query chunk,
    causal mask t >= (start+i+1)//ratio, [candidate mask], top-min(topk, end//ratio), ascending, +offset, -1 where
    masked.  q [b,s,H,D], weights [b,s,H], index_k [b,T,D] -> int32 [b,s,min(topk,end//ratio)].
    candidates (bool [b, s, >= T], a consumer layer, :854-866): scores of non-candidates are -inf (they stay valid
    positions: the selection takes them last, lowest index first).  candidate_source = (topk_blocks, block_size) (the
    source layer, :838-852): also returns the mask of select_candidate_blocks over the masked scores, [b, s, T]."""
    q = np.asarray(q, np.float32)
    b, s, H, D = q.shape
    kk = min(topk, (start_pos + s) // ratio)
    out = np.full((b, s, kk), -1, np.int32)
    T = np.asarray(index_k).shape[1]
    cmask = np.zeros((b, s, T), bool) if candidate_source is not None else None
    for bi in range(b):
        k = np.asarray(index_k[bi], np.float32)
        if k_scale is not None:
            k = k * np.asarray(k_scale[bi], np.float32).reshape(-1, 1)
        for q0 in range(0, s, query_chunk):
            q1 = min(q0 + query_chunk, s)
            sc = np.zeros((q1 - q0, k.shape[0]), np.float32)
            for h in range(H):
                sc += np.asarray(weights[bi, q0:q1, h], np.float32)[:, None] * np.maximum(q[bi, q0:q1, h] @ k.T, 0)
            cls = (start_pos + np.arange(q0, q1) + 1) // ratio
            if candidate_source is not None:
                cmask[bi, q0:q1] = select_candidate_blocks(sc, cls, candidate_source[0], candidate_source[1])
            elif candidates is not None:
                sc = np.where(np.asarray(candidates[bi, q0:q1, :k.shape[0]], bool), sc, -np.inf).astype(np.float32)
            sel = topk_indices(sc, kk, cls)
            out[bi, q0:q1] = np.where(sel >= 0, sel + offset, -1)
    return (out, cmask) if candidate_source is not None else out


# ----------------------------------------------------------------------------------------------- appends
def kv_write(x, w, cos, sin, pos, seq, cache, rd, eps) -> np.ndarray:
    """fused2.kv_write (dsv41/fused2.py:276-330): rmsnorm -> bf16 -> rope(last rd) -> bf16 -> fq8(32) -> bf16 into
    cache[seq, pos % W].  Returns the updated copy of cache."""
    cache = np.array(cache, np.float32, copy=True)
    W = cache.shape[1]
    y = bf16(rmsnorm(np.asarray(x, np.float32), w, eps))
    for r in range(y.shape[0]):
        p = max(int(pos[r]), 0)
        yr = rope(y[r], cos, sin, np.int64(p), rd)
        cache[int(seq[r]), p % W] = bf16(fake_quant_fp8(yr, 32))
    return cache


def window_kv(x, w, cos, sin, start_pos: int, ring, rd, eps):
    """Attention._window_kv (dsv41/model.py:1057-1298) for one sequence and a chunk of s >= 1 rows at positions
    start_pos..: rows = fq8(rope(rmsnorm(x))); history = the ring rows of positions start_pos - hist .. start_pos - 1
    (hist = min(start_pos, W - 1), captured BEFORE the commit, :1174-1200); the last min(s, W) chunk rows are then
    committed at pos % W (:1260-1296).  Returns ([history | rows] [hist + s, D], the updated ring copy [W, D])."""
    ring = np.array(ring, np.float32, copy=True)
    W = ring.shape[0]
    x = np.asarray(x, np.float32)
    s = x.shape[0]
    y = bf16(rmsnorm(x, w, eps))
    rows = np.stack([bf16(fake_quant_fp8(rope(y[r], cos, sin, np.int64(start_pos + r), rd), 32)) for r in range(s)])
    hist = min(int(start_pos), W - 1)
    history = np.stack([ring[(start_pos - hist + h) % W] for h in range(hist)]) if hist else rows[:0]
    for r in range(max(0, s - W), s):
        ring[(start_pos + r) % W] = rows[r]
    return np.concatenate([history, rows]), ring


def _pool(kv: np.ndarray, score: np.ndarray) -> np.ndarray:
    """sum over axis -2 of kv * softmax(score, axis -2) in fp32 (dsv41/model.py:624, 645, dsv41/decode.py:263)."""
    m = score.max(axis=-2, keepdims=True)
    e = np.exp((score - m).astype(np.float32))
    return (kv * (e / e.sum(axis=-2, keepdims=True))).sum(axis=-2).astype(np.float32)


def compress_pool(kv, score, start_pos: int, ratio: int, ring_kv, ring_sc, norm_w, eps):
    """Compressor.__call__ after the wkv / wgate projections (dsv41/model.py:593-660) for one sequence: kv, score fp32
    [s, D] at positions start_pos..; a continuation's partial group takes its earlier members from the ring
    (:600-606); every group that closes in the chunk is pooled, cast to bf16 and rmsnormed (:656-660); the chunk's last
    min(s, RING) positions then go to the ring (:607-610, written here after the partial read, as there).  Returns
    (latents bf16-valued [n_groups, D] (None when a continuation closes no group), ring_kv, ring_sc) (copies)."""
    kv = np.asarray(kv, np.float32)
    score = np.asarray(score, np.float32)
    ring_kv = np.array(ring_kv, np.float32, copy=True)
    ring_sc = np.array(ring_sc, np.float32, copy=True)
    R = ring_kv.shape[0]
    s = kv.shape[0]
    partial = start_pos % ratio
    pk = np.stack([ring_kv[(start_pos - partial + j) % R] for j in range(partial)]) if partial else kv[:0]
    ps = np.stack([ring_sc[(start_pos - partial + j) % R] for j in range(partial)]) if partial else score[:0]
    for j in range(max(0, s - R), s):
        ring_kv[(start_pos + j) % R] = kv[j]
        ring_sc[(start_pos + j) % R] = score[j]
    allk = np.concatenate([pk, kv])  # positions start_pos - partial ..
    alls = np.concatenate([ps, score])
    n_groups = allk.shape[0] // ratio
    if n_groups == 0:
        return (np.zeros((0, kv.shape[1]), np.float32) if start_pos == 0 else None), ring_kv, ring_sc
    g = _pool(allk[:n_groups * ratio].reshape(n_groups, ratio, -1), alls[:n_groups * ratio].reshape(n_groups, ratio, -1))
    return bf16(rmsnorm(bf16(g), norm_w, eps)), ring_kv, ring_sc


def compress_pool_decode(kv, score, pos, seq, ratio: int, ring_kv, ring_sc, norm_w, eps):
    """DecodeRuntime.compressor2 after the projections (dsv41/decode.py:243-265): every row's kv / score go to
    ring[seq, pos % RING] (all rows first, :258-259); each row then pools the `ratio` positions ending at pos from the
    ring (ratio 2: pos - 1 and pos, :260-263) -> bf16 -> rmsnorm; should = (pos + 1) % ratio == 0.  ring_* [S, RING, D].
    Returns (latent [B, D], should [B] bool, ring_kv, ring_sc)."""
    kv = np.asarray(kv, np.float32)
    score = np.asarray(score, np.float32)
    ring_kv = np.array(ring_kv, np.float32, copy=True)
    ring_sc = np.array(ring_sc, np.float32, copy=True)
    R = ring_kv.shape[1]
    pos = [int(p) for p in pos]
    seq = [int(x) for x in seq]
    for r in range(kv.shape[0]):
        ring_kv[seq[r], pos[r] % R] = kv[r]
        ring_sc[seq[r], pos[r] % R] = score[r]
    lat = []
    for r in range(kv.shape[0]):
        sl = [(pos[r] - ratio + 1 + j) % R for j in range(ratio)]
        lat.append(_pool(ring_kv[seq[r], sl], ring_sc[seq[r], sl]))
    lat = bf16(rmsnorm(bf16(np.stack(lat)), norm_w, eps))
    should = np.array([(p + 1) % ratio == 0 for p in pos])
    return lat, should, ring_kv, ring_sc


# ----------------------------------------------------------------------------------------------- projections
PERM_K = [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15]  # byte order of a 16-k group, dsv41/w8.py:23


def e4m3_decode(bits) -> np.ndarray:
    """Value of e4m3 (fn) bit patterns: s eeee mmm, bias 7, subnormals at e = 0, 0x7f / 0xff NaN (OCP FP8)."""
    b = np.asarray(bits, np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    return (sign * v).astype(np.float32)


def fp8_dequant(w8, s8, permuted: bool = True) -> np.ndarray:
    """dsv41/w8.py W8.bf16 / quant.dequant_fp8_block: e4m3 [N, K] (PERM_K byte order when permuted) times
    2^(s8[n // 32, k // 32] - 127) -> fp32 [N, K] (exact)."""
    w8 = np.asarray(w8, np.uint8)
    N, K = w8.shape
    if permuted:
        inv = [PERM_K.index(i) for i in range(16)]
        w8 = w8.reshape(N, K // 16, 16)[:, :, inv].reshape(N, K)
    sc = np.ldexp(np.float64(1.0), np.asarray(s8, np.int64) - 127)
    sc = np.repeat(np.repeat(sc, 32, 0)[:N], 32, 1)[:, :K]
    return (e4m3_decode(w8).astype(np.float64) * sc).astype(np.float32)


def fp8_gemm(x, w8, s8, group_cols: int = 0) -> np.ndarray:
    """dsv41/cukern.py fp8_gemm_tc (:164-200): x [M, K] (bf16 values) @ dequant(w8, s8)^T, accumulated exactly
    (float64) and returned as fp32 [Mo, N]; group_cols > 0: output row b, column n uses x row
    b * (N // group_cols) + n // group_cols."""
    x = np.asarray(x, np.float64)
    W = fp8_dequant(w8, s8).astype(np.float64)
    N = W.shape[0]
    if not group_cols:
        return (x @ W.T).astype(np.float32)
    G = N // group_cols
    Mo = x.shape[0] // G
    out = np.zeros((Mo, N), np.float64)
    for g in range(G):
        out[:, g * group_cols:(g + 1) * group_cols] = x[g::G] @ W[g * group_cols:(g + 1) * group_cols].T
    return out.astype(np.float32)


def compress_row(latent, cos, sin, pos, rd) -> np.ndarray:
    """Compressed-KV row (dsv41/decode.py:157-162, dsv41/model.py:1320-1346): rope(last rd) at the group's start
    position -> bf16 -> fq4(16, e4m3 scale) -> bf16."""
    y = rope(np.asarray(latent, np.float32), cos, sin, pos, rd)
    return bf16(fake_quant_fp4(y, 16, scale_e4m3=True))


def index_key_row(kraw, w, cos, sin, pos, rd, eps) -> np.ndarray:
    """Index-key row (dsv41/decode.py:270-275, dsv41/model.py:696-726): rmsnorm -> bf16 -> rope -> bf16 -> fq4(32)
    -> bf16."""
    y = bf16(rmsnorm(np.asarray(kraw, np.float32), w, eps))
    y = rope(y, cos, sin, pos, rd)
    return bf16(fake_quant_fp4(y, 32))


# ----------------------------------------------------------------------------------------------- the layer
def linear_fp8(x, w) -> np.ndarray:
    """dsv41/model.py:56-59 with a bf16-valued weight w [N, K]: fq8(x, 32) @ w^T, fp32 accumulation, bf16 result."""
    return bf16(fake_quant_fp8(np.asarray(x, np.float32), 32) @ np.asarray(w, np.float32).T)


def indexer_query(x, qr, wq_b, weights_proj, cos, sin, rd, start_pos: int, n_heads: int, head_dim: int = 128):
    """Indexer.__call__ query side (dsv41/model.py:734-746) for x [b, s, dim], qr [b, s, q_rank]: q =
    fq4(rope(linear_fp8(qr, wq_b)), 32) [b, s, n_heads, head_dim]; weights = bf16(bf16(x @ weights_proj^T) * scale),
    scale = head_dim^-1/2 n_heads^-1/2."""
    x = np.asarray(x, np.float32)
    b, s, _ = x.shape
    q = linear_fp8(qr, wq_b).reshape(b, s, n_heads, head_dim)
    for i in range(s):
        q[:, i] = rope(q[:, i], cos, sin, np.int64(start_pos + i), rd)
    q = bf16(fake_quant_fp4(q, 32))
    w = bf16(bf16(x @ np.asarray(weights_proj, np.float32).T) * np.float32(head_dim ** -0.5 * n_heads ** -0.5))
    return q, w


class AttentionLayer:
    """Attention.__call__ up to the o-projection (dsv41/model.py:1350-1573) for a layer that owns its window ring,
    compressor, index keys and compressed rows: the composition of window_kv, compress_pool, index_key_row,
    indexer_query, indexer_prefill, compress_row, sparse_attn and the inverse rope, holding the caches as numpy
    state.  Weights as bf16-valued arrays (c_wkv / c_wgate fp32)."""

    def __init__(self, weights: dict, *, n_heads, head_dim, rope_head_dim, window, ratio, index_n_heads, index_topk_k,
                 cos, sin, slots, cap, eps=1e-6):
        self.w = {k: np.asarray(v, np.float32) for k, v in weights.items()}
        self.H, self.D, self.rd, self.W, self.ratio = n_heads, head_dim, rope_head_dim, window, ratio
        self.HI, self.topk, self.eps, self.cos, self.sin = index_n_heads, index_topk_k, eps, cos, sin
        self.ring = np.zeros((slots, window, head_dim), np.float32)
        self.ckv = np.zeros((slots, cap, head_dim), np.float32)
        self.index_k = np.zeros((slots, cap, 128), np.float32)
        self.rk = np.zeros((slots, 8, head_dim), np.float32)
        self.rs = np.full((slots, 8, head_dim), -np.inf, np.float32)
        self.last_idx = None

    def attend(self, x, start_pos: int) -> np.ndarray:
        w, rd, eps, ratio = self.w, self.rd, self.eps, self.ratio
        x = np.asarray(x, np.float32)
        b, s, _ = x.shape
        cos, sin = self.cos, self.sin
        qr = bf16(rmsnorm(linear_fp8(x, w["wq_a"]), w["q_norm_w"], eps))                      # :1354
        q = linear_fp8(qr, w["wq_b"]).reshape(b, s, self.H, self.D)                            # :1355
        for i in range(s):
            q[:, i] = rope(q[:, i], cos, sin, np.int64(start_pos + i), rd)                     # :1356
        kv_raw = linear_fp8(x, w["wkv"])
        end = start_pos + s
        clen = end // ratio if ratio else 0
        kk = min(self.topk, clen)
        out = np.zeros((b, s, self.H, self.D), np.float32)
        hist, widx = prefill_window_idx(self.W, s, start_pos)
        if start_pos == 0:
            widx = window_idx(self.W, s, 0)
        lat_all = []
        for bi in range(b):
            rows, self.ring[bi] = window_kv(kv_raw[bi], w["kv_norm_w"], cos, sin, start_pos, self.ring[bi], rd, eps)
            if ratio:
                xf = x[bi]
                lat, self.rk[bi], self.rs[bi] = compress_pool(xf @ w["c_wkv"].T, xf @ w["c_wgate"].T, start_pos,
                                                              ratio, self.rk[bi], self.rs[bi], w["c_norm_w"], eps)
                lat_all.append(lat)
            off = rows.shape[0]
            idx = widx
            if kk:
                first = start_pos - start_pos % ratio
                if lat is not None:                                                            # :696-732
                    kraw = bf16(lat @ w["i_wk"].T)
                    for i in range(lat.shape[0]):
                        self.index_k[bi, start_pos // ratio + i] = index_key_row(
                            kraw[i], w["i_k_norm_w"], cos, sin, np.int64(first + i * ratio), rd, eps)
                qi, wi = indexer_query(x[bi:bi + 1], qr[bi:bi + 1], w["i_wq_b"], w["i_weights_proj"], cos, sin, rd,
                                       start_pos, self.HI)
                cidx = indexer_prefill(qi, wi, self.index_k[bi:bi + 1, :clen], start_pos, ratio, self.topk, off)[0]
                idx = np.concatenate([widx, cidx], -1)                                         # :1443
            if ratio and lat is not None:                                                      # :1320-1347
                first = start_pos - start_pos % ratio
                for i in range(lat.shape[0]):
                    self.ckv[bi, start_pos // ratio + i] = compress_row(lat[i], cos, sin,
                                                                        np.int64(first + i * ratio), rd)
            kv = np.concatenate([rows, self.ckv[bi, :clen]]) if clen else rows                 # :1442
            o = sparse_attn(q[bi:bi + 1], kv[None], w["attn_sink"], idx[None], self.D ** -0.5,
                            prefill_rounding=(s > 1))[0]                                       # :1526-1554
            for i in range(s):
                out[bi, i] = rope(o[i], cos, sin, np.int64(start_pos + i), rd, inverse=True)   # :1573
            self.last_idx = idx
        return out
