"""Cache appends of the path: SWA ring (decode and chunked prefill), compressed-KV rows and index-key rows.

These mirror Attention._window_kv (dsv41/model.py:1057-1298), Attention._compress_kv + SharedAttn.write_compress_kv
(dsv41/model.py:1300-1348, :508-541), the Indexer key append + SharedAttn.write_index_k (dsv41/model.py:696-732,
:543-574) and the decode-time appends of DecodeRuntime.attention2 / indexer (dsv41/decode.py:129-164, :270-282).
Cache tables are caller-owned torch tensors [slots, rows, width] (rows may be an as_strided view: the slot stride
is passed through)."""
from __future__ import annotations

import torch

from ._lib import as_i64, call, ptr, require_gpu, stream


_WIDX = {}  # window index tensors by shape: functions of (window, bsz, seqlen, start_pos or history length) only


def _cached_idx(key, make):
    t = _WIDX.get(key)
    if t is None:
        if len(_WIDX) > 256:
            _WIDX.clear()
        t = _WIDX[key] = make()
    return t


def window_topk_idxs(window: int, bsz: int, seqlen: int, start_pos: int, device) -> torch.Tensor:
    """get_window_topk_idxs (dsv41/model.py:132-254): physical ring slots (start_pos > 0) or temporary-row
    positions (start_pos == 0) of every query's causal window, -1 invalid; int32 [bsz, seqlen, width].  The result
    is cached per shape and must not be written to."""
    return _cached_idx(("slots", window, bsz, seqlen, start_pos, str(device)),
                       lambda: _window_topk_idxs(window, bsz, seqlen, start_pos, device))


def _window_topk_idxs(window: int, bsz: int, seqlen: int, start_pos: int, device) -> torch.Tensor:
    if seqlen <= 0:
        return torch.empty((bsz, 0, 0), dtype=torch.int32, device=device)
    if start_pos == 0:
        qpos = torch.arange(seqlen, device=device).unsqueeze(1)
        width = min(seqlen, window)
        a = (qpos - window + 1).clamp_min(0) + torch.arange(width, device=device).unsqueeze(0)
        idx = torch.where(a <= qpos, a, -1)
    else:
        qpos = (start_pos + torch.arange(seqlen, device=device)).unsqueeze(1)
        a = qpos - window + 1 + torch.arange(window, device=device).unsqueeze(0)
        idx = torch.where((a >= 0) & (a <= qpos), torch.remainder(a, window), -1)
    return idx.to(torch.int32).unsqueeze(0).expand(bsz, -1, -1).contiguous()


def window_kv(kv_raw: torch.Tensor, norm_w: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor, rd: int,
              ring: torch.Tensor, start_pos: int):
    """Attention._window_kv (dsv41/model.py:1057-1298) from the wkv projection output kv_raw [b, s, d]:
    rmsnorm -> rope -> fp8 fake quant, committed to ring [S, W, d] at pos % W.  Returns (window_kv, topk_idxs):
      start_pos == 0   : the chunk rows and positional window indices;
      s == 1           : the ring itself and ring-slot indices;
      continuation     : [history (<= W-1 rows copied out of the ring BEFORE the commit) | chunk rows] and
                         per-query causal indices into it."""
    b, s, d = kv_raw.shape
    dev = require_gpu(kv_raw, ring, cos, sin)
    W = ring.shape[1]
    x = kv_raw.reshape(b * s, d).contiguous()
    w = norm_w.to(torch.bfloat16).contiguous()
    st = stream(dev)
    if s == 1 and start_pos > 0:
        call("dsv41_kv_write", ptr(x), d, ptr(w), ptr(cos), ptr(sin), None, None, start_pos, 0, 1, ptr(ring),
             ring.stride(0), W, None, b, d, rd, float(eps), 0, st)
        return ring[:b], window_topk_idxs(W, b, 1, start_pos, dev)
    hist = min(int(start_pos), W - 1)
    tmp = torch.empty(b, hist + s, d, device=dev, dtype=kv_raw.dtype)
    # one launch per batch row: history copy-out (before the commit), chunk rows, ring commit
    for bi in range(b):
        call("dsv41_window_kv", ptr(x[bi * s:(bi + 1) * s]), d, ptr(w), ptr(cos), ptr(sin), int(start_pos), s,
             ptr(ring[bi:bi + 1]), W, ptr(tmp[bi]), hist, d, rd, float(eps), st)
    if start_pos == 0:
        return tmp, window_topk_idxs(W, b, s, 0, dev)

    def make():
        width = min(W, hist + s)
        qq = (hist + torch.arange(s, device=dev)).unsqueeze(1)
        idx = (qq - W + 1).clamp_min(0) + torch.arange(width, device=dev).unsqueeze(0)
        return torch.where(idx <= qq, idx, -1).to(torch.int32).unsqueeze(0).expand(b, -1, -1).contiguous()
    return tmp, _cached_idx(("hist", W, b, s, hist, str(dev)), make)


def write_compress_kv(cache: torch.Tensor, latent: torch.Tensor, start_pos: int, ratio: int, cos: torch.Tensor,
                      sin: torch.Tensor, rd: int) -> None:
    """Prefill compressed append (dsv41/model.py:1320-1347 + :508-541): latent [b, n, D] (compressor output) ->
    rope at first_group_start + i*ratio -> fq4(16, e4m3 scale) -> cache[:b, start_pos//ratio + i]."""
    b, n, D = latent.shape
    if n == 0:
        return
    dev = require_gpu(latent, cache)
    assert cache.stride(2) == 1 and cache.stride(1) == D
    if b > cache.shape[0] or start_pos // ratio + n > cache.shape[1] or cache.shape[2] != D:
        raise RuntimeError(f"write_compress_kv: rows {start_pos // ratio}+{n} x {b} do not fit cache {tuple(cache.shape)}")
    first = start_pos - (start_pos % ratio)
    x = latent.reshape(b * n, D).contiguous()
    call("dsv41_append_rows", ptr(x), D, None, 0.0, ptr(cos), ptr(sin), rd, None, first, ratio, 0, None, n, None,
         start_pos // ratio, ptr(cache), cache.stride(0), 2, 16, None, 0, None, 0, b * n, D, stream(dev))


def write_index_k(cache: torch.Tensor, k_raw: torch.Tensor, norm_w: torch.Tensor, eps: float, start_pos: int,
                  ratio: int, cos: torch.Tensor, sin: torch.Tensor, rd: int, k8: torch.Tensor | None = None,
                  k_scale: torch.Tensor | None = None) -> None:
    """Prefill index-key append (dsv41/model.py:696-732 + :543-574): k_raw [b, n, 128] (= wk . latent) -> rmsnorm ->
    rope at first_group_start + i*ratio -> fq4(32) -> cache[:b, start_pos//ratio + i]; with k8/k_scale also the e4m3
    copy with a per-row power-of-two scale."""
    b, n, D = k_raw.shape
    if n == 0:
        return
    dev = require_gpu(k_raw, cache)
    for tab in (cache, k8):
        if tab is not None and (b > tab.shape[0] or start_pos // ratio + n > tab.shape[1] or tab.shape[2] != D):
            raise RuntimeError(f"write_index_k: rows {start_pos // ratio}+{n} x {b} do not fit {tuple(tab.shape)}")
    first = start_pos - (start_pos % ratio)
    x = k_raw.reshape(b * n, D).contiguous()
    call("dsv41_append_rows", ptr(x), D, ptr(norm_w.to(torch.bfloat16).contiguous()), float(eps), ptr(cos), ptr(sin),
         rd, None, first, ratio, 0, None, n, None, start_pos // ratio, ptr(cache), cache.stride(0), 1, 32,
         ptr(k8) if k8 is not None else None, k8.stride(0) if k8 is not None else 0,
         ptr(k_scale) if k_scale is not None else None, k_scale.stride(0) if k_scale is not None else 0, b * n, D,
         stream(dev))


def append_compressed_decode(cache: torch.Tensor, latent: torch.Tensor, pos: torch.Tensor, seq: torch.Tensor,
                             row: torch.Tensor, ratio: int, cos: torch.Tensor, sin: torch.Tensor, rd: int) -> None:
    """Decode compressed append (dsv41/decode.py:157-162): rope_dev_(latent, add = 1 - ratio) -> fq4(16, e4m3) ->
    cache[seq, row] (row = compress_len - 1 when the group closed, else the caller's spare row)."""
    D = latent.shape[-1]
    x = latent.reshape(-1, D).contiguous()
    B = x.shape[0]
    dev = require_gpu(x, cache)
    assert cache.stride(2) == 1 and cache.stride(1) == D
    call("dsv41_append_rows", ptr(x), D, None, 0.0, ptr(cos), ptr(sin), rd, ptr(as_i64(pos.reshape(-1), dev)), 0, 0,
         1 - ratio, ptr(as_i64(seq.reshape(-1), dev)), 1, ptr(as_i64(row.reshape(-1), dev)), 0, ptr(cache),
         cache.stride(0), 2, 16, None, 0, None, 0, B, D, stream(dev))


def append_index_k_decode(cache: torch.Tensor, k_raw: torch.Tensor, norm_w: torch.Tensor, eps: float,
                          pos: torch.Tensor, seq: torch.Tensor, row: torch.Tensor, ratio: int, cos: torch.Tensor,
                          sin: torch.Tensor, rd: int, k8: torch.Tensor | None = None,
                          k_scale: torch.Tensor | None = None) -> None:
    """Decode index-key append (dsv41/decode.py:270-282): rmsnorm -> rope_dev_(add = 1 - ratio) -> fq4(32) ->
    cache[seq, row] (bf16, the reference storage; may be None) and/or the e4m3 copy k8[seq, row] + k_scale."""
    D = k_raw.shape[-1]
    x = k_raw.reshape(-1, D).contiguous()
    B = x.shape[0]
    dev = require_gpu(x, cache, k8)
    if cache is None and k8 is None:
        raise RuntimeError("append_index_k_decode: no destination table")
    call("dsv41_append_rows", ptr(x), D, ptr(norm_w.to(torch.bfloat16).contiguous()), float(eps), ptr(cos), ptr(sin),
         rd, ptr(as_i64(pos.reshape(-1), dev)), 0, 0, 1 - ratio, ptr(as_i64(seq.reshape(-1), dev)), 1,
         ptr(as_i64(row.reshape(-1), dev)), 0, ptr(cache), cache.stride(0) if cache is not None else 0, 1, 32,
         ptr(k8) if k8 is not None else None, k8.stride(0) if k8 is not None else 0,
         ptr(k_scale) if k_scale is not None else None, k_scale.stride(0) if k_scale is not None else 0, B, D,
         stream(dev))


def _nw(nw_tab, dev):
    """The no-write row table as contiguous int64 on the launch device (None stays None)."""
    return None if nw_tab is None else as_i64(nw_tab.reshape(-1), dev)


def decode_appends(kv_raw, kv_norm, ring, latent, ckv, k_raw, k_norm, kbf, k8, k_scale, pos, seq, ratio: int,
                   cos, sin, rd: int, eps: float, q_idx=None, w_idx=None, q8=None, wf=None, nw_tab=None) -> None:
    """Every cache write of one decode step in one launch (dsv41/decode.py:129-164, :270-282): the SWA ring row
    (kv_write), the compressed-KV row and the index-key row (bf16 table kbf and/or e4m3 table k8 + k_scale), each at
    compress_len - 1 when the step closes a compression group, else at the sequence's no-write row: nw_tab[seq]
    (int64 [S], the reference's per-slot table of the last row of each slot's own capacity under DSV41_SLOT_CAPS,
    dsv41/decode.py:62-68, :176-181) or, without a table, the table's spare last row.  latent / k_raw
    may be None (layers that own no compressor / indexer keys).  With q_idx ([B, 1, HI, 128] bf16) and w_idx
    ([B, HI] bf16) it also writes the prepared e4m3 index queries q8 [B, 64, 128] (uint8) and folded weights
    wf [B, 64] of the e4m3 score path."""
    dev = require_gpu(kv_raw, ring, latent, ckv, k_raw, kbf, k8)
    Dw = ring.shape[-1]
    x = kv_raw.reshape(-1, Dw).contiguous()
    B = x.shape[0]
    assert ring.stride(2) == 1 and ring.stride(1) == Dw
    lat = latent.reshape(B, -1).contiguous() if latent is not None else None
    kr = k_raw.reshape(B, -1).contiguous() if k_raw is not None else None
    tab = k8 if k8 is not None else kbf
    Dk = tab.shape[-1] if tab is not None else 128
    kcap = tab.shape[1] if tab is not None else 1
    call("dsv41_decode_appends", ptr(x), ptr(kv_norm.to(torch.bfloat16).contiguous()), ptr(ring), ring.stride(0),
         ring.shape[1], Dw, ptr(lat), ptr(ckv), ckv.stride(0) if ckv is not None else 0,
         ckv.shape[1] if ckv is not None else 1, ptr(kr),
         ptr(k_norm.to(torch.bfloat16).contiguous()) if k_norm is not None else None, ptr(kbf),
         kbf.stride(0) if kbf is not None else 0, ptr(k8), k8.stride(0) if k8 is not None else 0, ptr(k_scale),
         k_scale.stride(0) if k_scale is not None else 0, kcap, Dk, ptr(as_i64(pos.reshape(-1), dev)),
         ptr(as_i64(seq.reshape(-1), dev)), ptr(_nw(nw_tab, dev)), int(ratio), ptr(cos), ptr(sin), int(rd), float(eps),
         ptr(q_idx.contiguous()) if q_idx is not None else None,
         ptr(w_idx.to(torch.bfloat16).contiguous()) if q_idx is not None else None,
         q_idx.shape[-2] if q_idx is not None else 0, ptr(q8), ptr(wf), B, stream(dev))


def index_keys_to_e4m3(kbf16: torch.Tensor):
    """Snapshot conversion (dsv41/engine.py:1072-1230 stores the cache tensors as they are): the reference's bf16
    index-key table [..., 128] -> (e4m3 bytes as float8_e4m3fn [..., 128], fp32 per-row scale [...]), the encoding
    of the key appends.  Exact for the FP4-grid rows the reference writes."""
    dev = require_gpu(kbf16)
    assert kbf16.shape[-1] == 128
    x = kbf16.to(torch.bfloat16).contiguous()
    n = x.numel() // 128
    k8 = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    ks = torch.empty(x.shape[:-1], dtype=torch.float32, device=dev)
    call("dsv41_index_keys_encode", ptr(x), n, ptr(k8), ptr(ks), stream(dev))
    return k8.view(torch.float8_e4m3fn), ks


def index_keys_to_bf16(k8: torch.Tensor, k_scale: torch.Tensor) -> torch.Tensor:
    """The inverse: e4m3 table [..., 128] + per-row scales [...] -> the reference's bf16 table (e4m3 x scale)."""
    dev = require_gpu(k8, k_scale)
    assert k8.shape[-1] == 128 and tuple(k_scale.shape) == tuple(k8.shape[:-1])
    k = k8.contiguous().view(torch.uint8)
    s = k_scale.float().contiguous()
    out = torch.empty(k.shape, dtype=torch.bfloat16, device=dev)
    call("dsv41_index_keys_decode", ptr(k), ptr(s), k.numel() // 128, ptr(out), stream(dev))
    return out

