"""Drop-ins for the path's entries of dsv41/fused2.py: the SWA ring append (kv_write) and the graph-decode sparse
attention (sattn2)."""
from __future__ import annotations

import torch

from . import _lib
from ._lib import as_i64, attn_error_word, call, check_error_word, lib, ptr, require_gpu, stream


def kv_write(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor,
             cache: torch.Tensor, rd: int, eps: float, seq: torch.Tensor):
    """dsv41/fused2.py:303-330: x bf16 [B, d]; pos, seq int64 [B]; cache [S, W, d] ring, written at
    [seq, pos % W] with rmsnorm -> rope -> fp8 fake quant."""
    dev = require_gpu(x, cache, cos, sin)
    pos = as_i64(pos.reshape(-1), dev)
    seq = as_i64(seq.reshape(-1), dev)
    d = x.shape[-1]
    win = cache.shape[1]
    xc = x.reshape(-1, d).contiguous()
    B = xc.shape[0]
    assert cache.stride(2) == 1 and cache.stride(1) == d
    call("dsv41_kv_write", ptr(xc), d, ptr(w.to(torch.bfloat16).contiguous()), ptr(cos), ptr(sin), ptr(pos), ptr(seq),
         0, 0, 1, ptr(cache), cache.stride(0), win, None, B, d, rd, float(eps), 0, stream(dev))


def sattn2(q, kv_win, kv_c, idx, pos, attn_sink, cos, sin, rd, softmax_scale, seq, pmax, block_t: int = 64,
           plim=None, d_v: int | None = None, nsplit: int = 0, ws=None):
    """dsv41/fused2.py:417-446.  q: [B, 1, h, d] bf16 (row b at position pos[b] of sequence seq[b]); kv_win:
    [S, win, d] rings; pmax [B]: newest position written to the row's ring; kv_c: [S, n, d] compressed caches (may be
    an as_strided view) or None; idx: [B, 1, t] int32 rows of kv_c (-1 = none) or None; plim [B] (default pos):
    newest ring position the row may see.  Returns [B, 1, h, d_v] (d_v defaults to d) with the inverse rope on the
    last rd columns.  block_t is accepted for signature compatibility."""
    b, s, h, d = q.shape
    assert s == 1
    dv = d if d_v is None else d_v
    dev = require_gpu(q, kv_win, attn_sink)
    qc = q.contiguous()
    win = kv_win.shape[1]
    assert kv_win.stride(2) == 1 and kv_win.stride(1) == d
    pos = as_i64(pos.reshape(-1), dev)
    seq = as_i64(seq.reshape(-1), dev)
    pmax = as_i64(pmax.reshape(-1), dev)
    plim = as_i64(plim.reshape(-1), dev) if plim is not None else None
    if kv_c is None or idx is None:
        kvc, c_stride, n_c, ix, t = None, 0, 0, None, 0
    else:
        assert kv_c.stride(2) == 1 and kv_c.stride(1) == d
        kvc, c_stride, n_c = kv_c, kv_c.stride(0), kv_c.shape[1]
        ix = idx.to(torch.int32).reshape(b, -1).contiguous()
        t = ix.shape[-1]
    sink = attn_sink.float().contiguous()
    o = torch.empty(b, 1, h, dv, device=dev, dtype=q.dtype)
    nbytes = lib().dsv41_attn_workspace_bytes(b, h, win + t, dv, nsplit)
    if ws is None:  # the split-arrival counters at its start must be zero at first use; launches leave them ready
        ws = torch.zeros(max(nbytes, 4) // 4, device=dev, dtype=torch.float32) if nbytes > 0 else None
    else:
        assert ws.numel() * ws.element_size() >= nbytes, "workspace too small"
    call("dsv41_sattn2", ptr(qc), ptr(kv_win), kv_win.stride(0), win, ptr(kvc), c_stride, n_c, ptr(ix), t, ptr(pos),
         ptr(seq), ptr(pmax), ptr(plim), ptr(sink), ptr(cos), ptr(sin), int(rd), float(softmax_scale), ptr(o), b, h, d,
         dv, nsplit, ptr(ws), nbytes, stream(dev))
    if _lib.CHECK_ERRORS and (w := attn_error_word(ws, b, h, nbytes)) is not None:
        check_error_word("attention", w)
    return o
