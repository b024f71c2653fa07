"""Drop-ins for the path's entries of dsv41/fused.py: fake quantisation, rmsnorm, rotary, decode sparse attention.
Same call signatures as the reference; every call launches the HIP library on the tensor's current stream."""
from __future__ import annotations

import torch

from ._lib import as_i64, call, ptr, require_gpu, stream


def fake_quant(x: torch.Tensor, group: int, mode: int) -> torch.Tensor:
    """dsv41/fused.py:73-80. mode 0: fp8 pow2 scale; 1: fp4 pow2 scale; 2: fp4 e4m3 scale (per `group` columns)."""
    dev = require_gpu(x)
    if x.dtype != torch.bfloat16:
        raise RuntimeError("fake_quant: bf16 input expected")
    D = x.shape[-1]
    if mode == 0 and group == 32 and D > 1024:  # long rows (e.g. a hidden state): the norm_quant kernel, no norm
        return norm_quant(x, None, 0.0)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    call("dsv41_fake_quant", ptr(xc), ptr(y), xc.numel() // D, D, group, mode, stream(dev))
    return y


def fake_quant_fp8(x, block=32):
    """dsv41/fused.py:83-84."""
    return fake_quant(x, block, 0)


def fake_quant_fp4(x, block=32, scale_e4m3=False):
    """dsv41/fused.py:87-88."""
    return fake_quant(x, block, 2 if scale_e4m3 else 1)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """dsv41/fused.py:103-109 (bf16 rows, bf16 weight)."""
    dev = require_gpu(x, w)
    xc = x.contiguous()
    D = xc.shape[-1]
    if D > 1024 and xc.data_ptr() % 16:  # long rows go through 16-byte loads
        xc = xc.clone()
    y = torch.empty_like(xc)
    call("dsv41_rmsnorm", ptr(xc), ptr(w.to(torch.bfloat16).contiguous()), ptr(y), xc.numel() // D, D, float(eps),
         stream(dev))
    return y


def norm_quant(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    """dsv41/fused2.py:264-272: rmsnorm of each bf16 row then the per-32 fp8 fake quantisation -> bf16, rows of up to
    16384 (D % 32 == 0); w None: the fake quantisation alone (dsv41/fused.py:83-84 at any such row length)."""
    dev = require_gpu(x) if w is None else require_gpu(x, w)
    D = x.shape[-1]
    xc = x.contiguous()
    if xc.dtype != torch.bfloat16:
        xc = xc.to(torch.bfloat16)
    if xc.data_ptr() % 16:
        xc = xc.clone()
    y = torch.empty_like(xc)
    wc = None if w is None else w.to(torch.bfloat16).contiguous()
    call("dsv41_norm_quant", ptr(xc), ptr(wc), float(eps), ptr(y), xc.numel() // D, D, stream(dev))
    return y


def _rope_shape(x):
    if x.ndim == 3:
        b, s, d = x.shape
        h = 1
    else:
        b, s, h, d = x.shape
    return b, s, h, d


def rope_(x: torch.Tensor, rd: int, cos: torch.Tensor, sin: torch.Tensor, pos0: int, inverse: bool = False,
          pos_stride: int = 1) -> torch.Tensor:
    """dsv41/fused.py:223-234: rotate the last rd of every row of x ([b,s,d] or [b,s,h,d]) in place at position
    pos0 + s * pos_stride."""
    assert x.is_contiguous()
    dev = require_gpu(x, cos, sin)
    b, s, h, d = _rope_shape(x)
    call("dsv41_rope", ptr(x), ptr(cos), ptr(sin), None, int(pos0), 0, int(pos_stride), b * s * h, h, s, d, rd,
         int(inverse), stream(dev))
    return x


def rope_dev_(x: torch.Tensor, rd: int, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor, add: int = 0,
              inverse: bool = False, pos_stride: int = 1) -> torch.Tensor:
    """dsv41/fused.py:338-349: like rope_, with the base position read from the int64 device tensor pos (+ add)."""
    assert x.is_contiguous()
    dev = require_gpu(x, cos, sin)
    b, s, h, d = _rope_shape(x)
    p = as_i64(pos.reshape(-1), dev)
    call("dsv41_rope", ptr(x), ptr(cos), ptr(sin), ptr(p), 0, int(add), int(pos_stride), b * s * h, h, s, d, rd,
         int(inverse), stream(dev))
    return x


def _workspace(dev, R, H, L, dv, nsplit):
    from ._lib import lib
    n = lib().dsv41_attn_workspace_bytes(R, H, L, dv, nsplit)
    # zero-filled: the split-arrival counters at the end must start at zero (the library leaves them at zero)
    return (torch.zeros(max(n, 4) // 4, device=dev, dtype=torch.float32), n) if n > 0 else (None, 0)


def sparse_attn_decode(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                       softmax_scale: float) -> torch.Tensor:
    """dsv41/fused.py:269-280: q [b,1,h,d], kv [b,n,d], topk_idxs [b,1,t] int32 (-1 = empty) -> [b,1,h,d]."""
    b, s, h, d = q.shape
    assert s == 1
    from .kernels import sparse_attn
    return sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale)


def sparse_attn_decode2(q, kv1, kv2, attn_sink, topk_idxs, softmax_scale, nsplit: int = 1):
    """dsv41/fused.py:388-403: two KV sources; index < n1 reads kv1, otherwise kv2[index - n1]."""
    b, s, h, d = q.shape
    assert s == 1
    dev = require_gpu(q, kv1, kv2, attn_sink, topk_idxs)
    qc = q.contiguous()
    k1 = kv1.contiguous()
    k2 = kv2.contiguous() if kv2 is not None else None
    idx = topk_idxs.to(torch.int32).contiguous()
    t = idx.shape[-1]
    sink = attn_sink.float().contiguous()
    o = torch.empty_like(qc)
    ws, n = _workspace(dev, b, h, t, d, nsplit)
    call("dsv41_sparse_attn2", ptr(qc), ptr(k1), ptr(k2), ptr(sink), ptr(idx), ptr(o), b, h, d, k1.shape[1],
         k1.stride(0), k2.shape[1] if k2 is not None else 0, k2.stride(0) if k2 is not None else 0, t,
         float(softmax_scale), nsplit, ptr(ws), n, stream(dev))
    return o


def sparse_attn_decode_split(q, kv1, kv2, attn_sink, topk_idxs, softmax_scale, block_t: int = 64):
    """dsv41/fused.py:453-472 (flash-decoding split over the index list; the split count is the library's)."""
    return sparse_attn_decode2(q, kv1, kv2, attn_sink, topk_idxs, softmax_scale, nsplit=0)
