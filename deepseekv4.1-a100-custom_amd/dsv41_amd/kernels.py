"""Drop-in for kernels.sparse_attn (dsv41/kernels.py:172-256), the prefill sparse attention."""
from __future__ import annotations

import torch

from ._lib import call, ptr, require_gpu, stream


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                softmax_scale: float, q_chunk: int | None = None, d_v: int | None = None,
                kv2: torch.Tensor | None = None) -> torch.Tensor:
    """q: [b, s, h, d] bf16; kv: [b, n, d] bf16 (one shared K=V latent for all heads); attn_sink: [h] fp32;
    topk_idxs: [b, s, t] int32 with -1 (or >= n) = empty slot.  Returns [b, s, h, d_v] bf16 (d_v defaults to d;
    with d_v < d the values are the first d_v columns of each row, absorbed MLA).  q_chunk is accepted for
    signature compatibility; the kernel does not materialise the gathered rows.  kv2 [b, n2, d] (optional): a
    second source, as if kv were torch.cat([kv, kv2], dim=1) (dsv41/model.py:1442); topk_idxs may then be a
    column-sliced view (unit stride, any row stride)."""
    b, s, h, d = q.shape
    dv = d if d_v is None else d_v
    dev = require_gpu(q, kv, attn_sink, topk_idxs)
    n_kv = kv.shape[1]
    if n_kv <= 0 and s > 0:
        raise RuntimeError("sparse_attn received empty KV with non-empty queries")
    qc = q.contiguous()
    kvc = kv if kv.stride(-1) == 1 and kv.stride(-2) == d else kv.contiguous()
    idx = topk_idxs.to(torch.int32)
    if kv2 is None or idx.stride(-1) != 1 or idx.stride(-2) < idx.shape[-1] or idx.stride(0) != idx.stride(-2) * s:
        idx = idx.contiguous()
    t = idx.shape[-1]
    sink = attn_sink.float().contiguous()
    out = torch.empty(b, s, h, dv, device=dev, dtype=q.dtype)
    if b * s == 0:
        return out
    from ._lib import lib
    nbytes = lib().dsv41_attn_workspace_bytes(b * s, h, t, dv, 0)
    ws = torch.zeros(max(nbytes, 4) // 4, device=dev, dtype=torch.float32) if nbytes > 0 else None
    if kv2 is not None:
        k2 = kv2 if kv2.stride(-1) == 1 and kv2.stride(-2) == d else kv2.contiguous()
        call("dsv41_sparse_attn_kv2", ptr(qc), ptr(kvc), ptr(k2), ptr(sink), ptr(idx), ptr(out), b, s, h, d, dv, n_kv,
             kvc.stride(0), k2.shape[1], k2.stride(0), t, idx.stride(-2), float(softmax_scale), 0, ptr(ws), nbytes,
             stream(dev))
        return out
    call("dsv41_sparse_attn", ptr(qc), ptr(kvc), ptr(sink), ptr(idx), ptr(out), b, s, h, d, dv, n_kv, kvc.stride(0),
         t, float(softmax_scale), 0, ptr(ws), nbytes, stream(dev))
    return out
