"""Drop-in for kernels.sparse_attn (dsv41/kernels.py:172-256), the prefill sparse attention."""
from __future__ import annotations

import torch

from ._lib import call, ptr, require_gpu, stream


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                softmax_scale: float, q_chunk: int | None = None, d_v: int | None = None) -> torch.Tensor:
    """q: [b, s, h, d] bf16; kv: [b, n, d] bf16 (one shared K=V latent for all heads); attn_sink: [h] fp32;
    topk_idxs: [b, s, t] int32 with -1 (or >= n) = empty slot.  Returns [b, s, h, d_v] bf16 (d_v defaults to d;
    with d_v < d the values are the first d_v columns of each row, absorbed MLA).  q_chunk is accepted for
    signature compatibility; the kernel does not materialise the gathered rows."""
    b, s, h, d = q.shape
    dv = d if d_v is None else d_v
    dev = require_gpu(q, kv, attn_sink, topk_idxs)
    n_kv = kv.shape[1]
    if n_kv <= 0 and s > 0:
        raise RuntimeError("sparse_attn received empty KV with non-empty queries")
    qc = q.contiguous()
    kvc = kv if kv.stride(-1) == 1 and kv.stride(-2) == d else kv.contiguous()
    idx = topk_idxs.to(torch.int32).contiguous()
    t = idx.shape[-1]
    sink = attn_sink.float().contiguous()
    out = torch.empty(b, s, h, dv, device=dev, dtype=q.dtype)
    if b * s == 0:
        return out
    from ._lib import lib
    nbytes = lib().dsv41_attn_workspace_bytes(b * s, h, t, dv, 0)
    ws = torch.zeros(max(nbytes, 4) // 4, device=dev, dtype=torch.float32) if nbytes > 0 else None
    call("dsv41_sparse_attn", ptr(qc), ptr(kvc), ptr(sink), ptr(idx), ptr(out), b, s, h, d, dv, n_kv, kvc.stride(0),
         t, float(softmax_scale), 0, ptr(ws), nbytes, stream(dev))
    return out
