"""Lightning-indexer selection for a multi-token chunk: the score + top-k half of Indexer.__call__
(dsv41/model.py:766-893), on the HIP score kernel (bf16 or e4m3 keys, MFMA) and the radix-select top-k."""
from __future__ import annotations

import torch

from ._lib import call, ptr, require_gpu, stream


def index_topk(q: torch.Tensor, weights: torch.Tensor, index_k: torch.Tensor, start_pos: int, ratio: int, topk: int,
               offset: int, k_scale: torch.Tensor | None = None, return_score: bool = False):
    """q: bf16 [b, s, H, 128] (rope'd, FP4-rounded index queries); weights: [b, s, H] (already scaled by
    d^-1/2 H^-1/2); index_k: [>= b, >= end//ratio, 128] bf16, or float8_e4m3fn with k_scale [>= b, >= end//ratio]
    fp32; query i sees compressed positions t < (start_pos + i + 1) // ratio.  Returns int32
    [b, s, min(topk, end//ratio)]: selected positions ascending + offset, -1 where masked (dsv41/model.py:886-893)."""
    b, s, H, D = q.shape
    dev = require_gpu(q, weights, index_k)
    end = start_pos + s
    T = end // ratio
    kk = min(topk, T)
    out = torch.empty(b, s, kk, device=dev, dtype=torch.int32)
    if b * s == 0 or kk == 0:
        return (out, None) if return_score else out
    if index_k.shape[0] < b or index_k.shape[1] < T or D != 128 or H > 64:
        raise RuntimeError(f"index_topk: keys {tuple(index_k.shape)} do not cover {b} x {T} (D {D}, H {H})")
    qc = q.contiguous()
    w = weights.reshape(b * s, H).float().contiguous()
    assert index_k.stride(-1) == 1 and index_k.stride(-2) == D
    score = torch.empty(b * s, T, device=dev, dtype=torch.float32)
    st = stream(dev)
    if index_k.dtype == torch.float8_e4m3fn:
        if k_scale is None:
            raise RuntimeError("index_topk: e4m3 keys need k_scale")
        ks = k_scale.float() if k_scale.dtype != torch.float32 else k_scale
        q8 = torch.empty(b * s, 64, 128, dtype=torch.uint8, device=dev)
        wf = torch.empty(b * s, 64, dtype=torch.float32, device=dev)
        call("dsv41_index_qprep", ptr(qc), ptr(w), b * s, H, ptr(q8), ptr(wf), st)
        call("dsv41_index_score", ptr(q8), 64 * 128, ptr(wf), 64, b * s, H, D, 1, ptr(index_k), index_k.stride(0),
             ptr(ks), ks.stride(0), None, s, None, start_pos, ratio, T, 0, ptr(score), T, None, st)
    else:
        call("dsv41_index_score", ptr(qc), H * D, ptr(w), H, b * s, H, D, 0, ptr(index_k), index_k.stride(0), None, 0,
             None, s, None, start_pos, ratio, T, 0, ptr(score), T, None, st)
    call("dsv41_topk_indices", ptr(score), T, b * s, T, kk, None, start_pos, ratio, s, int(offset), ptr(out), kk, st)
    if return_score:  # positions at or past a row's causal limit are not written (the top-k never reads them)
        return out, score.view(b, s, T)
    return out
