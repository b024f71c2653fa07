"""Drop-ins for dsv41/fused3.py: the decode indexer score and the top-k selection."""
from __future__ import annotations

import torch

from ._lib import as_i64, call, ptr, require_gpu, stream


def index_score(q: torch.Tensor, index_k: torch.Tensor, weights: torch.Tensor, seq: torch.Tensor, cl: torch.Tensor,
                cand: torch.Tensor | None = None, k_scale: torch.Tensor | None = None) -> torch.Tensor:
    """dsv41/fused3.py:46-62.  q: bf16 [B, 1, H, D]; index_k: [S, n_pos, D] bf16 (reference storage) or
    float8_e4m3fn with k_scale fp32 [S, n_pos] (per-row scale); weights [B, 1, H] or [B, H] (already scaled);
    seq, cl: int64 [B] -> fp32 [B, n_pos], -inf for t >= cl.  Positions >= cl are not read."""
    if cand is not None:
        raise NotImplementedError("index_score: candidate-block masks are not supported by this path")
    B, _, H, D = q.shape
    dev = require_gpu(q, index_k, weights)
    n_pos = index_k.shape[1]
    out = torch.empty(B, n_pos, device=dev, dtype=torch.float32)
    qc = q.contiguous()
    w = weights.reshape(B, H).float().contiguous()
    seq = as_i64(seq.reshape(-1), dev)
    cl = as_i64(cl.reshape(-1), dev)
    assert index_k.stride(2) == 1 and index_k.stride(1) == D
    if index_k.dtype == torch.float8_e4m3fn:
        if k_scale is None:
            raise RuntimeError("index_score: e4m3 keys need k_scale")
        ks = k_scale if k_scale.dtype == torch.float32 else k_scale.float()
        assert ks.stride(-1) == 1
        call("dsv41_index_score", ptr(qc), H * D, ptr(w), H, B, H, D, 1, ptr(index_k), index_k.stride(0), ptr(ks),
             ks.stride(0), ptr(seq), 1, ptr(cl), 0, 1, n_pos, 1, ptr(out), n_pos, stream(dev))
    else:
        call("dsv41_index_score", ptr(qc), H * D, ptr(w), H, B, H, D, 0, ptr(index_k), index_k.stride(0), None, 0,
             ptr(seq), 1, ptr(cl), 0, 1, n_pos, 1, ptr(out), n_pos, stream(dev))
    return out


def topk_indices(score: torch.Tensor, k: int, cl: torch.Tensor) -> torch.Tensor:
    """dsv41/fused3.py:65-75.  score: fp32 [B, n] -> int32 [B, 1, k]: the k largest per row, ascending, -1 where the
    index >= cl[b].  Ties go to the lower index."""
    B, n = score.shape
    dev = require_gpu(score)
    assert score.stride(-1) == 1
    cl = as_i64(cl.reshape(-1), dev)
    out = torch.empty(B, k, device=dev, dtype=torch.int32)
    call("dsv41_topk_indices", ptr(score), score.stride(0), B, n, k, ptr(cl), 0, 1, 1, 0, ptr(out), k, stream(dev))
    return out.view(B, 1, k)
