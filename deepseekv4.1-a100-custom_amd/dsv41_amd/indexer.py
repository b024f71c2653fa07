"""Lightning-indexer selection for a multi-token chunk: the score + top-k half of Indexer.__call__
(dsv41/model.py:766-893), on the HIP score kernel (bf16 or e4m3 keys, MFMA) and the radix-select top-k."""
from __future__ import annotations

import torch

from ._lib import call, lib, ptr, require_gpu, stream


def select_candidate_blocks(logits: torch.Tensor, compress_lens: torch.Tensor, topk_blocks: int,
                            block_size: int) -> torch.Tensor:
    """dsv41/model.py:256-265: logits [..., T] fp32 (positions >= the row's compress length are ignored, as the
    reference's -inf masked entries), compress_lens broadcastable to logits.shape[:-1] + (1,) -> bool mask like logits:
    the blocks of block_size positions holding the topk_blocks largest block maxima (the block of the last valid
    position forced in; ties lowest block first), each kept only when its maximum is finite."""
    dev = require_gpu(logits)
    T = logits.shape[-1]
    rows = logits.reshape(-1, T).float().contiguous()
    R = rows.shape[0]
    cl = compress_lens.to(dev).expand(*logits.shape[:-1], 1).reshape(-1).to(torch.int64).contiguous()
    mask = torch.empty(R, T, dtype=torch.bool, device=dev)
    _candidate_blocks(rows, R, T, T, ptr(cl), 0, 1, 1, topk_blocks, block_size, mask, dev)
    return mask.view(logits.shape)


def _candidate_blocks(score, R, n, width, clp, cl_start, cl_ratio, rows_per_seq, topk_blocks, block_size, mask, dev):
    nb = lib().dsv41_candidate_blocks_workspace_bytes(R, n, int(topk_blocks), int(block_size))
    ws = torch.empty(max(nb, 4) // 4, dtype=torch.int32, device=dev)
    call("dsv41_candidate_blocks", ptr(score), score.stride(0), R, n, width, clp, int(cl_start), int(cl_ratio),
         int(rows_per_seq), int(topk_blocks), int(block_size), ptr(mask), mask.stride(0), ptr(ws), nb, stream(dev))


def index_topk(q: torch.Tensor, weights: torch.Tensor, index_k: torch.Tensor, start_pos: int, ratio: int, topk: int,
               offset: int, k_scale: torch.Tensor | None = None, return_score: bool = False,
               candidates: torch.Tensor | None = None, candidate_source: tuple | None = None,
               out: torch.Tensor | None = None):
    """q: bf16 [b, s, H, 128] (rope'd, FP4-rounded index queries); weights: [b, s, H] (already scaled by
    d^-1/2 H^-1/2); index_k: [>= b, >= end//ratio, 128] bf16, or float8_e4m3fn with k_scale [>= b, >= end//ratio]
    fp32; query i sees compressed positions t < (start_pos + i + 1) // ratio.  Returns int32
    [b, s, min(topk, end//ratio)]: selected positions ascending + offset, -1 where masked (dsv41/model.py:886-893).
    Candidate blocks (dsv41/model.py:838-866): candidates = bool [b, s, >= end//ratio] masks a consumer layer's
    scores (non-candidates score -inf and fill the selection last, lowest index first); candidate_source =
    (topk_blocks, block_size) makes this the source layer and also returns its mask, bool [b, s, index_k.shape[1]].
    With return_score the scores come second: (out, score[, mask]).  out (optional): an int32 [b, s, kk] view with
    unit column stride (e.g. the compressed columns of a preallocated [window | compressed] index buffer) that
    receives the selection."""
    b, s, H, D = q.shape
    dev = require_gpu(q, weights, index_k)
    end = start_pos + s
    T = end // ratio
    kk = min(topk, T)
    if out is None:
        out = torch.empty(b, s, kk, device=dev, dtype=torch.int32)
    elif (out.shape != (b, s, kk) or out.dtype != torch.int32 or out.stride(-1) != 1
          or out.stride(0) != out.stride(1) * s):
        raise RuntimeError(f"index_topk: out {tuple(out.shape)} {out.dtype} is not an int32 [{b}, {s}, {kk}] row view")
    if b * s == 0 or kk == 0:
        res = (out,) + ((None,) if return_score else ()) + (
            (torch.zeros(b, s, index_k.shape[1], dtype=torch.bool, device=dev),) if candidate_source is not None else ())
        return res[0] if len(res) == 1 else res
    if index_k.shape[0] < b or index_k.shape[1] < T or D != 128 or H > 64:
        raise RuntimeError(f"index_topk: keys {tuple(index_k.shape)} do not cover {b} x {T} (D {D}, H {H})")
    qc = q.contiguous()
    w = weights.reshape(b * s, H).float().contiguous()
    assert index_k.stride(-1) == 1 and index_k.stride(-2) == D
    score = torch.empty(b * s, T, device=dev, dtype=torch.float32)
    st = stream(dev)
    cp, cs = None, 0
    if candidates is not None:
        if candidate_source is not None:
            raise RuntimeError("index_topk: a layer is either the candidate source or a consumer")
        cand = candidates[:b, :s].reshape(b * s, -1)
        if cand.dtype not in (torch.bool, torch.uint8) or cand.shape[1] < T:
            raise RuntimeError(f"index_topk: candidate mask {tuple(candidates.shape)} does not cover {b} x {s} x {T}")
        cand = cand.contiguous()
        cp, cs = ptr(cand), cand.stride(0)
    if index_k.dtype == torch.float8_e4m3fn:
        if k_scale is None:
            raise RuntimeError("index_topk: e4m3 keys need k_scale")
        ks = k_scale.float() if k_scale.dtype != torch.float32 else k_scale
        q8 = torch.empty(b * s, 64, 128, dtype=torch.uint8, device=dev)
        wf = torch.empty(b * s, 64, dtype=torch.float32, device=dev)
        call("dsv41_index_qprep", ptr(qc), ptr(w), b * s, H, ptr(q8), ptr(wf), st)
        call("dsv41_index_score", ptr(q8), 64 * 128, ptr(wf), 64, b * s, H, D, 1, ptr(index_k), index_k.stride(0),
             ptr(ks), ks.stride(0), None, s, None, start_pos, ratio, T, 0, ptr(score), T, None, cp, cs, st)
    else:
        call("dsv41_index_score", ptr(qc), H * D, ptr(w), H, b * s, H, D, 0, ptr(index_k), index_k.stride(0), None, 0,
             None, s, None, start_pos, ratio, T, 0, ptr(score), T, None, cp, cs, st)
    call("dsv41_topk_indices", ptr(score), T, b * s, T, kk, None, start_pos, ratio, s, int(offset), ptr(out),
         out.stride(1), st)
    res = (out,)
    if return_score:  # positions at or past a row's causal limit are not written (the top-k never reads them)
        res += (score.view(b, s, T),)
    if candidate_source is not None:
        width = index_k.shape[1]
        mask = torch.empty(b * s, width, dtype=torch.bool, device=dev)
        _candidate_blocks(score, b * s, T, width, None, start_pos, ratio, s, candidate_source[0], candidate_source[1],
                          mask, dev)
        res += (mask.view(b, s, width),)
    return res[0] if len(res) == 1 else res
