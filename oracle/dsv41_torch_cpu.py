"""The reference's PyTorch path for the sparse-attention layer, restated on the CPU in the reference's own precision.

TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py times beside the GPU, and its pin in tests/test_oracle.py).
Nothing in the product path imports this module.

The reference runs these steps with torch ops when its Triton / CUDA kernels are not used: the decode indexer's
einsum path (dsv41/decode.py:303-317), the prefill indexer's per-head bmm loop (dsv41/model.py:780-893) and the
prefill attention kernels.sparse_attn (dsv41/kernels.py:172-256), which is also the decode call site's fallback
(dsv41/model.py:1530-1546).  Precision is the reference default DSV41_INDEX_BF16=1: bf16 matmuls, fp32 head
accumulation (dsv41/model.py:780-781, dsv41/decode.py:303-307); the attention einsums in bf16 with an fp32 softmax
(dsv41/kernels.py:249-254).  The numpy oracle (dsv41_oracle.py) computes the same quantities without the per-head
bf16 rounding; tests/test_oracle.py checks that the two agree within the path's tolerances."""
from __future__ import annotations

import torch

QUERY_CHUNK = 64  # the prefill indexer's query chunk, DSV41_INDEX_QUERY_CHUNK default (dsv41/model.py:765-767)


def decode_index_topk(q: torch.Tensor, index_k: torch.Tensor, weights: torch.Tensor, cl: torch.Tensor,
                      k: int) -> torch.Tensor:
    """dsv41/decode.py:303-317 (FUSED2 layout): q [B, 1, H, D], index_k [B, n_pos, D] (each row's sequence),
    weights [B, 1, H] -> int32 [B, 1, k] ascending, -1 where idx >= cl.  Scores: bf16 einsum, relu, x bf16 weight,
    fp32 head sum; positions >= cl are -inf."""
    score = decode_scores(q, index_k, weights, cl)
    c = cl.view(-1, 1)
    idx = score.topk(k, dim=-1, sorted=False).indices.sort(dim=-1).values
    return torch.where(idx < c, idx, -1).to(torch.int32).unsqueeze(1)


def decode_scores(q, index_k, weights, cl) -> torch.Tensor:
    """The scores of decode_index_topk, [B, n_pos] fp32 (-inf past cl)."""
    score = torch.einsum("bshd,btd->bsht", q.to(torch.bfloat16), index_k.to(torch.bfloat16))
    score = (score.relu_() * weights.to(torch.bfloat16).unsqueeze(-1)).sum(dim=2, dtype=torch.float32)
    n_pos = score.shape[-1]
    return score.masked_fill(torch.arange(n_pos) >= cl.view(-1, 1, 1), -torch.inf)[:, 0]


def prefill_index_topk(q: torch.Tensor, weights: torch.Tensor, index_k: torch.Tensor, start_pos: int, ratio: int,
                       topk: int, offset: int, rows=None) -> torch.Tensor:
    """dsv41/model.py:780-893 for one sequence: q [1, S, H, D], weights [1, S, H], index_k [1, T, D] -> int32
    [1, len(rows), min(topk, end // ratio)]: per query chunk of 64 and per head `score += w_h * relu(q_h . K^T)`
    (bf16 bmm, fp32 accumulation), causal mask t >= (start + i + 1) // ratio, top-k indices sorted ascending, -1
    where masked, + offset.  rows: the query rows to compute (default all), processed in chunks of 64."""
    S = q.shape[1]
    H = q.shape[2]
    end = start_pos + S
    k_eff = min(topk, end // ratio)
    kT = index_k.to(torch.bfloat16).transpose(1, 2)
    T = index_k.shape[1]
    rows = torch.arange(S) if rows is None else torch.as_tensor(rows)
    out = []
    for c0 in range(0, rows.numel(), QUERY_CHUNK):
        r = rows[c0:c0 + QUERY_CHUNK]
        qc = q[:, r].to(torch.bfloat16)
        wc = weights[:, r].to(torch.bfloat16)
        score = torch.zeros(1, r.numel(), T, dtype=torch.float32)
        for h in range(H):
            sh = torch.bmm(qc[:, :, h], kT)
            sh.relu_()
            sh.mul_(wc[:, :, h].unsqueeze(-1))
            score.add_(sh)
        cls = (start_pos + r + 1) // ratio
        mask = torch.arange(T)[None, None, :] >= cls[None, :, None]
        score.masked_fill_(mask, -torch.inf)
        idx = score.topk(k_eff, dim=-1).indices.sort(dim=-1).values
        out.append(torch.where(idx < cls[None, :, None], idx + offset, -1).to(torch.int32))
    return torch.cat(out, dim=1)


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, sink: torch.Tensor, idx: torch.Tensor, scale: float,
                dv: int | None = None, q_chunk: int = 128) -> torch.Tensor:
    """kernels.sparse_attn (dsv41/kernels.py:172-256): q [b, s, H, Dqk] bf16, kv [b, n, Dqk] bf16, idx [b, s, t]
    int (-1 or >= n invalid), sink [H] fp32 -> [b, s, H, dv] bf16.  Gather, bf16 einsum, fp32 masked softmax with the
    sink in the denominator, bf16 probabilities times V (the first dv columns of each row)."""
    b, s, H, d = q.shape
    dv = d if dv is None else dv
    n = kv.shape[1]
    out = torch.empty(b, s, H, dv, dtype=torch.bfloat16)
    for s0 in range(0, s, q_chunk):
        s1 = min(s0 + q_chunk, s)
        ix = idx[:, s0:s1].long()
        valid = (ix >= 0) & (ix < n)
        g = torch.gather(kv, 1, ix.clamp(0, n - 1).reshape(b, -1, 1).expand(-1, -1, d)).view(b, s1 - s0, -1, d)
        scores = torch.einsum("bshd,bstd->bsht", q[:, s0:s1], g).float() * scale
        scores = scores.masked_fill(~valid.unsqueeze(2), float("-inf"))
        mx = scores.amax(dim=-1, keepdim=True).clamp_min(-1e30)
        p = torch.exp(scores - mx)
        denom = p.sum(dim=-1) + torch.exp(sink - mx.squeeze(-1))
        o = torch.einsum("bsht,bstd->bshd", p.to(g.dtype), g[..., :dv]).float() / denom.unsqueeze(-1)
        out[:, s0:s1] = o.to(torch.bfloat16)
    return out
