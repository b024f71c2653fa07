"""Compressor pooling (dsv41/model.py:577-660, DecodeRuntime.compressor2 dsv41/decode.py:243-265) after the wkv / wgate
projections: the softmax-gated pooling over `ratio` positions and the rmsnorm that produce the latent rows the
compressed-KV append stores.  The projections themselves (fp32 GEMMs) are computed by the caller."""
from __future__ import annotations

import torch

from ._lib import as_i64, call, ptr, require_gpu, stream

RING = 8  # positions kept per sequence (Compressor.RING, dsv41/model.py:588)


def new_rings(slots: int, D: int, device, ring: int = RING):
    """(kv ring zeros, score ring -inf), fp32 [slots, ring, D], as Compressor.__init__ (dsv41/model.py:583-592)."""
    return (torch.zeros(slots, ring, D, dtype=torch.float32, device=device),
            torch.full((slots, ring, D), -torch.inf, dtype=torch.float32, device=device))


def compress_pool(kv: torch.Tensor, score: torch.Tensor, start_pos: int, ratio: int, ring_kv: torch.Tensor,
                  ring_score: torch.Tensor, norm_w: torch.Tensor, eps: float):
    """Compressor.__call__ after the projections (dsv41/model.py:593-660): kv, score fp32 [b, s, D] of positions
    start_pos.. (batch row i uses ring row i).  Returns the latents of the groups that close in the chunk, bf16
    [b, n_groups, D] (None when no group closes), and updates the rings."""
    b, s, D = kv.shape
    dev = require_gpu(kv, score, ring_kv, ring_score)
    ring = ring_kv.shape[1]
    first_end = start_pos + (ratio - 1 - start_pos % ratio)
    last = start_pos + s - 1
    n_groups = (last - first_end) // ratio + 1 if first_end <= last else 0
    kvc = kv.float().contiguous()
    scc = score.float().contiguous()
    w = norm_w.to(torch.bfloat16).contiguous()
    out = torch.empty(b, n_groups, D, dtype=torch.bfloat16, device=dev)
    assert ring_kv.is_contiguous() and ring_score.is_contiguous() and ring_kv.shape == ring_score.shape
    for bi in range(b):
        call("dsv41_compress_pool_prefill", ptr(kvc[bi]), ptr(scc[bi]), D, ptr(ring_kv[bi]), ptr(ring_score[bi]), ring,
             int(start_pos), s, D, int(ratio), ptr(w), float(eps), ptr(out[bi]), D, int(n_groups), stream(dev))
    if n_groups == 0:  # a fresh chunk shorter than ratio pools an empty tensor, a continuation returns None (:651-652)
        return out[:, :0] if start_pos == 0 else None
    return out


def compress_pool_decode(kv: torch.Tensor, score: torch.Tensor, pos: torch.Tensor, seq: torch.Tensor, ratio: int,
                         ring_kv: torch.Tensor, ring_score: torch.Tensor, norm_w: torch.Tensor, eps: float):
    """DecodeRuntime.compressor2 after the projections (dsv41/decode.py:243-265): kv, score fp32 [B, 1, D] (or [B, D])
    at positions pos of sequences seq.  Returns (latent bf16 [B, 1, D], should bool [B]); updates the rings."""
    dev = require_gpu(kv, score, ring_kv, ring_score)
    D = kv.shape[-1]
    kvc = kv.reshape(-1, D).float().contiguous()
    scc = score.reshape(-1, D).float().contiguous()
    B = kvc.shape[0]
    latent = torch.empty(B, 1, D, dtype=torch.bfloat16, device=dev)
    should = torch.empty(B, dtype=torch.bool, device=dev)
    assert ring_kv.is_contiguous() and ring_score.is_contiguous()
    call("dsv41_compress_pool_decode", ptr(kvc), ptr(scc), D, ptr(ring_kv), ptr(ring_score), ring_kv.stride(0),
         ring_kv.shape[1], ptr(as_i64(pos.reshape(-1), dev)), ptr(as_i64(seq.reshape(-1), dev)), B, D, int(ratio),
         ptr(norm_w.to(torch.bfloat16).contiguous()), float(eps), ptr(latent), D, ptr(should), stream(dev))
    return latent, should
