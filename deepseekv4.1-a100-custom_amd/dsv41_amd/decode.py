"""One decode layer-step of the sparse-attention path on the HIP library, the part of DecodeRuntime.attention2
(dsv41/decode.py:106-174) between the projections and the o-projection:

  SWA ring append (kv_write)  ->  compressed-KV append + index-key append (rows at compress_len - 1, or the spare
  row when no group closes)   ->  indexer score (e4m3 keys, fp8 MFMA)  ->  top-k  ->  sattn2 over ring + top-k rows.

All launches go to the current stream, allocate only through torch (capturable in a CUDA/HIP graph)."""
from __future__ import annotations

import torch

from . import cache as C
from .fused2 import kv_write, sattn2
from .fused3 import index_score, topk_indices


class DecodeLayer:
    """Per-layer state: ring [S, W, dqk], compressed rows [S, cap, dqk], index keys [S, cap, 128] (e4m3) + scales,
    rope tables and the sink.  `ratio` is the compression ratio, `topk` the indexer's k."""

    def __init__(self, ring, ckv, k8, ks, sink, cos, sin, ratio: int, topk: int, rd: int = 64, dv: int = 512,
                 eps: float = 1e-6, kbf16=None):
        self.ring, self.ckv, self.k8, self.ks, self.sink = ring, ckv, k8, ks, sink
        self.cos, self.sin = cos, sin
        self.ratio, self.topk, self.rd, self.dv, self.eps = ratio, topk, rd, dv, eps
        self.kbf16 = kbf16
        self.scale = ckv.shape[-1] ** -0.5

    def appends(self, kv_raw, kv_norm, latent, k_raw, k_norm, pos, seq):
        """Cache writes of this step (dsv41/decode.py:134, :157-164, :270-282)."""
        kv_write(kv_raw, kv_norm, self.cos, self.sin, pos, self.ring, self.rd, self.eps, seq)
        cl = torch.div(pos + 1, self.ratio, rounding_mode="floor")
        should = torch.remainder(pos + 1, self.ratio) == 0
        row = torch.where(should, cl - 1, torch.full_like(cl, self.ckv.shape[1] - 1))
        C.append_compressed_decode(self.ckv, latent, pos, seq, row, self.ratio, self.cos, self.sin, self.rd)
        C.append_index_k_decode(self.kbf16, k_raw, k_norm, self.eps, pos, seq, row, self.ratio, self.cos, self.sin,
                                self.rd, k8=self.k8, k_scale=self.ks)
        return cl

    def select(self, q_idx, w_idx, pos, seq, cl=None):
        if cl is None:
            cl = torch.div(pos + 1, self.ratio, rounding_mode="floor")
        score = index_score(q_idx, self.k8, w_idx, seq, cl, k_scale=self.ks)
        return topk_indices(score, self.topk, cl)

    def attend(self, q, idx, pos, seq, pmax, plim=None):
        return sattn2(q, self.ring, self.ckv, idx, pos, self.sink, self.cos, self.sin, 0 if self.dv < q.shape[-1]
                      else self.rd, self.scale, seq, pmax, plim=plim, d_v=self.dv)

    def step(self, q, q_idx, w_idx, pos, seq, pmax, plim=None):
        idx = self.select(q_idx, w_idx, pos, seq)
        return self.attend(q, idx, pos, seq, pmax, plim)
