"""The attention layer of the path as one drop-in: Attention.__call__ (dsv41/model.py:1350-1576) and the Indexer's
query side (dsv41/model.py:734-746), composed from the HIP entry points of this package.

  qr   = rmsnorm(linear_fp8(x, wq_a))                         q = rope(linear_fp8(qr, wq_b))
  window rows + indices  (cache.window_kv: rmsnorm(linear_fp8(x, wkv)) -> rope -> fp8 grid -> ring)
  compressor latents     (compressor.compress_pool over the fp32 wkv / wgate projections)
  index keys             (cache.write_index_k of rmsnorm(wk . latent))          before the selection, as there
  index queries/weights  (indexer_query)  ->  selection (indexer.index_topk)
  compressed rows        (cache.write_compress_kv)
  o    = sparse_attn over [window rows | compressed rows] read in place, one index buffer for both (the reference
         concatenates both, :1442-1443), then the inverse rope (:1573); optional o-projection (:1574-1576).

The GEMMs of the projections are either the FP8 block-scaled weights of the checkpoint (W8, dsv41_fp8_gemm) or bf16 /
fp32 tensors (plain library GEMMs through torch, as the reference's F.linear).  Everything else runs on the HIP
library; nothing here falls back to a CPU path."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import cache as C
from .compressor import compress_pool, new_rings
from .fused import fake_quant_fp4, fake_quant_fp8, rmsnorm, rope_, rope_dev_
from .indexer import index_topk
from .kernels import sparse_attn
from .w8 import W8, fp8_gemm_tc


def linear_w(x: torch.Tensor, w) -> torch.Tensor:
    """dsv41/w8.py:64-85: F.linear for a bf16 weight tensor, the FP8 GEMM for a W8 weight (bf16 x, bf16 result)."""
    if not isinstance(w, W8):
        return F.linear(x, w)
    lead = x.shape[:-1]
    y = fp8_gemm_tc(x.reshape(-1, x.shape[-1]), w.w8, w.s8)
    return y.view(*lead, w.shape[0])


def linear_fp8(x: torch.Tensor, w) -> torch.Tensor:
    """dsv41/model.py:56-59: the activation rounded to the fp8 grid (per 32, power-of-two scale), then the GEMM."""
    return linear_w(fake_quant_fp8(x, 32), w)


def indexer_query(x: torch.Tensor, qr: torch.Tensor, wq_b, weights_proj: torch.Tensor, cos: torch.Tensor,
                  sin: torch.Tensor, rd: int, start_pos: int, n_heads: int, head_dim: int = 128,
                  pos: torch.Tensor | None = None):
    """Indexer.__call__ query side (dsv41/model.py:734-746): q = fake_quant_fp4(rope(linear_fp8(qr, wq_b)), 32) as
    [b, s, n_heads, head_dim] bf16 (rope at start_pos + i, or at the int64 device positions pos [b] + i when given),
    weights = F.linear(x, weights_proj) * (head_dim^-1/2 * n_heads^-1/2) as [b, s, n_heads] bf16."""
    q = linear_fp8(qr, wq_b).unflatten(-1, (n_heads, head_dim)).contiguous()
    if pos is None:
        rope_(q, rd, cos, sin, start_pos)
    else:
        rope_dev_(q, rd, cos, sin, pos)
    q = fake_quant_fp4(q, 32)
    weights = F.linear(x, weights_proj) * (head_dim ** -0.5 * n_heads ** -0.5)
    return q, weights


class SparseAttention:
    """One attention layer that owns its window ring, compressor, index keys and compressed rows (a kv- and
    index-source layer of dsv41/model.py:1013-1056).  Weights: wq_a, q_norm_w, wq_b, wkv, kv_norm_w (bf16 tensors or
    W8), attn_sink fp32 [H]; with ratio > 0 the compressor's fp32 c_wkv / c_wgate [D, dim] and c_norm_w, and the
    indexer's i_wq_b, i_weights_proj [HI, dim], i_wk [128, D], i_k_norm_w; wo_a / wo_b (optional) for the
    o-projection.  Caches for `slots` sequences (batch row i is sequence i): ring [slots, window, D], compressed rows
    [slots, cap, D], index keys [slots, cap, 128] (bf16, the reference storage; with e4m3=True also an e4m3 copy +
    per-row scales, which the selection then reads), compressor rings [slots, 8, D]."""

    def __init__(self, weights: dict, *, n_heads: int, head_dim: int, rope_head_dim: int, window: int, ratio: int,
                 index_n_heads: int, index_topk_k: int, cos: torch.Tensor, sin: torch.Tensor, slots: int, cap: int,
                 eps: float = 1e-6, e4m3: bool = True, n_groups: int = 0, o_lora_rank: int = 0):
        self.w = weights
        self.H, self.D, self.rd, self.W, self.ratio = n_heads, head_dim, rope_head_dim, window, ratio
        self.HI, self.topk, self.eps = index_n_heads, index_topk_k, eps
        self.n_groups, self.o_lora_rank = n_groups, o_lora_rank
        self.cos, self.sin = cos, sin
        self.scale = head_dim ** -0.5
        dev = cos.device
        self.sink = weights["attn_sink"].float().contiguous()
        self.ring = torch.zeros(slots, window, head_dim, dtype=torch.bfloat16, device=dev)
        if ratio:
            self.ckv = torch.zeros(slots, cap, head_dim, dtype=torch.bfloat16, device=dev)
            self.index_k = torch.zeros(slots, cap, 128, dtype=torch.bfloat16, device=dev)
            self.k8 = torch.zeros(slots, cap, 128, dtype=torch.uint8, device=dev) if e4m3 else None
            self.ks = torch.zeros(slots, cap, dtype=torch.float32, device=dev) if e4m3 else None
            self.ring_kv, self.ring_score = new_rings(slots, head_dim, dev)

    def _keys(self, b: int):
        if self.k8 is not None:
            return self.k8[:b].view(torch.float8_e4m3fn), self.ks[:b]
        return self.index_k[:b], None

    def attend(self, x: torch.Tensor, start_pos: int) -> torch.Tensor:
        """Attention.__call__ up to the o-projection (dsv41/model.py:1350-1573): x [b, s, dim] bf16 of positions
        start_pos.. -> o [b, s, H, D] bf16 after the inverse rope.  Updates the caches."""
        w = self.w
        b, s, _ = x.shape
        rd, eps = self.rd, self.eps
        qr = rmsnorm(linear_fp8(x, w["wq_a"]), w["q_norm_w"], eps)
        q = linear_fp8(qr, w["wq_b"]).unflatten(-1, (self.H, self.D)).contiguous()
        rope_(q, rd, self.cos, self.sin, start_pos)
        win_kv, widx = C.window_kv(linear_fp8(x, w["wkv"]), w["kv_norm_w"], eps, self.cos, self.sin, rd, self.ring,
                                   start_pos)
        if not self.ratio:
            o = sparse_attn(q, win_kv, self.sink, widx, self.scale)
        else:
            ratio = self.ratio
            end = start_pos + s
            clen = end // ratio
            if clen > self.ckv.shape[1]:
                raise RuntimeError(f"SparseAttention: {clen} compressed rows exceed the cache capacity {self.ckv.shape[1]}")
            xf = x.float()
            latent = compress_pool(F.linear(xf, w["c_wkv"]), F.linear(xf, w["c_wgate"]), start_pos, ratio,
                                   self.ring_kv[:b], self.ring_score[:b], w["c_norm_w"], eps)
            new = latent is not None and latent.shape[1] > 0
            ww = widx.shape[-1]
            kk = min(self.topk, clen)
            idx = torch.empty(b, s, ww + kk, dtype=torch.int32, device=x.device)
            idx[:, :, :ww].copy_(widx)
            if kk:
                if new:  # the indexer's key append precedes its selection (dsv41/model.py:696-732)
                    C.write_index_k(self.index_k, F.linear(latent, w["i_wk"]), w["i_k_norm_w"], eps, start_pos,
                                    ratio, self.cos, self.sin, rd, k8=self.k8, k_scale=self.ks)
                qi, wi = indexer_query(x, qr, w["i_wq_b"], w["i_weights_proj"], self.cos, self.sin, rd, start_pos,
                                       self.HI)
                keys, ks = self._keys(b)
                index_topk(qi, wi, keys, start_pos, ratio, self.topk, win_kv.shape[1], k_scale=ks,
                           out=idx[:, :, ww:])
            if new:
                C.write_compress_kv(self.ckv, latent, start_pos, ratio, self.cos, self.sin, rd)
            o = sparse_attn(q, win_kv, self.sink, idx, self.scale, kv2=self.ckv[:b, :clen] if clen else None)
        rope_(o, rd, self.cos, self.sin, start_pos, inverse=True)
        return o

    def __call__(self, x: torch.Tensor, start_pos: int) -> torch.Tensor:
        """Attention.__call__ (dsv41/model.py:1350-1576): attend() then, with wo_a / wo_b given, the block-diagonal
        o-projection over n_groups and wo_b (dsv41/w8.py:86-105)."""
        o = self.attend(x, start_pos)
        w = self.w
        if "wo_a" not in w or "wo_b" not in w:
            return o
        b, s = o.shape[:2]
        g = o.view(b, s, self.n_groups, -1)
        if isinstance(w["wo_a"], W8):
            oa = fp8_gemm_tc(g.reshape(b * s * self.n_groups, -1), w["wo_a"].w8, w["wo_a"].s8,
                             group_cols=self.o_lora_rank).view(b, s, -1)
        else:
            oa = torch.einsum("bsgd,grd->bsgr", g, w["wo_a"].view(self.n_groups, self.o_lora_rank, -1)).flatten(2)
        return linear_fp8(oa, w["wo_b"])
