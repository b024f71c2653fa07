"""One decode layer-step of the sparse-attention path on the HIP library, the part of DecodeRuntime.attention2
(dsv41/decode.py:106-174) between the projections and the o-projection:

  SWA ring append (kv_write)  ->  compressed-KV append + index-key append (rows at compress_len - 1, or the spare
  row when no group closes)   ->  indexer score (e4m3 keys, fp8 MFMA)  ->  top-k  ->  sattn2 over ring + top-k rows.

All launches go to the current stream, allocate only through torch (capturable in a CUDA/HIP graph)."""
from __future__ import annotations

import torch

from . import cache as C
from .fused2 import sattn2
from .fused3 import DecodeSelector


class DecodeLayer:
    """Per-layer state: ring [S, W, dqk], compressed rows [S, cap, dqk], index keys [S, cap, 128] (e4m3) + scales,
    rope tables and the sink.  `ratio` is the compression ratio, `topk` the indexer's k.  nw_tab (int64 [S], may be
    None): the row a step that closes no compression group writes, per sequence -- the reference's per-slot table
    under DSV41_SLOT_CAPS (the last row of the slot's own capacity, dsv41/decode.py:62-68, :176-181), needed when
    the tables are as_strided views of per-slot capacities (dsv41/slots.py:1-11); None: the tables' spare last
    row."""

    def __init__(self, ring, ckv, k8, ks, sink, cos, sin, ratio: int, topk: int, rd: int = 64, dv: int = 512,
                 eps: float = 1e-6, kbf16=None, nw_tab=None):
        self.ring, self.ckv, self.k8, self.ks, self.sink = ring, ckv, k8, ks, sink
        self.cos, self.sin = cos, sin
        self.ratio, self.topk, self.rd, self.dv, self.eps = ratio, topk, rd, dv, eps
        self.kbf16 = kbf16
        self.nw_tab = None if nw_tab is None else nw_tab.to(device=ring.device, dtype=torch.int64).contiguous()
        self.scale = ckv.shape[-1] ** -0.5
        self._selectors = {}
        self._qbufs = {}
        self._attn_ws = {}
        self._prepared = None

    def _qbuf(self, B, dev):
        buf = self._qbufs.get(B)
        if buf is None:
            buf = self._qbufs[B] = (torch.empty(B, 64, 128, dtype=torch.uint8, device=dev),
                                    torch.empty(B, 64, dtype=torch.float32, device=dev))
        return buf

    def appends(self, kv_raw, kv_norm, latent, k_raw, k_norm, pos, seq, q_idx=None, w_idx=None):
        """Cache writes of this step in one launch (dsv41/decode.py:134, :157-164, :270-282); with q_idx/w_idx the
        same launch prepares the e4m3 index queries that select() then uses."""
        q8 = wf = None
        if q_idx is not None:
            q8, wf = self._qbuf(q_idx.shape[0], q_idx.device)
        C.decode_appends(kv_raw, kv_norm, self.ring, latent, self.ckv, k_raw, k_norm, self.kbf16, self.k8, self.ks,
                         pos, seq, self.ratio, self.cos, self.sin, self.rd, self.eps, q_idx, w_idx, q8, wf,
                         nw_tab=self.nw_tab)
        self._prepared = (q8, wf) if q_idx is not None else None

    def appends_select(self, kv_raw, kv_norm, latent, k_raw, k_norm, pos, seq, q_idx, w_idx, cl=None, cand=None):
        """appends() followed by select(), the appends inside the indexer's first launch (dsv41_decode_select when
        the selection fits one launch, else dsv41_decode_score and the top-k launches) when the keys are e4m3; the
        rows' sequences must be distinct (one row per slot).  Falls back to the two calls otherwise.  Returns the
        top-k indices [B, 1, k]."""
        from ._lib import as_i64
        dev = q_idx.device
        if cl is None:
            cl = torch.div(pos + 1, self.ratio, rounding_mode="floor")
        sel = self.selector(q_idx.shape[0], dev)
        if self.k8 is None or k_raw is None:
            self.appends(kv_raw, kv_norm, latent, k_raw, k_norm, pos, seq, q_idx, w_idx)
            return self.select(q_idx, w_idx, pos, seq, cl)
        app = dict(kv_raw=kv_raw, kv_norm=kv_norm, ring=self.ring, latent=latent, ckv=self.ckv, k_raw=k_raw,
                   k_norm=k_norm, kbf=self.kbf16, k8=self.k8, k_scale=self.ks, ratio=self.ratio, cos=self.cos,
                   sin=self.sin, rd=self.rd, eps=self.eps, q_idx=q_idx, w_idx=w_idx, nw_tab=self.nw_tab)
        self._prepared = None
        return sel.select_with_appends(app, as_i64(pos.reshape(-1), dev), as_i64(seq.reshape(-1), dev),
                                       as_i64(cl.reshape(-1), dev), cand)

    def select(self, q_idx, w_idx, pos, seq, cl=None):
        """Indexer score over the e4m3 keys + top-k (dsv41/decode.py:284-294), histogram-assisted selection."""
        if cl is None:
            cl = torch.div(pos + 1, self.ratio, rounding_mode="floor")
        sel = self.selector(q_idx.shape[0], q_idx.device)
        return sel(q_idx, self.k8, w_idx, seq, cl, k_scale=self.ks, prepared=self._prepared)

    def selector(self, rows: int, device) -> DecodeSelector:
        sel = self._selectors.get(rows)
        if sel is None:
            # cl never covers the tables' spare last row
            sel = self._selectors[rows] = DecodeSelector(rows, self.k8.shape[1], self.topk, device,
                                                         max_cl=self.k8.shape[1] - 1)
        return sel

    def attn_workspace(self, B: int, h: int, L: int, device) -> torch.Tensor:
        """Persistent zero-initialised attention workspace for B rows x h heads over L key positions (split partials
        + arrival counters, which every launch leaves at zero), reallocated when a wider index list needs more;
        allocate it before graph capture.  Calls sharing it must be stream-ordered."""
        from ._lib import lib
        n = lib().dsv41_attn_workspace_bytes(B, h, L, self.dv, 0)
        ws = self._attn_ws.get((B, h))
        if ws is None or ws.numel() * 4 < n:
            ws = self._attn_ws[(B, h)] = torch.zeros(max(n, 4) // 4, device=device, dtype=torch.float32)
        return ws

    def check(self) -> None:
        """Raise RuntimeError when a launch of this layer reported an error through a workspace error word (the
        indexer's row barriers, the attention's in-launch split merge); clears the words.  Synchronises."""
        from ._lib import attn_error_word, check_error_word
        for sel in self._selectors.values():
            sel.check()
        for (B, h), ws in self._attn_ws.items():
            w = attn_error_word(ws, B, h, ws.numel() * 4)
            if w is not None:
                check_error_word("attention", w)

    def attend(self, q, idx, pos, seq, pmax, plim=None):
        ws = self.attn_workspace(q.shape[0], q.shape[2], self.ring.shape[1] + idx.shape[-1], q.device)
        return sattn2(q, self.ring, self.ckv, idx, pos, self.sink, self.cos, self.sin, 0 if self.dv < q.shape[-1]
                      else self.rd, self.scale, seq, pmax, plim=plim, d_v=self.dv, ws=ws)

    def step(self, q, q_idx, w_idx, pos, seq, pmax, plim=None):
        idx = self.select(q_idx, w_idx, pos, seq)
        return self.attend(q, idx, pos, seq, pmax, plim)
