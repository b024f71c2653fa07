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
    rope tables and the sink.  `ratio` is the compression ratio, `topk` the indexer's k."""

    def __init__(self, ring, ckv, k8, ks, sink, cos, sin, ratio: int, topk: int, rd: int = 64, dv: int = 512,
                 eps: float = 1e-6, kbf16=None):
        self.ring, self.ckv, self.k8, self.ks, self.sink = ring, ckv, k8, ks, sink
        self.cos, self.sin = cos, sin
        self.ratio, self.topk, self.rd, self.dv, self.eps = ratio, topk, rd, dv, eps
        self.kbf16 = kbf16
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
                         pos, seq, self.ratio, self.cos, self.sin, self.rd, self.eps, q_idx, w_idx, q8, wf)
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
                   sin=self.sin, rd=self.rd, eps=self.eps, q_idx=q_idx, w_idx=w_idx)
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

    def fused_fits(self, B: int, h: int) -> bool:
        """Whether dsv41_decode_step (the whole layer-step in one launch) takes B rows of h heads here."""
        from ._lib import lib
        dqk = self.ckv.shape[-1]
        dv = 512 if dqk == 576 else dqk
        return bool(lib().dsv41_decode_step_fits(B, self.k8.shape[1] - 1, h, self.topk, self.ring.shape[1], dqk, dv))

    def step_fused(self, q, kv_raw, kv_norm, latent, k_raw, k_norm, pos, seq, q_idx, w_idx, pmax, plim=None,
                   cl=None, idx_out=None, score_out=None, out=None):
        """The whole decode layer-step in one launch (dsv41_decode_step): the cache appends, the indexer (scores +
        top-k) and sattn2 over ring + selected rows -> o [B, 1, h, dv].  The rows' sequences must be distinct and
        fused_fits(B, h) true.  idx_out (int32 [B, k]) / score_out (fp32 [B, >= n_pos]) optionally receive the
        selection and the scores."""
        from ._lib import as_i64, call, lib, ptr, require_gpu, stream
        dev = require_gpu(q, kv_raw, q_idx)
        B, _, h, dqk = q.shape
        dv = 512 if dqk == 576 else dqk
        n_sel = self.k8.shape[1] - 1  # the tables' spare last row is never valid
        if not self.fused_fits(B, h):
            raise RuntimeError(f"step_fused: {B} rows x {h} heads over {n_sel} positions do not fit one launch")
        pos = as_i64(pos.reshape(-1), dev)
        seq = as_i64(seq.reshape(-1), dev)
        pmax = as_i64(pmax.reshape(-1), dev)
        plim = as_i64(plim.reshape(-1), dev) if plim is not None else None
        if cl is None:
            cl = torch.div(pos + 1, self.ratio, rounding_mode="floor")
        cl = as_i64(cl.reshape(-1), dev)
        key = ("step", B, n_sel, h, dv)
        ws = self._attn_ws.get(key)
        if ws is None:
            n = lib().dsv41_decode_step_workspace_bytes(B, n_sel, h, dv)
            ws = self._attn_ws[key] = torch.zeros((n + 255) // 256 * 64, device=dev, dtype=torch.float32)
        nbytes = ws.numel() * 4
        o = out if out is not None else torch.empty(B, 1, h, dv, device=dev, dtype=torch.bfloat16)
        ring, ckv, k8, ks = self.ring, self.ckv, self.k8, self.ks
        Dw = ring.shape[-1]
        x = kv_raw.reshape(B, Dw).contiguous()
        lat = latent.reshape(B, -1).contiguous() if latent is not None else None
        call("dsv41_decode_step", ptr(x), ptr(kv_norm.to(torch.bfloat16).contiguous()), ptr(ring), ring.stride(0),
             ring.shape[1], Dw, ptr(lat), ptr(ckv), ckv.stride(0), ckv.shape[1],
             ptr(k_raw.reshape(B, -1).contiguous()), ptr(k_norm.to(torch.bfloat16).contiguous()), ptr(self.kbf16),
             self.kbf16.stride(0) if self.kbf16 is not None else 0, ptr(k8), k8.stride(0), ptr(ks), ks.stride(0),
             k8.shape[1], ptr(pos), ptr(seq), B, int(self.ratio), ptr(self.cos), ptr(self.sin), int(self.rd),
             float(self.eps), ptr(q_idx.contiguous()), ptr(w_idx.to(torch.bfloat16).contiguous()), q_idx.shape[-2],
             ptr(cl), n_sel, int(self.topk), 0, ptr(q.contiguous()), h, ptr(pmax), ptr(plim), ptr(self.sink),
             0 if dv < dqk else int(self.rd), float(self.scale), ptr(o), ptr(idx_out),
             idx_out.stride(0) if idx_out is not None else 0, ptr(score_out),
             score_out.stride(0) if score_out is not None else 0, ptr(ws), nbytes, stream(dev))
        from . import _lib
        if _lib.CHECK_ERRORS:
            from ._lib import check_error_word
            check_error_word("decode_step", ws.view(torch.int32)[:1])
        return o

    def step(self, q, q_idx, w_idx, pos, seq, pmax, plim=None):
        idx = self.select(q_idx, w_idx, pos, seq)
        return self.attend(q, idx, pos, seq, pmax, plim)
