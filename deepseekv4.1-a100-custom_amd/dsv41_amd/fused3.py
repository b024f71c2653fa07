"""Drop-ins for dsv41/fused3.py: the decode indexer score and the top-k selection, plus the fused decode selector
(score + histogram-assisted multi-workgroup top-k) used by the graph-decode layer step."""
from __future__ import annotations

import torch

from . import _lib
from ._lib import as_i64, call, check_error_word, lib, ptr, require_gpu, stream


def qprep(q: torch.Tensor, weights: torch.Tensor):
    """e4m3 index queries [B, 64, 128] (bytes) + folded head weights [B, 64] fp32 for the e4m3 score path."""
    B, _, H, D = q.shape
    dev = q.device
    q8 = torch.empty(B, 64, 128, dtype=torch.uint8, device=dev)
    wf = torch.empty(B, 64, dtype=torch.float32, device=dev)
    w = weights.reshape(B, H).float().contiguous()
    call("dsv41_index_qprep", ptr(q.contiguous()), ptr(w), B, H, ptr(q8), ptr(wf), stream(dev))
    return q8, wf


def _cand_args(cand, B: int, n_pos: int):
    """(pointer, row stride) of a candidate mask bool/uint8 [B, 1, >= n_pos] or [B, >= n_pos] (None: no mask)."""
    if cand is None:
        return None, 0
    c = cand.reshape(B, -1)
    if c.dtype not in (torch.bool, torch.uint8) or c.shape[1] < n_pos or c.stride(1) != 1:
        raise RuntimeError(f"index_score: candidate mask {tuple(cand.shape)} {cand.dtype} does not cover {n_pos}")
    return ptr(c), c.stride(0)


def _score(q, index_k, weights, seq, cl, k_scale, out, write_masked: bool, hist, prepared=None, cand=None):
    """prepared = (q8, wf) from qprep / decode_appends for e4m3 keys (computed here when None)."""
    B, _, H, D = q.shape
    dev = q.device
    n_pos = index_k.shape[1]
    cp, cs = _cand_args(cand, B, n_pos)
    assert index_k.stride(2) == 1 and index_k.stride(1) == D and D == 128 and H <= 64
    if index_k.dtype == torch.float8_e4m3fn:
        if k_scale is None:
            raise RuntimeError("index_score: e4m3 keys need k_scale")
        ks = k_scale if k_scale.dtype == torch.float32 else k_scale.float()
        assert ks.stride(-1) == 1
        q8, wf = prepared if prepared is not None else qprep(q, weights)
        call("dsv41_index_score", ptr(q8), 64 * 128, ptr(wf), 64, B, H, D, 1, ptr(index_k), index_k.stride(0), ptr(ks),
             ks.stride(0), ptr(seq), 1, ptr(cl), 0, 1, n_pos, int(write_masked), ptr(out), out.stride(0), ptr(hist),
             cp, cs, stream(dev))
    else:
        qc = q.contiguous()
        w = weights.reshape(B, H).float().contiguous()
        call("dsv41_index_score", ptr(qc), H * D, ptr(w), H, B, H, D, 0, ptr(index_k), index_k.stride(0), None, 0,
             ptr(seq), 1, ptr(cl), 0, 1, n_pos, int(write_masked), ptr(out), out.stride(0), ptr(hist), cp, cs,
             stream(dev))


def index_score(q: torch.Tensor, index_k: torch.Tensor, weights: torch.Tensor, seq: torch.Tensor, cl: torch.Tensor,
                cand: torch.Tensor | None = None, k_scale: torch.Tensor | None = None) -> torch.Tensor:
    """dsv41/fused3.py:46-62.  q: bf16 [B, 1, H, D]; index_k: [S, n_pos, D] bf16 (reference storage) or
    float8_e4m3fn with k_scale fp32 [S, n_pos] (per-row scale); weights [B, 1, H] or [B, H] (already scaled);
    seq, cl: int64 [B] -> fp32 [B, n_pos], -inf for t >= cl.  Positions >= cl are not read.  cand: bool [B, 1,
    >= n_pos] (the candidate mask of dsv41/decode.py:311-315): positions that are not candidates score -inf."""
    B, _, H, D = q.shape
    dev = require_gpu(q, index_k, weights)
    out = torch.empty(B, index_k.shape[1], device=dev, dtype=torch.float32)
    _score(q, index_k, weights, as_i64(seq.reshape(-1), dev), as_i64(cl.reshape(-1), dev), k_scale, out, True, None,
           cand=cand)
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


class DecodeSelector:
    """index_score + topk_indices of the graph decode (dsv41/decode.py:289-294) for a fixed (rows, n_pos, k).  With
    e4m3 keys and a grid that fits (rows * ceil(n_sel / 512) <= 512 workgroups, n_sel <= 65536) both run in one
    launch (dsv41_index_select); otherwise the score kernel builds a 4096-bin histogram of the score keys and the
    top-k follows from it (one workgroup per row up to 36864 positions, else a compaction pass plus a finalize).
    Holds the score buffer and the zero-initialised workspaces, which every call leaves ready for the next
    (reusable, graph-capturable).  keep_scores: also write the scores (self.score) on the one-launch path.
    max_cl: the largest valid count cl the caller will pass (the decode tables end with a spare row that cl never
    covers, dsv41/decode.py:176-181, 287); the one-launch path scores and selects positions < n_sel = min(n_pos,
    max_cl) only."""

    def __init__(self, rows: int, n_pos: int, k: int, device, keep_scores: bool = False, max_cl: int | None = None,
                 one_launch_max_chunks: int = 128):
        self.rows, self.n_pos, self.k = rows, n_pos, k
        self.n_sel = n_pos if max_cl is None else max(1, min(n_pos, int(max_cl)))
        nbytes = lib().dsv41_select_workspace_bytes(rows, n_pos)
        self.ws = torch.zeros(nbytes // 4, dtype=torch.int32, device=device)
        self.nbytes = nbytes
        ld = (n_pos + 3) // 4 * 4  # 16-byte aligned rows: the selection reads float4
        self.score = torch.empty(rows, ld, dtype=torch.float32, device=device)[:, :n_pos]
        self.out = torch.empty(rows, 1, k, dtype=torch.int32, device=device)
        ns = (self.n_sel + 511) // 512
        # one launch up to 128 chunks per row: every chunk's workgroup gathers all chunks' counts and candidate
        # prefixes, so past that the multi-launch path is faster (C4, 512 chunks: 82 us one launch vs ~49 us)
        self.one_launch = ns <= min(int(one_launch_max_chunks), 512) and rows * ns <= 512
        self.keep_scores = keep_scores
        if self.one_launch:
            self.fnbytes = lib().dsv41_index_select_workspace_bytes(rows, self.n_sel)
            self.fws = torch.zeros(self.fnbytes // 4, dtype=torch.int32, device=device)

    def score_into(self, q, index_k, weights, seq, cl, k_scale=None, prepared=None, cand=None) -> None:
        """The score kernel alone (scores + histogram into this object's buffers)."""
        require_gpu(q, index_k, weights)
        B = q.shape[0]
        if B != self.rows or index_k.shape[1] != self.n_pos:
            raise RuntimeError(f"DecodeSelector built for {self.rows} x {self.n_pos}, got {B} x {index_k.shape[1]}")
        _score(q, index_k, weights, seq, cl, k_scale, self.score, False, self.ws, prepared, cand=cand)

    def select(self, cl) -> torch.Tensor:
        """Top-k from the buffered scores + histogram; leaves the histogram zeroed."""
        call("dsv41_select_topk", ptr(self.score), self.score.stride(0), self.rows, self.n_pos, self.k, ptr(cl), 0,
             ptr(self.ws), self.nbytes, ptr(self.out), self.k, stream(self.score.device))
        if _lib.CHECK_ERRORS:
            self.check()
        return self.out

    def check(self) -> None:
        """Raise RuntimeError (and clear the word) when the last launch reported an error through its workspace: a row
        barrier that gave up, or a cl clamped to the positions scored.  Synchronises."""
        check_error_word("index_select", self.ws[-4:-3])
        if self.one_launch:
            check_error_word("index_select", self.fws[-4:-3])

    def select_one_launch(self, q8, wf, H: int, index_k, k_scale, seq, cl, cand=None) -> torch.Tensor:
        """Scores + top-k in one launch from the prepared e4m3 queries (q8, wf)."""
        ks = k_scale if k_scale.dtype == torch.float32 else k_scale.float()
        cp, cs = _cand_args(cand, self.rows, self.n_sel)
        call("dsv41_index_select", ptr(q8), 64 * 128, ptr(wf), 64, self.rows, H, ptr(index_k), index_k.stride(0),
             ptr(ks), ks.stride(0), ptr(seq), ptr(cl), self.n_sel, self.k, 0, ptr(self.fws), self.fnbytes,
             ptr(self.score) if self.keep_scores else None, self.score.stride(0), ptr(self.out), self.k, cp, cs,
             stream(self.score.device))
        if _lib.CHECK_ERRORS:
            self.check()
        return self.out

    def select_with_appends(self, app: dict, pos, seq, cl, cand=None) -> torch.Tensor:
        """The decode step's cache appends and scores + top-k: in one launch (dsv41_decode_select) when the selection
        fits one, else the appends and the scores with their histogram in one launch (dsv41_decode_score) and the
        top-k after it.  app: the arguments of cache.decode_appends as keywords (kv_raw, kv_norm, ring, latent, ckv,
        k_raw, k_norm, kbf, k8, k_scale, ratio, cos, sin, rd, eps, q_idx [B, 1, HI, 128], w_idx [B, HI], optional
        nw_tab: int64 [S] no-write row per sequence, dsv41/decode.py:176-181); the rows' sequences must be distinct.  The keys scored are app["k8"] / app["k_scale"]."""
        dev = self.score.device
        ring, ckv, k8, ks, kbf = app["ring"], app.get("ckv"), app["k8"], app["k_scale"], app.get("kbf")
        Dw = ring.shape[-1]
        x = app["kv_raw"].reshape(-1, Dw).contiguous()
        B = x.shape[0]
        if B != self.rows or k8.shape[1] != self.n_pos or k8.shape[-1] != 128:
            raise RuntimeError(f"select_with_appends: built for {self.rows} x {self.n_pos}, got {B} x {k8.shape[1]}")
        lat = app["latent"].reshape(B, -1).contiguous() if app.get("latent") is not None else None
        q_idx, w_idx = app["q_idx"], app["w_idx"]
        HI = q_idx.shape[-2]
        assert ring.stride(2) == 1 and ring.stride(1) == Dw and ks.dtype == torch.float32
        nw = app.get("nw_tab")
        nw = as_i64(nw.reshape(-1), dev) if nw is not None else None
        if not self.one_launch:
            cp, cs = _cand_args(cand, self.rows, self.n_pos)
            call("dsv41_decode_score", ptr(x), ptr(app["kv_norm"].to(torch.bfloat16).contiguous()), ptr(ring),
                 ring.stride(0), ring.shape[1], Dw, ptr(lat), ptr(ckv), ckv.stride(0) if ckv is not None else 0,
                 ckv.shape[1] if ckv is not None else 1, ptr(app["k_raw"].reshape(B, -1).contiguous()),
                 ptr(app["k_norm"].to(torch.bfloat16).contiguous()), ptr(kbf),
                 kbf.stride(0) if kbf is not None else 0, ptr(k8), k8.stride(0), ptr(ks), ks.stride(0), k8.shape[1],
                 ptr(pos), ptr(seq), ptr(nw), B, int(app["ratio"]), ptr(app["cos"]), ptr(app["sin"]),
                 int(app["rd"]), float(app["eps"]), ptr(q_idx.contiguous()), ptr(w_idx.to(torch.bfloat16).contiguous()), HI, ptr(cl),
                 self.n_pos, ptr(self.score), self.score.stride(0), ptr(self.ws), cp, cs, stream(dev))
            return self.select(cl)
        cp, cs = _cand_args(cand, self.rows, self.n_sel)
        call("dsv41_decode_select", ptr(x), ptr(app["kv_norm"].to(torch.bfloat16).contiguous()), ptr(ring),
             ring.stride(0), ring.shape[1], Dw, ptr(lat), ptr(ckv), ckv.stride(0) if ckv is not None else 0,
             ckv.shape[1] if ckv is not None else 1, ptr(app["k_raw"].reshape(B, -1).contiguous()),
             ptr(app["k_norm"].to(torch.bfloat16).contiguous()), ptr(kbf), kbf.stride(0) if kbf is not None else 0,
             ptr(k8), k8.stride(0), ptr(ks), ks.stride(0), k8.shape[1], ptr(pos), ptr(seq), ptr(nw), B,
             int(app["ratio"]), ptr(app["cos"]), ptr(app["sin"]), int(app["rd"]), float(app["eps"]),
             ptr(q_idx.contiguous()),
             ptr(w_idx.to(torch.bfloat16).contiguous()), HI, ptr(cl), self.n_sel, self.k, 0, ptr(self.fws),
             self.fnbytes, ptr(self.score) if self.keep_scores else None, self.score.stride(0), ptr(self.out), self.k,
             cp, cs, stream(dev))
        if _lib.CHECK_ERRORS:
            self.check()
        return self.out

    def __call__(self, q, index_k, weights, seq, cl, k_scale=None, prepared=None, cand=None) -> torch.Tensor:
        dev = require_gpu(q, index_k, weights)
        seq = as_i64(seq.reshape(-1), dev)
        cl = as_i64(cl.reshape(-1), dev)
        if self.one_launch and index_k.dtype == torch.float8_e4m3fn and k_scale is not None:
            if q.shape[0] != self.rows or index_k.shape[1] != self.n_pos:
                raise RuntimeError(f"DecodeSelector built for {self.rows} x {self.n_pos}, got {q.shape[0]} x "
                                   f"{index_k.shape[1]}")
            q8, wf = prepared if prepared is not None else qprep(q, weights)
            return self.select_one_launch(q8, wf, q.shape[2], index_k, k_scale, seq, cl, cand)
        self.score_into(q, index_k, weights, seq, cl, k_scale, prepared, cand)
        return self.select(cl)
