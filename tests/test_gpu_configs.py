"""GPU parity of the decode layer-step at the BASELINE configs' real shapes, through the production path the bench
times (DecodeLayer: the appends, the indexer launches, the attention launches), against the oracle.

C5: 8 slots with contexts {524288, 131072 x 3, 65536, 32768, 8192, 2048}, 6 query rows each (1 + 5 MTP drafts at
positions p-5 .. p, causal among drafts: plim = the row's own position, dsv41/fused2.py:355-360), k 2048 (the
reference's verify shape, dsv41/engine.py:4947).  Production kernels: decode_appends_kernel, the draft-row group
score kernel, the chunk compaction + finalize top-k, the 64-head key-split attention + combine.
C4: 1 slot of 262144 compressed positions: the appends + scores in one launch (dsv41_decode_score), the two-launch
top-k and the decode attention over a 262144-row table.

Bars: every row's selection bit-exact against the oracle's top-k of the kernel's own scores; scores within 1e-2 of
the oracle's on sampled rows (every row of C4); attention within 2e-2 max / 2e-3 mean on >= 8 sampled rows (the
oracle's CPU time bounds the sample)."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ATT_MAX, ATT_MEAN = 2e-2, 2e-3


def _layer(name, seed):
    from dsv41_amd.decode import DecodeLayer
    from dsv41_amd.workloads import CONFIGS, make_decode_inputs
    cfg = CONFIGS[name]
    layers, st = make_decode_inputs(cfg, DEV, seed=seed)
    rd = 64
    ang = torch.outer(torch.arange(max(cfg.ctx) + 8, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    l0 = layers[0]
    lay = DecodeLayer(l0["ring"], l0["ckv"], l0["k8"], l0["ks"], st["sink"], cos, sin, cfg.ratio, cfg.topk, rd=rd)
    return cfg, lay, st


def _check_rows(cfg, lay, st, idx, score, o, score_rows, attn_rows, tag):
    """Selection of every row against the oracle's top-k of the kernel's scores; the sampled rows' scores and
    attention against the oracle over the tables as the step left them."""
    pos = st["pos"].cpu().numpy()
    seq = st["seq"].cpu().numpy()
    cl = (pos + 1) // cfg.ratio
    idx = idx.reshape(len(pos), -1).cpu().numpy()
    sc = score.cpu().numpy()
    for r in range(len(pos)):
        want = O.topk_indices(sc[r:r + 1, :cl[r]], cfg.topk, [cl[r]])[0]
        np.testing.assert_array_equal(idx[r], want, err_msg=f"{tag} row {r} (slot {seq[r]}, cl {cl[r]})")
    qi = st["q_idx"].float().cpu().numpy()
    w = st["w_idx"].float().cpu().numpy()
    for r in score_rows:
        s = int(seq[r])
        k8 = lay.k8[s, :cl[r]].float().cpu().numpy()
        ks = lay.ks[s, :cl[r]].cpu().numpy()
        ref = O.index_score(qi[r:r + 1], k8[None], w[r:r + 1], [0], [cl[r]], k_scale=ks[None])[0]
        rel = np.abs(sc[r, :cl[r]] - ref).max() / np.abs(ref).max()
        print(f"[{tag}] row {r} score rel err {rel:.2e}", flush=True)
        assert rel <= 1e-2, (tag, r, rel)
    q = st["q"].float().cpu().numpy()
    sink = st["sink"].cpu().numpy()
    pmax = st["pmax"].cpu().numpy()
    got = o.float().cpu().numpy()
    for r in attn_rows:
        s = int(seq[r])
        ix = torch.from_numpy(idx[r]).long().to(DEV)
        rows = lay.ckv[s][ix.clamp_min(0)].float().cpu().numpy()  # the gathered rows, remapped to 0..k-1
        local = np.where(idx[r] >= 0, np.arange(cfg.topk), -1)
        want = O.sattn2(q[r:r + 1], lay.ring[s:s + 1].float().cpu().numpy(), rows[None], local[None], [pos[r]],
                        [0], [pmax[r]], [pos[r]], sink, None, None, 0, lay.scale, dv=lay.dv)
        err = np.abs(got[r] - want[0])
        print(f"[{tag}] row {r} attention max {err.max():.3e} mean {err.mean():.3e}", flush=True)
        assert err.max() <= ATT_MAX and err.mean() <= ATT_MEAN, (tag, r, err.max(), err.mean())


def test_c5_real_contexts():
    cfg, lay, st = _layer("C5", 31)
    R = cfg.slots * cfg.rows_per_slot
    pos, seq = st["pos"], st["seq"]
    print(f"[C5] {R} rows, contexts {cfg.ctx}", flush=True)
    lay.appends(st["kv_raw"], st["kv_norm"], st["latent"], st["k_raw"], st["k_norm"], pos, seq, st["q_idx"],
                st["w_idx"])
    idx = lay.select(st["q_idx"], st["w_idx"], pos, seq).clone()
    o = lay.attend(st["q"], idx, pos, seq, st["pmax"], plim=pos)
    torch.cuda.synchronize()
    lay.check()
    sel = lay.selector(R, DEV)
    assert not sel.one_launch
    # scores: the first and last draft of the longest slot, one row of each other length; attention: 10 rows
    # spread over every context length (first / last draft of the long slots)
    score_rows = [0, 5, 8, 21, 26, 33, 40, 47]
    attn_rows = [0, 5, 6, 17, 24, 29, 31, 36, 42, 47]
    _check_rows(cfg, lay, st, idx, sel.score, o[:, 0], score_rows, attn_rows, "C5")


def test_c4_fused_score_path():
    cfg, lay, st = _layer("C4", 32)
    pos, seq = st["pos"], st["seq"]
    sel = lay.selector(1, DEV)
    assert not sel.one_launch  # 512 chunks: dsv41_decode_score + the two-launch top-k
    print(f"[C4] 1 row over {lay.k8.shape[1] - 1} positions", flush=True)
    idx = lay.appends_select(st["kv_raw"], st["kv_norm"], st["latent"], st["k_raw"], st["k_norm"], pos, seq,
                             st["q_idx"], st["w_idx"]).clone()
    o = lay.attend(st["q"], idx, pos, seq, st["pmax"], plim=pos)
    torch.cuda.synchronize()
    lay.check()
    _check_rows(cfg, lay, st, idx, sel.score, o[:, 0], [0], [0], "C4")
