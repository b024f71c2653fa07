"""GPU parity of the decode appends under per-slot cache capacities (the reference's DSV41_SLOT_CAPS layout,
dsv41/slots.py:1-11): the compressed-KV and index-key tables are one flat buffer per layer in which slot s owns
k_s consecutive units of U rows, seen through an as_strided view [n_units, max_rows, D] whose slot stride is ONE
unit.  A step that closes no compression group writes the slot's own no-write row (the last row of its capacity,
dsv41/decode.py:62-68, :176-181), not the view's last row, which for a small slot lies inside the next slot's live
rows.  Every fused append path (dsv41_decode_appends, dsv41_decode_select, dsv41_decode_score) is checked against
the oracle: the intended rows written, every other row of the flat buffers bit-unchanged, and the selection of the
fused indexer paths against the oracle's scores over the final tables."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
U, D, DI, W, RATIO, RD, K = 64, 576, 128, 128, 4, 64, 16


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(O.bf16(x))).to(torch.bfloat16).to(DEV)


def _i64(x):
    return torch.tensor(np.asarray(x, np.int64), device=DEV)


def _fp8_close(got, want, tag):
    """Quantised rows: identical except for rare one-step flips (fp32 rmsnorm reduction order)."""
    diff = got != want
    print(f"[{tag}] mismatching elements {diff.sum()} ({diff.mean():.2e})", flush=True)
    assert diff.mean() <= 2e-3, tag
    if diff.any():
        rel = np.abs(got[diff] - want[diff]) / np.maximum(np.abs(want[diff]), 1e-30)
        assert rel.max() <= 0.34, (tag, rel.max())


def _setup(seed):
    """Two sequences: A = unit 0 (capacity U rows), B = units 1-2 (capacity 2U rows); flat buffers of 3U rows."""
    r = np.random.default_rng(seed)
    n_flat = 3 * U
    ckv0 = O.bf16(r.standard_normal((n_flat, D)).astype(np.float32) * 0.1)
    kbf0 = O.bf16(O.fake_quant_fp4(r.standard_normal((n_flat, DI)).astype(np.float32) * 0.1, 32))
    kq, ksc = O.key_encode_fp8(kbf0)
    flat = {"ckv": _bf(ckv0), "k8": torch.from_numpy(kq).to(torch.float8_e4m3fn).to(DEV),
            "ks": torch.from_numpy(ksc[:, 0].copy()).to(DEV)}
    view = {"ckv": flat["ckv"].as_strided((2, 2 * U, D), (U * D, D, 1)),
            "k8": flat["k8"].as_strided((2, 2 * U, DI), (U * DI, DI, 1)),
            "ks": flat["ks"].as_strided((2, 2 * U), (U, 1))}
    nw_tab = _i64([U - 1, 2 * U - 1])  # seq 0 -> flat row U - 1; seq 1 -> flat row U + 2U - 1
    return r, flat, view, nw_tab, ckv0, kbf0


@pytest.mark.parametrize("path", ["appends", "select", "score"])
def test_slot_caps_no_write_rows(path):
    from dsv41_amd.decode import DecodeLayer
    r, flat, view, nw_tab, ckv0, kbf0 = _setup(21)
    cos, sin = O.rope_tables(RD, 4096, 0, 10000.0, 1.0, 32, 1)
    ring = _bf(np.zeros((2, W, D), np.float32))
    sink = torch.zeros(64, device=DEV)
    lay = DecodeLayer(ring, view["ckv"], view["k8"], view["ks"], sink, torch.from_numpy(cos).to(DEV),
                      torch.from_numpy(sin).to(DEV), RATIO, K, rd=RD, nw_tab=nw_tab)
    want_c, want_k = ckv0.copy(), kbf0.copy()
    seq = [0, 1]
    # step 0: neither row closes a group (A's no-write row U-1 lies below B's live rows; the view's last row 2U-1
    # would be flat row 2U-1 = B's live position U-1); step 1: B closes its group at compressed row 100
    for step, pos in enumerate([[161, 402], [165, 403]]):
        kv_raw = O.bf16(r.standard_normal((2, D)).astype(np.float32))
        kvn = O.bf16(r.random(D).astype(np.float32) + 0.5)
        lat = O.bf16(r.standard_normal((2, 1, D)).astype(np.float32))
        kraw = O.bf16(r.standard_normal((2, DI)).astype(np.float32) * 2)
        kn = O.bf16(r.random(DI).astype(np.float32) + 0.5)
        q_idx = O.bf16(O.fake_quant_fp4(r.standard_normal((2, 1, 64, DI)).astype(np.float32), 32))
        w_idx = O.bf16(r.standard_normal((2, 64)).astype(np.float32) * 0.05)
        cl = [(p + 1) // RATIO for p in pos]
        print(f"[slot caps] path {path} step {step} pos {pos} cl {cl}", flush=True)
        args = (_bf(kv_raw), _bf(kvn), _bf(lat), _bf(kraw), _bf(kn), _i64(pos), _i64(seq), _bf(q_idx), _bf(w_idx))
        sel = lay.selector(2, DEV)
        sel.keep_scores = True
        if path == "appends":
            lay.appends(*args)
        else:
            if path == "score":
                sel.one_launch = False
            idx = lay.appends_select(*args, cl=_i64(cl)).clone()
        torch.cuda.synchronize()
        for i in range(2):
            p = pos[i]
            unit0 = 0 if seq[i] == 0 else U  # first flat row of the sequence's units
            row = (p + 1) // RATIO - 1 if (p + 1) % RATIO == 0 else [U - 1, 2 * U - 1][i]
            p0 = np.int64(p + 1 - RATIO)
            want_c[unit0 + row] = O.compress_row(lat[i, 0], cos, sin, p0, RD)
            want_k[unit0 + row] = O.index_key_row(kraw[i], kn, cos, sin, p0, RD, 1e-6)
        got_c = flat["ckv"].float().cpu().numpy()
        got_k = (flat["k8"].float() * flat["ks"][:, None]).cpu().numpy()
        changed = np.flatnonzero((want_c != ckv0).any(axis=1) | (want_k != kbf0).any(axis=1))
        keep = np.setdiff1d(np.arange(3 * U), changed)
        # rows no step meant to write: bit-unchanged (the neighbour slot's live rows included)
        np.testing.assert_array_equal(got_c[keep], ckv0[keep], err_msg=f"step {step}: compressed rows clobbered")
        np.testing.assert_array_equal(got_k[keep], kbf0[keep], err_msg=f"step {step}: index-key rows clobbered")
        assert 2 * U - 1 in keep, "B's live row under the view's last row must be among the untouched rows"
        _fp8_close(got_c[changed], want_c[changed], f"{path} step {step} compressed rows")
        _fp8_close(got_k[changed], want_k[changed], f"{path} step {step} index-key rows")
        if path != "appends":
            # scores of the final tables (the kernel's own written rows) against the oracle; the selection bit-exact
            # against the oracle's top-k of the kernel's scores
            k8v = view["k8"].float().cpu().numpy()
            ksv = view["ks"].cpu().numpy()
            sc_ref = O.index_score(q_idx, k8v, w_idx, seq, cl, k_scale=ksv)
            sc = sel.score.cpu().numpy()
            for i in range(2):
                c = cl[i]
                rel = np.abs(sc[i, :c] - sc_ref[i, :c]).max() / np.abs(sc_ref[i, :c]).max()
                assert rel <= 1e-2, (path, step, i, rel)
            want_idx = O.topk_indices(np.where(np.arange(sc.shape[1]) < np.array(cl)[:, None], sc, -np.inf), K, cl)
            np.testing.assert_array_equal(idx.cpu().numpy().reshape(2, K), want_idx, err_msg=f"{path} step {step}")
