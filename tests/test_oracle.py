"""Pins the CPU oracle (oracle/dsv41_oracle.py) against known answers, library routines, closed forms and brute
force -- never against a retyped copy of its own formula.  CPU only."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def test_bf16_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0,
                        np.array([0.0, -0.0, 1e-40, 3.4e38, 1.00390625, 1.01171875], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16(x), ref)


def test_round_e4m3_known_and_torch():
    np.testing.assert_array_equal(O.round_e4m3(np.array(GOLD["round_e4m3_in"], np.float32)),
                                  np.array(GOLD["round_e4m3_out"], np.float32))
    rng = np.random.default_rng(1)
    x = np.clip(rng.standard_normal(65536).astype(np.float32) * np.exp2(rng.integers(-12, 9, 65536)), -448, 448)
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(O.round_e4m3(x), ref)
    # every e4m3 value is a fixed point
    allv = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    allv = allv[np.isfinite(allv)]
    np.testing.assert_array_equal(O.round_e4m3(allv), allv)


def test_round_e2m1_known_answers():
    np.testing.assert_array_equal(O.round_e2m1(np.array(GOLD["round_e2m1_in"], np.float32)),
                                  np.array(GOLD["round_e2m1_out"], np.float32))
    g = np.array(GOLD["e2m1_grid"], np.float32)
    np.testing.assert_array_equal(O.round_e2m1(g), g)


def test_ceil_log2_known():
    np.testing.assert_array_equal(O.ceil_log2(np.array(GOLD["ceil_log2_in"], np.float32)), GOLD["ceil_log2_out"])
    for v in [1e-30, 0.3, 1.0, 7.0, 1e20]:
        assert int(O.ceil_log2(np.array([v], np.float32))[0]) == math.ceil(math.log2(np.float32(v)))


def test_fake_quant_fp8_against_library_cast():
    rng = np.random.default_rng(2)
    x = O.bf16(rng.standard_normal((64, 256)).astype(np.float32) * 3)
    y = O.fake_quant_fp8(x, 32)
    g = x.reshape(-1, 32)
    amax = np.maximum(np.abs(g).max(1, keepdims=True), 1e-4)
    s = np.exp2(np.ceil(np.log2(amax.astype(np.float64) / 448.0))).astype(np.float32)
    ref = torch.from_numpy(np.clip(g / s, -448, 448)).to(torch.float8_e4m3fn).float().numpy() * s
    np.testing.assert_array_equal(y.reshape(-1, 32), ref)
    np.testing.assert_array_equal(O.fake_quant_fp8(y, 32), y)  # idempotent
    row = ((np.arange(32) - 15.5) * 0.25).astype(np.float32)
    q = O.fake_quant_fp8(row, 32)
    assert GOLD["fake_quant_fp8_row"]["scale"] == 0.015625
    # |v| < 2: at most 4 significant bits at scale 2^-6 -> exact; above 2 the e4m3 ulp (16 x 2^-6) rounds to even
    np.testing.assert_array_equal(q[8:24], row[8:24])
    np.testing.assert_array_equal(q[:8], [-4.0, -3.5, -3.5, -3.0, -3.0, -2.5, -2.5, -2.0])


@pytest.mark.parametrize("scale_e4m3,block", [(False, 32), (True, 16)])
def test_fake_quant_fp4_grid_and_idempotence(scale_e4m3, block):
    rng = np.random.default_rng(3)
    x = O.bf16(rng.standard_normal((32, 576)).astype(np.float32))
    y = O.fake_quant_fp4(x, block, scale_e4m3)
    g = y.reshape(-1, block)
    xg = x.reshape(-1, block)
    amax = np.abs(xg).max(1, keepdims=True)
    if scale_e4m3:
        s = torch.from_numpy(np.maximum(amax, 6 * 2.0 ** -9).astype(np.float32) / 6).to(torch.float8_e4m3fn)
        s = s.float().numpy()
    else:
        s = np.exp2(np.ceil(np.log2(amax.astype(np.float64) / 6.0))).astype(np.float32)
    q = g / s
    grid = np.array(GOLD["e2m1_grid"], np.float32)
    assert np.isin(q, grid).all()
    # nearest grid value (brute force over the grid); ties to the even code
    xs = np.clip(xg / s, -6, 6)
    d = np.abs(xs[..., None] - grid[None, None, :])
    best = d.min(-1)
    assert np.all(np.abs(np.abs(xs - q) - best) <= 1e-6)
    np.testing.assert_array_equal(O.fake_quant_fp4(y, block, scale_e4m3), y)


def test_key_encode_fp8_exact_on_fp4_grid_rows():
    rng = np.random.default_rng(4)
    k = O.bf16(O.fake_quant_fp4(O.bf16(rng.standard_normal((512, 128)).astype(np.float32) * 0.1), 32))
    q, s = O.key_encode_fp8(k)
    np.testing.assert_array_equal(q * s, k)
    ref = torch.from_numpy(q).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(ref, q)


def test_rope_against_complex_rotation_and_inverse():
    cos, sin = O.rope_tables(64, 4096, 65536, 160000.0, 16.0, 32, 1)
    rng = np.random.default_rng(5)
    x = O.bf16(rng.standard_normal((3, 512)).astype(np.float32))
    pos = np.array([100, 101, 102])
    y = O.rope(x, cos, sin, pos, 64)
    z = x[:, -64:].reshape(3, 32, 2)
    c = (z[..., 0] + 1j * z[..., 1]) * (cos[pos] + 1j * sin[pos])
    ref = np.stack([c.real, c.imag], -1).reshape(3, 64)
    np.testing.assert_allclose(y[:, -64:], ref, atol=0.02, rtol=0.01)
    np.testing.assert_array_equal(y[:, :-64], x[:, :-64])
    back = O.rope(y, cos, sin, pos, 64, inverse=True)
    np.testing.assert_allclose(back, x, atol=0.03)
    # the table itself: angle = pos * freq with freq from the YaRN ramp; pos 0 is the identity
    np.testing.assert_array_equal(cos[0], np.ones(32, np.float32))
    np.testing.assert_array_equal(sin[0], np.zeros(32, np.float32))


def test_rope_tables_yarn_ramp():
    """The YaRN correction of rope_tables (dsv41/model.py:76-117), from the table's angle at position 1: frequency
    pairs below the fast correction dimension keep base^(-2i/d), those at or above the slow one are divided by
    `factor`, and the ratio to base^(-2i/d) falls monotonically from 1 to 1/factor in between (YaRN, Peng et al.
    2023, section 3.2: the correction dimension of r rotations is d ln(L / (2 pi r)) / (2 ln base))."""
    import math
    dim, L, base, factor = 64, 65536, 160000.0, 16.0
    cos, sin = O.rope_tables(dim, 8, L, base, factor, 32, 1)
    freq = np.arctan2(sin[1].astype(np.float64), cos[1].astype(np.float64))
    plain = base ** (-np.arange(0, dim, 2) / dim)
    ratio = freq / plain
    cd = lambda rot: dim * math.log(L / (rot * 2 * math.pi)) / (2 * math.log(base))  # noqa: E731
    low, high = math.floor(cd(32)), math.ceil(cd(1))
    assert 0 < low < high < dim // 2
    np.testing.assert_allclose(ratio[:low + 1], 1.0, rtol=1e-5)
    np.testing.assert_allclose(ratio[high:], 1.0 / factor, rtol=1e-5)
    mid = ratio[low:high + 1]
    assert np.all(np.diff(mid) < 0) and 1.0 / factor < mid[1:-1].min() and mid[1:-1].max() < 1.0
    # no correction without an original length: the plain table
    cos0, sin0 = O.rope_tables(dim, 8, 0, base, factor, 32, 1)
    np.testing.assert_allclose(np.arctan2(sin0[1], cos0[1]), plain, rtol=1e-5)


@pytest.mark.parametrize("start", [0, 3, 127, 128, 300])
def test_window_idx_brute_force(start):
    W, S = 128, 7
    idx = O.window_idx(W, S, start)
    for i in range(S):
        q = start + i
        if start == 0:
            want = [p for p in range(max(0, q - W + 1), q + 1)]
            got = [v for v in idx[i] if v >= 0]
            assert got == want
        else:
            want = sorted(p % W for p in range(max(0, q - W + 1), q + 1))
            got = sorted(v for v in idx[i] if v >= 0)
            assert got == want


@pytest.mark.parametrize("pos,pmax,plim", [(50, 50, 50), (300, 300, 300), (301, 305, 301), (0, 0, 0), (130, 135, 132)])
def test_ring_valid_brute_force(pos, pmax, plim):
    W = 128
    v = O.ring_valid(pos, pmax, plim, W)
    # brute force: slot s holds the newest position p <= pmax with p % W == s
    for s in range(W):
        held = max([p for p in range(0, pmax + 1) if p % W == s], default=-1)
        want = held >= 0 and held <= plim and pos - held < W
        assert bool(v[s]) == want


def _dense_attn(q, rows, valid, sink, scale):
    """Dense softmax over [scores ; sink], sink column dropped after the softmax (dsv41/test_kernels.py:40-49)."""
    sc = (q.astype(np.float64) @ rows.astype(np.float64).T) * scale
    sc = np.where(valid[None, :], sc, -np.inf)
    sc = np.concatenate([sc, sink[:, None].astype(np.float64)], 1)
    sc = sc - sc.max(1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(1, keepdims=True)
    return p[:, :-1] @ rows.astype(np.float64)


def test_sparse_attn_vs_dense_softmax():
    rng = np.random.default_rng(6)
    b, s, h, d, n = 1, 5, 4, 64, 40
    q = O.bf16(rng.standard_normal((b, s, h, d)).astype(np.float32))
    kv = O.bf16(rng.standard_normal((b, n, d)).astype(np.float32))
    sink = rng.standard_normal(h).astype(np.float32)
    idx = rng.integers(0, n, (b, s, 8)).astype(np.int32)
    idx[0, 0, :3] = -1
    o = O.sparse_attn(q, kv, sink, idx, d ** -0.5)
    for i in range(s):
        sel = idx[0, i]
        ref = _dense_attn(q[0, i], kv[0, np.maximum(sel, 0)], sel >= 0, sink, d ** -0.5)
        np.testing.assert_allclose(o[0, i], ref, atol=2e-2)
    # all-invalid row -> zeros
    idx2 = np.full((1, 1, 8), -1, np.int32)
    assert np.all(O.sparse_attn(q[:, :1], kv, sink, idx2, 0.1) == 0)


def test_sattn2_equals_decode_over_explicit_indices():
    rng = np.random.default_rng(7)
    H, d, W, rd = 16, 64, 32, 16
    cos, sin = O.rope_tables(rd, 1024, 0, 10000.0, 1.0, 32, 1)
    q = O.bf16(rng.standard_normal((1, 1, H, d)).astype(np.float32))
    ring = O.bf16(rng.standard_normal((1, W, d)).astype(np.float32))
    ckv = O.bf16(rng.standard_normal((1, 300, d)).astype(np.float32))
    sink = rng.standard_normal(H).astype(np.float32)
    for p in (10, 100):
        idx = rng.integers(0, 150, (1, 1, 48)).astype(np.int32)
        idx[..., 40:] = -1
        o = O.sattn2(q, ring, ckv, idx, [p], [0], [p], None, sink, cos, sin, rd, d ** -0.5)
        slot = p % W
        widx = (np.arange(W) + slot + 1) % W
        widx = np.where(widx > p, -1, widx).astype(np.int32)
        full = np.concatenate([widx, np.where(idx[0, 0] >= 0, idx[0, 0] + W, -1)])[None, None]
        ref = O.sparse_attn_decode2(q, ring, ckv, sink, full, d ** -0.5)
        ref = O.rope(ref[0, 0], cos, sin, np.int64(p), rd, inverse=True)
        np.testing.assert_allclose(o[0, 0], ref, atol=1e-6)
        # split invariance: two halves merged by log-sum-exp == single pass (dsv41/test_fused.py:90-94)
        rows = np.concatenate([ring[0], ckv[0][np.maximum(idx[0, 0], 0)]])
        valid = np.concatenate([O.ring_valid(p, p, p, W), idx[0, 0] >= 0])
        sc = (q[0, 0] @ rows.T) * d ** -0.5
        sc = np.where(valid[None], sc, -1e30)
        parts = []
        for a, b in ((0, 40), (40, rows.shape[0])):
            m = sc[:, a:b].max(1)
            pp = np.where(valid[None, a:b], np.exp(sc[:, a:b] - m[:, None]), 0)
            parts.append((m, pp.sum(1), pp @ rows[a:b]))
        mx = np.maximum(parts[0][0], parts[1][0])
        num = sum(np.exp(m - mx)[:, None] * acc for m, l, acc in parts)
        den = sum(np.exp(m - mx) * l for m, l, acc in parts) + np.exp(sink - mx)
        merged = O.rope(O.bf16(num / den[:, None]), cos, sin, np.int64(p), rd, inverse=True)
        np.testing.assert_allclose(o[0, 0], merged, atol=2e-2)


def test_index_score_brute_force_and_chunk_invariance():
    rng = np.random.default_rng(8)
    B, H, D, n = 2, 8, 128, 50
    q = rng.standard_normal((B, 1, H, D)).astype(np.float32)
    keys = rng.standard_normal((3, n, D)).astype(np.float32)
    w = rng.standard_normal((B, H)).astype(np.float32)
    seq = [2, 0]
    cl = [37, 50]
    s = O.index_score(q, keys, w, seq, cl)
    for b in range(B):
        for t in range(n):
            if t >= cl[b]:
                assert s[b, t] == -np.inf
                continue
            ref = sum(float(w[b, h]) * max(0.0, float(np.dot(q[b, 0, h].astype(np.float64), keys[seq[b], t])))
                      for h in range(H))
            assert abs(s[b, t] - ref) <= 1e-4 * (1 + abs(ref))
    # prefill: chunked == full exactly (dsv41/test_long_prefill.py:66-96)
    qp = O.bf16(rng.standard_normal((1, 40, H, D)).astype(np.float32))
    wp = rng.standard_normal((1, 40, H)).astype(np.float32)
    kp = O.bf16(rng.standard_normal((1, 60, D)).astype(np.float32))
    a = O.indexer_prefill(qp, wp, kp, 200, 4, 16, 128, query_chunk=7)
    b = O.indexer_prefill(qp, wp, kp, 200, 4, 16, 128, query_chunk=1000)
    np.testing.assert_array_equal(a, b)


def test_topk_brute_force():
    rng = np.random.default_rng(9)
    for n, k, cl in [(100, 10, 100), (100, 10, 60), (100, 10, 7), (1000, 64, 999), (37, 37, 37)]:
        sc = rng.standard_normal((3, n)).astype(np.float32)
        sc[1, ::3] = sc[1, 0]  # ties
        out = O.topk_indices(sc, k, [cl] * 3)
        for r in range(3):
            c = min(cl, n)
            want = sorted(sorted(range(c), key=lambda i: (-float(sc[r, i]), i))[:k])
            want = want + [-1] * (k - len(want))
            assert out[r].tolist() == want
    for name in ("topk_ties", "topk_cl_short", "topk_negzero"):
        g = GOLD[name]
        out = O.topk_indices(np.array([g["score"]], np.float32), g["k"], [g["cl"]])
        assert out[0].tolist() == g["out"], name


def test_kv_write_composition():
    rng = np.random.default_rng(10)
    d, W, rd = 512, 128, 64
    cos, sin = O.rope_tables(rd, 4096, 0, 10000.0, 1.0, 32, 1)
    x = O.bf16(rng.standard_normal((2, d)).astype(np.float32) * 2)
    w = O.bf16(rng.random(d).astype(np.float32) + 0.5)
    cache = np.zeros((3, W, d), np.float32)
    out = O.kv_write(x, w, cos, sin, [300, 5], [2, 0], cache, rd, 1e-6)
    row = O.rope(O.bf16(O.rmsnorm(x[0:1], w, 1e-6)), cos, sin, np.int64(300), rd)
    np.testing.assert_array_equal(out[2, 300 % W], O.bf16(O.fake_quant_fp8(row, 32))[0])
    assert np.count_nonzero(out) == np.count_nonzero(out[2, 300 % W]) + np.count_nonzero(out[0, 5])


def test_window_kv_history_brute_force():
    """Attention._window_kv (dsv41/model.py:1057-1298): feeding a sequence chunk by chunk, every returned history
    equals the last min(start, W-1) rows produced before the chunk (a plain list of all rows, no ring arithmetic),
    and the ring holds exactly the last W rows at their slots."""
    r = np.random.default_rng(5)
    W, D, rd = 16, 64, 16
    cos, sin = O.rope_tables(rd, 512, 0, 10000.0, 1.0, 32, 1)
    w = O.bf16(r.random(D).astype(np.float32) + 0.5)
    ring = np.zeros((W, D), np.float32)
    produced = []
    start = 0
    for s in [5, 1, 9, 16, 3, 40, 1, 17, 2]:
        x = O.bf16(r.standard_normal((s, D)).astype(np.float32))
        out, ring = O.window_kv(x, w, cos, sin, start, ring, rd, 1e-6)
        hist = min(start, W - 1)
        want_hist = np.stack(produced[start - hist:start]) if hist else np.zeros((0, D), np.float32)
        np.testing.assert_array_equal(out[:hist], want_hist)
        produced.extend(out[hist:])
        start += s
        for p in range(max(0, start - W), start):
            np.testing.assert_array_equal(ring[p % W], produced[p])
    # the chunk rows themselves are the kv_write composition (rmsnorm -> rope -> fq8) at their positions
    x = O.bf16(r.standard_normal((3, D)).astype(np.float32))
    out, _ = O.window_kv(x, w, cos, sin, 100, np.zeros((W, D), np.float32), rd, 1e-6)
    cache = O.kv_write(x, w, cos, sin, [100, 101, 102], [0, 0, 0], np.zeros((1, W, D), np.float32), rd, 1e-6)
    np.testing.assert_array_equal(out[W - 1:], cache[0, [100 % W, 101 % W, 102 % W]])


def test_select_candidate_blocks_properties():
    """select_candidate_blocks (dsv41/model.py:256-265): the block of the last valid position is always kept; exactly
    min(topk_blocks, blocks with a finite maximum) blocks are kept; every kept block's maximum is >= every dropped
    finite block's maximum (strictly > with ties broken to the lower block); the mask is a union of whole blocks."""
    r = np.random.default_rng(21)
    T, bs, kb = 203, 8, 5
    sc = r.standard_normal((6, T)).astype(np.float32)
    sc[2] = np.round(sc[2])  # ties between block maxima
    cls = [203, 150, 77, 8, 1, 0]
    m = O.select_candidate_blocks(sc, cls, kb, bs)
    nb = -(-T // bs)
    for i, c in enumerate(cls):
        blocks = [m[i, b * bs:(b + 1) * bs] for b in range(nb)]
        assert all(x.all() or not x.any() for x in blocks)
        kept = [b for b in range(nb) if blocks[b].any()]
        bmax = [sc[i, b * bs:min((b + 1) * bs, c)].max() if b * bs < c else -np.inf for b in range(nb)]
        finite = [b for b in range(nb) if bmax[b] > -np.inf]
        assert len(kept) == min(kb, len(finite))
        if c > 0:
            assert (c - 1) // bs in kept
        others = [b for b in kept if b != (c - 1) // bs]
        dropped = [b for b in finite if b not in kept]
        for a in others:
            for d in dropped:
                assert bmax[a] > bmax[d] or (bmax[a] == bmax[d] and a < d)
    assert not m[5].any()  # no valid position: nothing kept (the forced block does not exist)


@pytest.mark.parametrize("start", [0, 3, 1025])
def test_indexer_candidates_chunk_invariant(start):
    """dsv41/test_long_prefill.py:66-96 with candidates: for the plain, source and consumer modes, query chunks of 32
    give exactly the selections (and source masks) of a single chunk."""
    r = np.random.default_rng(22)
    n, H, D, ratio, topk = 137, 2, 8, 2, 16
    T = (start + n) // ratio
    q = r.standard_normal((1, n, H, D)).astype(np.float32)
    w = r.standard_normal((1, n, H)).astype(np.float32)
    keys = r.standard_normal((1, T, D)).astype(np.float32)
    cand = r.random((1, n, T)) > 0.3
    for mode in ("plain", "source", "consumer"):
        kw = {"candidate_source": (4, 8)} if mode == "source" else ({"candidates": cand} if mode == "consumer" else {})
        full = O.indexer_prefill(q, w, keys, start, ratio, topk, 128, query_chunk=10000, **kw)
        part = O.indexer_prefill(q, w, keys, start, ratio, topk, 128, query_chunk=32, **kw)
        if mode == "source":
            np.testing.assert_array_equal(full[0], part[0])
            np.testing.assert_array_equal(full[1], part[1])
        else:
            np.testing.assert_array_equal(full, part)
    # consumer: fewer finite candidates than topk -> the non-candidates (score -inf) fill in, lowest index first
    sparse = np.zeros((1, n, T), bool)
    sparse[:, :, ::9] = True
    sel = O.indexer_prefill(q, w, keys, start, ratio, topk, 0, candidates=sparse)
    i = n - 1
    c = (start + i + 1) // ratio
    finite = [t for t in range(0, c, 9)]
    row = sel[0, i][sel[0, i] >= 0]
    assert set(finite[:topk]) <= set(row.tolist()) or len(finite) > topk
    if len(finite) < topk:
        fill = [t for t in range(c) if t % 9 != 0][:topk - len(finite)]
        assert sorted(row.tolist()) == sorted(finite + fill)


@pytest.mark.parametrize("ratio", [2, 4])
def test_compress_pool_chunk_invariant(ratio):
    """Compressor.__call__ / DecodeRuntime.compressor2 (dsv41/model.py:593-660, dsv41/decode.py:243-265): a sequence
    fed as a mix of prefill chunks and single decode rows yields, for every group that closes, the latent of the
    one-call start_pos 0 pooling of the whole sequence; decode rows that do not close a group say should=False."""
    r = np.random.default_rng(31)
    D, R, n = 64, 8, 57
    kv = r.standard_normal((n, D)).astype(np.float32)
    sc = (2 * r.standard_normal((n, D))).astype(np.float32)
    w = O.bf16(r.random(D).astype(np.float32) + 0.5)
    ring0 = (np.zeros((R, D), np.float32), np.full((R, D), -np.inf, np.float32))
    full, _, _ = O.compress_pool(kv, sc, 0, ratio, *ring0, w, 1e-6)
    assert full.shape == (n // ratio, D)
    got = {}
    rk, rs = ring0
    start = 0
    for s in [3, 1, 1, 6, 1, 13, 1, 2, 20, 1, 1, 1, 1, 5]:
        s = min(s, n - start)
        if s == 1 and start > 0:
            lat, should, rk3, rs3 = O.compress_pool_decode(kv[start:start + 1], sc[start:start + 1], [start], [0], ratio,
                                                           rk[None], rs[None], w, 1e-6)
            rk, rs = rk3[0], rs3[0]
            assert should[0] == ((start + 1) % ratio == 0)
            if should[0]:
                got[start // ratio] = lat[0]
        else:
            lat, rk, rs = O.compress_pool(kv[start:start + s], sc[start:start + s], start, ratio, rk, rs, w, 1e-6)
            first = start // ratio
            for g in range(0 if lat is None else lat.shape[0]):
                got[first + g] = lat[g]
        start += s
    assert start == n and sorted(got) == list(range(n // ratio))
    for g in range(n // ratio):
        np.testing.assert_array_equal(got[g], full[g])


def test_compress_pool_closed_forms():
    """Equal gate scores pool to the group mean; a dominant gate score (+80 over the rest) selects its member; the
    pooling equals the torch.softmax composition of dsv41/model.py:624."""
    import torch
    r = np.random.default_rng(32)
    D, ratio = 32, 4
    kv = r.standard_normal((12, D)).astype(np.float32)
    w = np.ones(D, np.float32)
    ring = (np.zeros((8, D), np.float32), np.full((8, D), -np.inf, np.float32))
    eq, _, _ = O.compress_pool(kv, np.full((12, D), 0.3, np.float32), 0, ratio, *ring, w, 1e-6)
    mean = kv.reshape(3, ratio, D).mean(axis=1)
    np.testing.assert_array_equal(eq, O.bf16(O.rmsnorm(O.bf16(mean), w, 1e-6)))
    sc = np.zeros((12, D), np.float32)
    sc[2::ratio] = 80.0
    dom, _, _ = O.compress_pool(kv, sc, 0, ratio, *ring, w, 1e-6)
    np.testing.assert_array_equal(dom, O.bf16(O.rmsnorm(O.bf16(kv[2::ratio]), w, 1e-6)))
    sc = r.standard_normal((12, D)).astype(np.float32)
    t = (torch.from_numpy(kv).view(3, ratio, D) * torch.from_numpy(sc).view(3, ratio, D).softmax(dim=1)).sum(dim=1)
    np.testing.assert_allclose(O._pool(kv.reshape(3, ratio, D), sc.reshape(3, ratio, D)), t.numpy(), rtol=1e-6,
                               atol=1e-6)


def test_e4m3_decode_all_codes():
    """e4m3 decode of all 256 bit patterns == torch.float8_e4m3fn -> float32 (NaN codes included)."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(O.e4m3_decode(codes), want)


def test_fp8_gemm_oracle():
    """fp8_gemm (dsv41/cukern.py:164-200) == torch matmul of the dequantised weight (exact products, float64);
    PERM_K is the byte order of dsv41/w8.py:23 (permute -> unpermute round trip); the block-diagonal form == the dense
    product with the off-group blocks zeroed."""
    import torch
    r = np.random.default_rng(41)
    N, K, M = 96, 256, 3
    codes = r.integers(0, 256, (N, K)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    s8 = r.integers(118, 136, (N // 32, K // 32)).astype(np.uint8)
    perm = codes.reshape(N, K // 16, 16)[:, :, O.PERM_K].reshape(N, K)
    assert O.PERM_K == [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15]
    W = torch.from_numpy(codes).view(torch.float8_e4m3fn).double() * torch.from_numpy(
        np.repeat(np.repeat(np.ldexp(1.0, s8.astype(np.int64) - 127), 32, 0), 32, 1))
    np.testing.assert_array_equal(O.fp8_dequant(perm, s8), W.float().numpy())
    x = O.bf16(r.standard_normal((M, K)).astype(np.float32))
    want = (torch.from_numpy(x).double() @ W.T).float().numpy()
    np.testing.assert_array_equal(O.fp8_gemm(x, perm, s8), want)
    # block-diagonal: 3 groups of 32 columns, x rows b * 3 + g
    xb = O.bf16(r.standard_normal((2 * 3, K)).astype(np.float32))
    got = O.fp8_gemm(xb, perm, s8, group_cols=32)
    for b in range(2):
        for g in range(3):
            Wz = W.clone()
            Wz[:g * 32] = 0
            Wz[(g + 1) * 32:] = 0
            dense = (torch.from_numpy(xb[b * 3 + g]).double() @ Wz.T).float().numpy()
            np.testing.assert_array_equal(got[b, g * 32:(g + 1) * 32], dense[g * 32:(g + 1) * 32])


def test_attention_layer_chunk_invariance():
    """AttentionLayer (Attention.__call__ up to the o-projection, dsv41/model.py:1350-1573): a sequence fed as one
    prefill chunk or as a fresh chunk plus continuations (partial compression groups, chunks shorter and longer than
    the window) gives the same outputs, caches and compressed selections (dsv41/test_long_prefill.py:66-96), and a
    following decode step agrees; the window and compressed rows of the selection are causal."""
    from _layer_weights import layer_weights
    rng = np.random.default_rng(90)
    dim, q_rank, H, D, rd, W, ratio, HI, topk = 128, 64, 4, 64, 16, 16, 4, 4, 8
    wts = layer_weights(rng, dim, q_rank, H, D, HI)
    cos, sin = O.rope_tables(rd, 256, 0, 10000.0, 1.0, 32, 1)
    kw = dict(n_heads=H, head_dim=D, rope_head_dim=rd, window=W, ratio=ratio, index_n_heads=HI, index_topk_k=topk,
              cos=cos, sin=sin, slots=1, cap=40)
    x = O.bf16(rng.standard_normal((1, 61, dim)).astype(np.float32))
    full = O.AttentionLayer(wts, **kw)
    o_full = full.attend(x[:, :60], 0)
    part = O.AttentionLayer(wts, **kw)
    outs = []
    for a, b in ((0, 21), (21, 38), (38, 60)):
        outs.append(part.attend(x[:, a:b], a))
    np.testing.assert_allclose(np.concatenate(outs, 1), o_full, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(part.ring, full.ring)
    np.testing.assert_array_equal(part.ckv, full.ckv)
    np.testing.assert_array_equal(part.index_k, full.index_k)
    assert np.abs(full.ckv[0, :15]).sum() > 0 and np.abs(full.ckv[0, 15:]).sum() == 0  # 60 // 4 rows written
    np.testing.assert_allclose(part.attend(x[:, 60:61], 60), full.attend(x[:, 60:61], 60), rtol=1e-5, atol=1e-6)
    idx = full.last_idx  # decode step: W window rows then top-k compressed rows + offset, all causal
    assert idx.shape == (1, W + topk)
    c = idx[0, W:] - W
    assert np.all((c >= 0) & (c < 61 // ratio)) and np.all(np.diff(c) > 0)


def test_torch_cpu_restatement_against_oracle():
    """The torch-CPU restatement in the reference's precision (bf16 matmuls, fp32 head sum; the CPU baseline bench.py
    times) against the numpy oracle: decode and prefill scores within 1e-2 relative, the selections agreeing on
    >= 99 % of entries (bf16 per-head rounding moves only near-threshold entries), attention within the bf16 bars."""
    from oracle import dsv41_torch_cpu as TC
    r = np.random.default_rng(40)
    n, H, D, k = 3000, 64, 128, 256
    keys = O.bf16(O.fake_quant_fp4(r.standard_normal((2, n, D)).astype(np.float32) * 0.1, 32))
    q = O.bf16(O.fake_quant_fp4(r.standard_normal((2, 1, H, D)).astype(np.float32), 32))
    w = O.bf16(r.standard_normal((2, 1, H)).astype(np.float32) * 0.05)
    cl = np.array([3000, 1700])
    tb = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)  # noqa: E731
    sc = TC.decode_scores(tb(q), tb(keys), tb(w), torch.from_numpy(cl)).numpy()
    ref = O.index_score(q, keys, w[:, 0], [0, 1], cl)
    for b in range(2):
        c = cl[b]
        assert np.abs(sc[b, :c] - ref[b, :c]).max() / np.abs(ref[b, :c]).max() <= 1e-2
        assert np.all(np.isneginf(sc[b, c:]))
    got = TC.decode_index_topk(tb(q), tb(keys), tb(w), torch.from_numpy(cl), k).numpy()[:, 0]
    np.testing.assert_array_equal(got, O.topk_indices(sc, k, cl))  # exact given the same scores
    want = O.topk_indices(ref, k, cl)
    assert np.mean([len(set(got[b]) & set(want[b])) / k for b in range(2)]) >= 0.99
    # prefill: rows of a chunk after 4000 tokens, ratio 4 -> causal lengths 1000 + (i + 1) // 4
    S, start, ratio = 96, 4000, 4
    T = (start + S) // ratio
    pk = O.bf16(O.fake_quant_fp4(r.standard_normal((1, T, D)).astype(np.float32) * 0.1, 32))
    pq = O.bf16(O.fake_quant_fp4(r.standard_normal((1, S, H, D)).astype(np.float32), 32))
    pw = O.bf16(r.standard_normal((1, S, H)).astype(np.float32) * 0.05)
    rows = [0, 5, 63, 64, 95]
    got = TC.prefill_index_topk(tb(pq), tb(pw), tb(pk), start, ratio, 512, 7, rows=rows).numpy()[0]
    for j, i in enumerate(rows):
        c = (start + i + 1) // ratio
        ref = O.index_score(pq[:, i:i + 1], pk, pw[:, i], [0], [c])
        want = set(O.topk_indices(ref, 512, [c])[0].tolist())
        assert len(set((got[j] - 7).tolist()) & want) / 512 >= 0.99
    # attention: kernels.sparse_attn math against the oracle's prefill rounding
    kv = O.bf16(r.standard_normal((1, 700, 576)).astype(np.float32) * 0.1)
    qa = O.bf16(r.standard_normal((1, 3, 64, 576)).astype(np.float32) * 0.1)
    ia = r.integers(-1, 700, (1, 3, 300)).astype(np.int32)
    sink = r.standard_normal(64).astype(np.float32)
    o = TC.sparse_attn(tb(qa), tb(kv), torch.from_numpy(sink), torch.from_numpy(ia), 576 ** -0.5, dv=512)
    want = O.sparse_attn(qa, kv, sink, ia, 576 ** -0.5, dv=512)
    err = np.abs(o.float().numpy() - want)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
