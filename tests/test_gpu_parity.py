"""GPU parity: every HIP entry point against the CPU oracle on the same seeded inputs.

Bars: top-k index sets bit-exact given identical scores; indexer scores within 1e-2
relative; attention output max |err| <= 2e-2 and mean |err| <= 2e-3; quantised cache rows bit-exact except for
rare one-step fp8/fp4 flips caused by the last-ulp difference of the fp32 rmsnorm reduction order."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ATT_MAX, ATT_MEAN = 2e-2, 2e-3


def bf(x):
    return torch.from_numpy(np.ascontiguousarray(O.bf16(x))).to(torch.bfloat16).to(DEV)


def f32(x):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float32))).to(DEV)


def i64(x):
    return torch.tensor(np.asarray(x, np.int64), device=DEV)


def host(t):
    return t.float().cpu().numpy()


def attn_close(got, want, tag=""):
    err = np.abs(got - want)
    print(f"[{tag}] max {err.max():.3e} mean {err.mean():.3e}", flush=True)
    assert err.max() <= ATT_MAX, (tag, err.max())
    assert err.mean() <= ATT_MEAN, (tag, err.mean())


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------------------------------------ numerics
@pytest.mark.parametrize("D,group,mode", [(512, 32, 0), (5120, 32, 0), (128, 32, 1), (512, 16, 2), (576, 16, 2),
                                          (576, 32, 1)])
def test_fake_quant(D, group, mode):
    import dsv41_amd
    x = O.bf16(rng(1).standard_normal((37, D)).astype(np.float32) * 4)
    y = host(dsv41_amd.fake_quant(bf(x), group, mode))
    if mode == 0:
        want = O.fake_quant_fp8(x, group)
    else:
        want = O.fake_quant_fp4(x, group, scale_e4m3=(mode == 2))
    np.testing.assert_array_equal(y, O.bf16(want))


def test_rmsnorm_and_rope():
    import dsv41_amd
    r = rng(2)
    x = O.bf16(r.standard_normal((3, 7, 512)).astype(np.float32) * 4)
    w = O.bf16(r.standard_normal(512).astype(np.float32))
    y = host(dsv41_amd.rmsnorm(bf(x), bf(w), 1e-6))
    want = O.bf16(O.rmsnorm(x, w, 1e-6))
    np.testing.assert_allclose(y, want, rtol=8e-3, atol=1e-6)
    xw = O.bf16(r.standard_normal((3, 5120)).astype(np.float32) * 4)  # a hidden-state row (past 1024 elements)
    ww = O.bf16(r.standard_normal(5120).astype(np.float32))
    np.testing.assert_allclose(host(dsv41_amd.rmsnorm(bf(xw), bf(ww), 1e-6)), O.bf16(O.rmsnorm(xw, ww, 1e-6)),
                               rtol=8e-3, atol=1e-6)
    cos, sin = O.rope_tables(64, 4096, 65536, 160000.0, 16.0, 32, 1)
    cs, sn = f32(cos), f32(sin)
    q = O.bf16(r.standard_normal((1, 3, 64, 512)).astype(np.float32))
    t = bf(q)
    dsv41_amd.rope_(t, 64, cs, sn, 100)
    want = np.stack([O.rope(q[0, i], cos, sin, np.int64(100 + i), 64) for i in range(3)])[None]
    np.testing.assert_allclose(host(t), want, atol=1e-2, rtol=8e-3)
    dsv41_amd.rope_(t, 64, cs, sn, 100, inverse=True)
    np.testing.assert_allclose(host(t), q, atol=3e-2)
    k = O.bf16(r.standard_normal((2, 1, 512)).astype(np.float32))
    t = bf(k)
    dsv41_amd.rope_dev_(t, 64, cs, sn, i64([7, 300]), add=-3)
    want = np.stack([O.rope(k[0], cos, sin, np.int64(4), 64), O.rope(k[1], cos, sin, np.int64(297), 64)])
    np.testing.assert_allclose(host(t), want, atol=1e-2, rtol=8e-3)


def _fp8_close(got, want, tag):
    """Quantised rows: identical except for rare one-step flips."""
    diff = got != want
    frac = diff.mean()
    print(f"[{tag}] mismatching elements {diff.sum()} ({frac:.2e})", flush=True)
    assert frac <= 2e-3, tag
    if diff.any():
        rel = np.abs(got[diff] - want[diff]) / np.maximum(np.abs(want[diff]), 1e-30)
        assert rel.max() <= 0.34, (tag, rel.max())


@pytest.mark.parametrize("D", [512, 576])
def test_kv_write(D):
    import dsv41_amd
    r = rng(3)
    W, rd = 128, 64
    cos, sin = O.rope_tables(rd, 4096, 0, 10000.0, 1.0, 32, 1)
    x = O.bf16(r.standard_normal((4, D)).astype(np.float32) * 2)
    w = O.bf16(r.random(D).astype(np.float32) + 0.5)
    cache = np.zeros((5, W, D), np.float32)
    pos, seq = [300, 0, 129, 4000], [4, 0, 2, 1]
    want = O.kv_write(x, w, cos, sin, pos, seq, cache, rd, 1e-6)
    ct = bf(cache)
    dsv41_amd.kv_write(bf(x), bf(w), f32(cos), f32(sin), i64(pos), ct, rd, 1e-6, i64(seq))
    _fp8_close(host(ct), want, f"kv_write D={D}")


def test_window_kv_chunks():
    """Attention._window_kv (dsv41/model.py:1057-1298) over a sequence fed in chunks (fresh chunk longer than W,
    continuations shorter and longer than W, single rows): [history | chunk] rows, window indices and the ring after
    the commit, for two batch rows, against the oracle."""
    import dsv41_amd  # noqa: F401
    from dsv41_amd import cache as C
    r = rng(14)
    W, D, rd, b = 128, 576, 64, 2
    cos, sin = O.rope_tables(rd, 8192, 0, 10000.0, 1.0, 32, 1)
    w = O.bf16(r.random(D).astype(np.float32) + 0.5)
    ring_t = bf(np.zeros((b, W, D), np.float32))
    ring = [np.zeros((W, D), np.float32) for _ in range(b)]
    start = 0
    for s in [200, 60, 1, 300, 5, 128, 1]:
        x = O.bf16(r.standard_normal((b, s, D)).astype(np.float32) * 2)
        print(f"[window_kv] start {start} chunk {s}", flush=True)
        out, idx = C.window_kv(bf(x), bf(w), 1e-6, f32(cos), f32(sin), rd, ring_t, start)
        for bi in range(b):
            want, ring[bi] = O.window_kv(x[bi], w, cos, sin, start, ring[bi], rd, 1e-6)
            if s == 1 and start > 0:  # decode shape: the ring itself and its slot indices
                np.testing.assert_array_equal(host(idx[bi]), O.window_idx(W, 1, start))
            else:
                hist, want_idx = (0, O.window_idx(W, s, 0)) if start == 0 else O.prefill_window_idx(W, s, start)
                assert out.shape[1] == hist + s
                _fp8_close(host(out[bi]), want, f"window_kv rows b{bi} start {start}")
                np.testing.assert_array_equal(host(idx[bi]), want_idx)
            _fp8_close(host(ring_t[bi]), ring[bi], f"window_kv ring b{bi} start {start}")
        start += s


def test_compressed_and_index_key_appends():
    import dsv41_amd
    from dsv41_amd import cache as C
    r = rng(4)
    rd, ratio = 64, 4
    cos, sin = O.rope_tables(rd, 8192, 0, 10000.0, 1.0, 32, 1)
    # decode compressed append: rope at pos + 1 - ratio, fq4(16, e4m3) -> cache[seq, row]
    lat = O.bf16(r.standard_normal((3, 1, 576)).astype(np.float32))
    pos, seq, row = [7, 403, 4095], [1, 0, 2], [1, 100, -1]
    cache = np.zeros((3, 1030, 576), np.float32)
    ct = bf(cache)
    C.append_compressed_decode(ct, bf(lat), i64(pos), i64(seq), i64(row), ratio, f32(cos), f32(sin), rd)
    want = cache.copy()
    for i in range(3):
        if row[i] >= 0:
            want[seq[i], row[i]] = O.compress_row(lat[i, 0], cos, sin, np.int64(pos[i] + 1 - ratio), rd)
    _fp8_close(host(ct), want, "compressed append")
    # prefill index-key append with the e4m3 sidecar
    kraw = O.bf16(r.standard_normal((2, 9, 128)).astype(np.float32) * 3)
    nw = O.bf16(r.random(128).astype(np.float32) + 0.5)
    kc = bf(np.zeros((2, 64, 128), np.float32))
    k8 = torch.zeros(2, 64, 128, dtype=torch.uint8, device=DEV)
    ks = torch.zeros(2, 64, dtype=torch.float32, device=DEV)
    start = 10
    C.write_index_k(kc, bf(kraw), bf(nw), 1e-6, start, ratio, f32(cos), f32(sin), rd, k8=k8, k_scale=ks)
    first = start - start % ratio
    want = np.zeros((2, 64, 128), np.float32)
    for b in range(2):
        for i in range(9):
            want[b, start // ratio + i] = O.index_key_row(kraw[b, i], nw, cos, sin, np.int64(first + i * ratio), rd, 1e-6)
    got = host(kc)
    _fp8_close(got, want, "index-key append")
    dec = k8.view(torch.float8_e4m3fn).float().cpu().numpy() * ks.cpu().numpy()[..., None]
    np.testing.assert_array_equal(dec, got)  # the e4m3 copy is exact for FP4-grid rows
    # prefill compressed append (start_pos > 0: first group start)
    lat2 = O.bf16(r.standard_normal((1, 5, 512)).astype(np.float32))
    c2 = bf(np.zeros((1, 40, 512), np.float32))
    C.write_compress_kv(c2, bf(lat2), 17, ratio, f32(cos), f32(sin), rd)
    want2 = np.zeros((1, 40, 512), np.float32)
    for i in range(5):
        want2[0, 17 // ratio + i] = O.compress_row(lat2[0, i], cos, sin, np.int64(16 + i * ratio), rd)
    _fp8_close(host(c2), want2, "prefill compressed append")


# ------------------------------------------------------------------------------------------------ attention
def test_sparse_attn_reference_unit_shape():
    """dsv41/test_kernels.py:33-49 shape: b=1, s=5, h=4, d=64, n=40, t=8 with three -1 slots."""
    import dsv41_amd
    r = rng(5)
    b, s, h, d, n = 1, 5, 4, 64, 40
    q = O.bf16(r.standard_normal((b, s, h, d)).astype(np.float32))
    kv = O.bf16(r.standard_normal((b, n, d)).astype(np.float32))
    sink = r.standard_normal(h).astype(np.float32)
    idx = r.integers(0, n, (b, s, 8)).astype(np.int32)
    idx[0, 0, :3] = -1
    idx[0, 1, 0] = n + 5  # out of range = invalid (dsv41/kernels.py:204-207)
    o = host(dsv41_amd.sparse_attn(bf(q), bf(kv), f32(sink), torch.from_numpy(idx).to(DEV), d ** -0.5))
    attn_close(o, O.sparse_attn(q, kv, sink, idx, d ** -0.5), "sparse_attn unit")


@pytest.mark.parametrize("dqk,dv,s,t", [(512, 512, 3, 640), (576, 512, 2, 2176), (576, 512, 1, 100)])
def test_sparse_attn_latent(dqk, dv, s, t):
    import dsv41_amd
    r = rng(6)
    b, h, n = 2, 64, 3000
    q = O.bf16(r.standard_normal((b, s, h, dqk)).astype(np.float32))
    kv = O.bf16(r.standard_normal((b, n, dqk)).astype(np.float32) * 0.1)
    sink = r.standard_normal(h).astype(np.float32)
    idx = r.integers(0, n, (b, s, t)).astype(np.int32)
    idx[..., 5:40] = -1
    scale = dqk ** -0.5
    o = host(dsv41_amd.sparse_attn(bf(q), bf(kv), f32(sink), torch.from_numpy(idx).to(DEV), scale, d_v=dv))
    attn_close(o, O.sparse_attn(q, kv, sink, idx, scale, dv=dv), f"sparse_attn {dqk}/{dv} s={s} t={t}")


def test_sparse_attn_decode_and_split():
    """dsv41/test_fused.py:64-70 (700 rows, 640 idx, 35 x -1) and :90-94 (ring 128 + compressed 2049)."""
    import dsv41_amd
    r = rng(7)
    q = O.bf16(r.standard_normal((1, 1, 64, 512)).astype(np.float32))
    kv = O.bf16(r.standard_normal((1, 700, 512)).astype(np.float32))
    sink = r.standard_normal(64).astype(np.float32)
    idx = r.integers(0, 700, (1, 1, 640)).astype(np.int32)
    idx[0, 0, 5:40] = -1
    o = host(dsv41_amd.sparse_attn_decode(bf(q), bf(kv), f32(sink), torch.from_numpy(idx).to(DEV), 512 ** -0.5))
    attn_close(o, O.sparse_attn(q, kv, sink, idx, 512 ** -0.5, prefill_rounding=False), "sparse_attn_decode")
    kv1 = O.bf16(r.standard_normal((1, 128, 512)).astype(np.float32))
    kv2 = O.bf16(r.standard_normal((1, 2049, 512)).astype(np.float32))
    idx2 = np.concatenate([r.integers(0, 128, (1, 1, 128)), 128 + r.integers(0, 2049, (1, 1, 512))], -1).astype(np.int32)
    idx2[0, 0, 3:20] = -1
    want = O.sparse_attn_decode2(q, kv1, kv2, sink, idx2, 512 ** -0.5)
    for fn in (dsv41_amd.sparse_attn_decode2, dsv41_amd.sparse_attn_decode_split):
        o = host(fn(bf(q), bf(kv1), bf(kv2), f32(sink), torch.from_numpy(idx2).to(DEV), 512 ** -0.5))
        attn_close(o, want, fn.__name__)


@pytest.mark.parametrize("p", [50, 300])
def test_sattn2_reference_geometry(p):
    """dsv41/test_fused2_units.py:50-68: window only, and window + 512 compressed idx (112 x -1) over 4097 rows."""
    import dsv41_amd
    r = rng(8 + p)
    H, hd, win, rd = 64, 512, 128, 64
    cos, sin = O.rope_tables(rd, 4096, 0, 10000.0, 1.0, 32, 1)
    q = O.bf16(r.standard_normal((1, 1, H, hd)).astype(np.float32))
    sink = r.standard_normal(H).astype(np.float32)
    ring = O.bf16(r.standard_normal((1, win, hd)).astype(np.float32))
    ckv = O.bf16(r.standard_normal((1, 4097, hd)).astype(np.float32))
    idx = r.integers(0, 150, (1, 1, 512)).astype(np.int32)
    idx[..., 400:] = -1
    for with_c in (False, True):
        o = dsv41_amd.sattn2(bf(q), bf(ring), bf(ckv) if with_c else None,
                             torch.from_numpy(idx).to(DEV) if with_c else None, i64([p]), f32(sink), f32(cos),
                             f32(sin), rd, hd ** -0.5, i64([0]), i64([p]))
        want = O.sattn2(q, ring, ckv if with_c else None, idx if with_c else None, [p], [0], [p], None, sink, cos, sin,
                        rd, hd ** -0.5)
        attn_close(host(o), want, f"sattn2 ref pos={p} c={with_c}")


@pytest.mark.parametrize("H", [64, 40])
def test_sattn2_absorbed_mla_ragged_with_drafts(H):
    """576/512 absorbed MLA, k = 2048, 4 slots at ragged positions, plus 6 draft rows of one sequence with plim
    causal masking (the MTP verify shape, dsv41/fused2.py:351-360), at 64 and 40 heads.  Calls with different split
    counts share one workspace (its split counters must be left ready whatever the previous call's split count)."""
    import dsv41_amd
    from dsv41_amd._lib import lib
    r = rng(9)
    dqk, dv, win, k = 576, 512, 128, 2048
    S, n_c = 4, 4096
    q = O.bf16(r.standard_normal((10, 1, H, dqk)).astype(np.float32))
    sink = r.standard_normal(H).astype(np.float32)
    ring = O.bf16(r.standard_normal((S, win, dqk)).astype(np.float32) * 0.1)
    ckv = O.bf16(r.standard_normal((S, n_c, dqk)).astype(np.float32) * 0.1)
    pos = [16383, 100, 5000, 7, 900, 901, 902, 903, 904, 905]
    seq = [0, 1, 2, 3, 1, 1, 1, 1, 1, 1]
    pmax = [16383, 100, 5000, 7, 905, 905, 905, 905, 905, 905]
    idx = np.full((10, 1, k), -1, np.int32)
    for b in range(10):
        cl = (pos[b] + 1) // 4
        nv = min(k, cl)
        idx[b, 0, :nv] = np.sort(r.choice(cl, nv, replace=False))
    cos = np.zeros((1, 1), np.float32)
    want = O.sattn2(q, ring, ckv, idx, pos, seq, pmax, pos, sink, cos, cos, 0, dqk ** -0.5, dv=dv)
    splits = [0, 0, 3, 5, 2, 0]
    nbytes = max(lib().dsv41_attn_workspace_bytes(10, H, win + k, dv, n) for n in splits)
    ws = torch.zeros(max(nbytes, 4) // 4, dtype=torch.float32, device=DEV)
    for call_no, ns in enumerate(splits):
        o = dsv41_amd.sattn2(bf(q), bf(ring), bf(ckv), torch.from_numpy(idx).to(DEV), i64(pos), f32(sink), f32(cos),
                             f32(cos), 0, dqk ** -0.5, i64(seq), i64(pmax), plim=i64(pos), d_v=dv, nsplit=ns, ws=ws)
        attn_close(host(o), want, f"sattn2 mla ragged+drafts H={H} call {call_no} nsplit {ns}")


@pytest.mark.parametrize("H", [64, 40])
@pytest.mark.parametrize("rows", [4, 1])
def test_sattn2_decode_kernels_32_and_16_heads(rows, H, monkeypatch):
    """The decode attention's two kernels (32-head workgroups with one gather round trip per split of <= 128 keys,
    and 16-head workgroups over 64-key tiles; DSV41_ATTN_DEC32 selects) at the C2 / C4 shapes: 576/512 absorbed MLA,
    ring 128 + k 2048, slots at ragged positions (short contexts leave whole splits without a valid key), against
    the oracle; calls alternating between the kernels share one workspace (its counters stay ready for either)."""
    import dsv41_amd
    from dsv41_amd._lib import lib
    r = rng(19 + rows)
    dqk, dv, win, k = 576, 512, 128, 2048
    S, n_c = 4, 4096
    q = O.bf16(r.standard_normal((rows, 1, H, dqk)).astype(np.float32))
    sink = r.standard_normal(H).astype(np.float32)
    ring = O.bf16(r.standard_normal((S, win, dqk)).astype(np.float32) * 0.1)
    ckv = O.bf16(r.standard_normal((S, n_c, dqk)).astype(np.float32) * 0.1)
    pos = [16383, 100, 5000, 7][:rows]
    seq = [0, 1, 2, 3][:rows]
    idx = np.full((rows, 1, k), -1, np.int32)
    for b in range(rows):
        cl = (pos[b] + 1) // 4
        nv = min(k, cl)
        idx[b, 0, :nv] = np.sort(r.choice(cl, nv, replace=False))
    cos = np.zeros((1, 1), np.float32)
    want = O.sattn2(q, ring, ckv, idx, pos, seq, pos, pos, sink, cos, cos, 0, dqk ** -0.5, dv=dv)
    nbytes = 0
    for flag in ("1", "0"):
        monkeypatch.setenv("DSV41_ATTN_DEC32", flag)
        nbytes = max(nbytes, lib().dsv41_attn_workspace_bytes(rows, H, win + k, dv, 0))
    ws = torch.zeros(max(nbytes, 4) // 4, dtype=torch.float32, device=DEV)
    for call_no, flag in enumerate(["1", "0", "1", "1", "0"]):
        monkeypatch.setenv("DSV41_ATTN_DEC32", flag)
        print(f"[sattn2 decode kernels] rows {rows} H {H} call {call_no} dec32={flag}", flush=True)
        o = dsv41_amd.sattn2(bf(q), bf(ring), bf(ckv), torch.from_numpy(idx).to(DEV), i64(pos), f32(sink), f32(cos),
                             f32(cos), 0, dqk ** -0.5, i64(seq), i64(pos), plim=i64(pos), d_v=dv, ws=ws)
        attn_close(host(o), want, f"sattn2 decode rows={rows} H={H} call {call_no} dec32={flag}")
        assert int(ws.view(torch.int32)[0].item()) == 0, "a cooperative merge stopped waiting for its unit"


# ------------------------------------------------------------------------------------------------ indexer
def _fp4_rows(r, shape, scale=0.1):
    return O.bf16(O.fake_quant_fp4(O.bf16(r.standard_normal(shape).astype(np.float32) * scale), 32))


@pytest.mark.parametrize("fmt", ["bf16", "e4m3"])
def test_index_score(fmt):
    import dsv41_amd
    r = rng(10)
    B, H, D, S, n = 3, 64, 128, 4, 5000
    q = _fp4_rows(r, (B, 1, H, D), 1.0)
    keys = _fp4_rows(r, (S, n, D))
    keys[:, :, [3, 40, 77, 120]] *= 8  # outlier channels
    keys = O.bf16(O.fake_quant_fp4(keys, 32))
    w = O.bf16(r.standard_normal((B, 1, H)).astype(np.float32) * 0.1)
    seq, cl = [2, 0, 3], [4321, 5000, 17]
    if fmt == "bf16":
        kt, ks = bf(keys), None
        want = O.index_score(q, keys, w, seq, cl)
    else:
        q8, s8 = O.key_encode_fp8(keys)
        kt = torch.from_numpy(q8).to(torch.float8_e4m3fn).to(DEV)
        ks = f32(s8[..., 0])
        want = O.index_score(q, q8, w, seq, cl, k_scale=s8[..., 0])
    got = host(dsv41_amd.index_score(bf(q), kt, bf(w), i64(seq), i64(cl), k_scale=ks))
    fin = np.isfinite(want)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    for b in range(B):
        m = fin[b]
        scale = np.abs(want[b][m]).max()
        err = np.abs(got[b][m] - want[b][m]).max() / scale
        print(f"[index_score {fmt}] row {b} rel err {err:.2e}", flush=True)
        assert err <= 1e-2


@pytest.mark.parametrize("n,k,cl", [(32768, 2048, 32768), (32768, 2048, 20000), (1000, 2048, 1000), (4097, 512, 4097),
                                    (262144, 2048, 262144), (100000, 2048, 50001), (16896, 2048, 16500)])
def test_topk_bit_exact(n, k, cl):
    import dsv41_amd
    r = rng(11)
    B = 3
    sc = r.standard_normal((B, n)).astype(np.float32)
    sc[1, ::5] = 0.25  # many exact ties
    sc[2] = np.round(sc[2] * 4) / 4  # coarse values: ties at the threshold
    sc[:, cl:] = -np.inf
    got = dsv41_amd.topk_indices(f32(sc), k, i64([cl] * B)).cpu().numpy()[:, 0]
    want = O.topk_indices(sc, k, [cl] * B)
    np.testing.assert_array_equal(got, want)


def test_topk_many_rows_ties_and_fallback():
    """The many-row top-k (512-thread workgroups, rows staged in LDS) on ragged rows built to reach each of its paths:
    no ties; ties at the threshold taken in part by several waves (coarse values); an all-equal row (the first k
    positions); ties every 5th position; every key in one 12-bit histogram bin (the candidate lists overflow: the
    range-normalised radix path); +0 / -0 mixtures (-0 equals +0); valid counts of k + 1 and of 64 m + 1; bit-exact
    against the oracle."""
    import dsv41_amd
    r = rng(13)
    R, n, k = 512, 6000, 2048
    sc = r.standard_normal((R, n)).astype(np.float32)
    cl = r.integers(k + 1, n + 1, R)
    cl[:3] = [k + 1, n, 4097]
    for b in range(R):
        kind = b % 6
        if kind == 1:
            sc[b] = np.round(sc[b] * 4) / 4
        elif kind == 2:
            sc[b] = 1.0
        elif kind == 3:
            sc[b, ::5] = 0.25
        elif kind == 4:
            sc[b] = 1.0 + r.random(n).astype(np.float32) * 0.1  # [1, 1.1): one bin of the top 12 key bits
        elif kind == 5:
            sc[b] = np.where(r.random(n) < 0.5, np.float32(0.0), np.float32(-0.0))
            sc[b, ::7] = r.random(len(sc[b, ::7])).astype(np.float32) + 0.5
        sc[b, cl[b]:] = -np.inf
    print(f"[topk many rows] R {R} n {n} k {k} cl {cl.min()}..{cl.max()}", flush=True)
    got = dsv41_amd.topk_indices(f32(sc), k, i64(cl)).cpu().numpy()[:, 0]
    want = O.topk_indices(sc, k, cl)
    bad = np.nonzero((got != want).any(1))[0]
    assert len(bad) == 0, f"rows {bad[:10].tolist()} (kinds {(bad[:10] % 6).tolist()}) differ"


def test_index_topk_prefill():
    """Indexer.__call__ chunk selection (dsv41/model.py:766-893): per-query causal compressed length."""
    import dsv41_amd
    r = rng(12)
    b, s, H, D, start, ratio, topk, offset = 1, 96, 64, 128, 1000, 4, 64, 1127
    T = (start + s) // ratio
    q = _fp4_rows(r, (b, s, H, D), 1.0)
    w = O.bf16(r.standard_normal((b, s, H)).astype(np.float32) * 0.1)
    keys = _fp4_rows(r, (b, T + 10, D))
    q8, s8 = O.key_encode_fp8(keys)
    want = O.indexer_prefill(q, w, keys, start, ratio, topk, offset)
    got, score = dsv41_amd.index_topk(bf(q), bf(w), bf(keys), start, ratio, topk, offset, return_score=True)
    got8 = dsv41_amd.index_topk(bf(q), bf(w), torch.from_numpy(q8).to(torch.float8_e4m3fn).to(DEV), start, ratio,
                                topk, offset, k_scale=f32(s8[..., 0]))
    # bit-exact index sets given identical scores: re-select from the GPU's own scores with the oracle
    sc = score.cpu().numpy()[0]
    cls = (start + np.arange(s) + 1) // ratio
    resel = O.topk_indices(sc, min(topk, T), cls)
    np.testing.assert_array_equal(got.cpu().numpy()[0], np.where(resel >= 0, resel + offset, -1))
    np.testing.assert_array_equal(got.cpu().numpy(), got8.cpu().numpy())
    # and against the oracle end to end (scores exact up to fp32 summation order -> identical sets here)
    agree = (got.cpu().numpy() == want).mean()
    print(f"[index_topk] agreement with oracle {agree:.5f}", flush=True)
    assert agree >= 0.999


def test_decode_appends_fused():
    """The one-launch decode appends == ring kv_write + compressed append + index-key append (spare row when no
    group closes)."""
    from dsv41_amd import cache as C
    r = rng(13)
    D, W, rd, ratio, S, cap = 576, 128, 64, 4, 3, 40
    cos, sin = O.rope_tables(rd, 8192, 0, 10000.0, 1.0, 32, 1)
    B = 4
    kv_raw = O.bf16(r.standard_normal((B, D)).astype(np.float32) * 2)
    kvn = O.bf16(r.random(D).astype(np.float32) + 0.5)
    lat = O.bf16(r.standard_normal((B, 1, D)).astype(np.float32))
    kraw = O.bf16(r.standard_normal((B, 128)).astype(np.float32) * 3)
    kn = O.bf16(r.random(128).astype(np.float32) + 0.5)
    pos, seq = [7, 100, 131, 11], [0, 2, 1, 1]
    ring = bf(np.zeros((S, W, D), np.float32))
    ckv = bf(np.zeros((S, cap, D), np.float32))
    kbf = bf(np.zeros((S, cap, 128), np.float32))
    k8 = torch.zeros(S, cap, 128, dtype=torch.uint8, device=DEV)
    ks = torch.zeros(S, cap, dtype=torch.float32, device=DEV)
    C.decode_appends(bf(kv_raw), bf(kvn), ring, bf(lat), ckv, bf(kraw), bf(kn), kbf, k8, ks, i64(pos), i64(seq),
                     ratio, f32(cos), f32(sin), rd, 1e-6)
    want_ring = O.kv_write(kv_raw, kvn, cos, sin, pos, seq, np.zeros((S, W, D), np.float32), rd, 1e-6)
    want_c = np.zeros((S, cap, D), np.float32)
    want_k = np.zeros((S, cap, 128), np.float32)
    for i in range(B):
        row = (pos[i] + 1) // ratio - 1 if (pos[i] + 1) % ratio == 0 else cap - 1
        p0 = np.int64(pos[i] + 1 - ratio)
        want_c[seq[i], row] = O.compress_row(lat[i, 0], cos, sin, p0, rd)
        want_k[seq[i], row] = O.index_key_row(kraw[i], kn, cos, sin, p0, rd, 1e-6)
    _fp8_close(host(ring), want_ring, "decode appends ring")
    _fp8_close(host(ckv), want_c, "decode appends compressed")
    _fp8_close(host(kbf), want_k, "decode appends index key")
    dec = k8.view(torch.float8_e4m3fn).float().cpu().numpy() * ks.cpu().numpy()[..., None]
    np.testing.assert_array_equal(dec, host(kbf))


@pytest.mark.parametrize("n,k,cls", [(32769, 2048, [32768, 32768, 20000, 1500]), (262145, 2048, [262144]),
                                     (4097, 512, [4096, 4000, 511, 0]), (32768, 2048, [32768, 32768, 20000, 1500]),
                                     (262145, 2048, [262144, 200000]),
                                     (200000, 2048, [200000, 150000]), (131072, 1024, [131072, 100000] * 5),
                                     (65536, 2048, [65536] * 9 + [40000, 3000, 2049]), (32768, 512, [32768, 9000] * 10),
                                     (32768, 512, [32768, 30000, 513, 512, 7, 32768]), (36864, 1024, [36864, 33000])])
def test_select_topk_histogram_path(n, k, cls):
    """Decode top-k from (scores, histogram): bit-exact against the oracle's selection on the same scores,
    including heavy ties (a coarse-valued row -> the threshold bin overflows the LDS candidate stage)."""
    from dsv41_amd._lib import call, lib, ptr
    r = rng(14)
    R = len(cls)
    sc = (r.standard_normal((R, n)).astype(np.float32) * 0.5 + 3.0).astype(np.float32)
    if R > 1:
        sc[1] = np.round(sc[1] * 2) / 2  # ties everywhere
    keys = O.score_key(sc) >> 20
    hist = np.zeros((R, 4096), np.int32)
    for i, c in enumerate(cls):
        np.add.at(hist[i], keys[i, :c].astype(np.int64), 1)
    nbytes = lib().dsv41_select_workspace_bytes(R, n)
    ws = torch.zeros(nbytes // 4, dtype=torch.int32, device=DEV)
    st = f32(sc)
    cl = i64(cls)
    want = O.topk_indices(sc, k, cls)
    for call_no in range(2):  # the workspace is reused: the selection leaves it ready for the next call
        ws[:R * 4096] = torch.from_numpy(hist.reshape(-1)).to(DEV)
        out = torch.empty(R, k, dtype=torch.int32, device=DEV)
        call("dsv41_select_topk", ptr(st), n, R, n, k, ptr(cl), 0, ptr(ws), nbytes, ptr(out), k,
             torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want, err_msg=f"call {call_no}")
        assert int(ws[:R * 4096].abs().sum().item()) == 0, "histogram not cleared"
        assert int(ws[-4].item()) == 0, "row barrier wait gave up"


@pytest.mark.parametrize("cls", [[32768, 32768, 20000, 1500], [2048, 100000, 3, 65000]])
def test_decode_selector_end_to_end(cls):
    """Decode selector (one launch: scores + histogram + selection; or the score kernel then the selection) ==
    oracle top-k on the kernel's own scores (bit-exact), and the scores match the oracle within 1e-2."""
    from dsv41_amd.fused3 import DecodeSelector
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(15)
    R, H, n = len(cls), 64, max(cls) + 1
    keys = fp4_round(torch.randn(3, n, 128, generator=g, device=DEV) * 0.1)
    k8, ks = encode_e4m3_rows(keys)
    q = fp4_round(torch.randn(R, 1, H, 128, generator=g, device=DEV))
    w = (torch.randn(R, H, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    seq = i64([0, 2, 1, 2])
    sel = DecodeSelector(R, n, 2048, DEV, keep_scores=True)
    assert sel.one_launch == (n <= 65536)  # one launch (score + select) for the first case, two kernels for the other
    for rep in range(2):  # the second call checks the workspace is reusable
        idx = sel(q, k8, w, seq, i64(cls), k_scale=ks)
        torch.cuda.synchronize()
        sc = sel.score.cpu().numpy()
        np.testing.assert_array_equal(idx.cpu().numpy()[:, 0], O.topk_indices(sc, 2048, cls))
        if sel.one_launch:
            assert int(sel.fws[-4].item()) == 0, "row barrier wait gave up"
    want = O.index_score(q.float().cpu().numpy(), k8.float().cpu().numpy(), w.float().cpu().numpy(),
                         [0, 2, 1, 2], cls, k_scale=ks.cpu().numpy())
    for b, c in enumerate(cls):
        if c == 0:
            continue
        err = np.abs(sc[b, :c] - want[b, :c]).max() / np.abs(want[b, :c]).max()
        assert err <= 1e-2, (b, err)


@pytest.mark.parametrize("layout", ["drafts", "interleaved"])
def test_decode_selector_draft_rows(layout):
    """More than four decode rows through the score kernel then the selection (n_pos > 65536): a sequence's draft
    rows are consecutive rows of one slot (runs longer than 8 rows, a slot that reappears later, ragged counts down
    to a few positions), or the slots interleave row by row.  Top-k == oracle top-k of the kernel's own scores
    (bit-exact; the selection reads the kernel's histogram), scores within 1e-2 of the oracle, twice in a row
    (the histogram is left zeroed for the next call)."""
    from dsv41_amd.fused3 import DecodeSelector
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(23)
    if layout == "drafts":
        seq_l = [0] * 6 + [1] * 6 + [2] * 3 + [3] * 11 + [4] * 2 + [0] * 2
        base = {0: 70000, 1: 30000, 2: 513, 3: 66000, 4: 5}
        cls = []
        for i, s in enumerate(seq_l):
            j = sum(1 for t in seq_l[:i] if t == s)  # draft j of its sequence: one more valid position each
            cls.append(min(base[s] + j, 70000))
    else:
        seq_l = [0, 1, 2, 3] * 3
        cls = [70000, 40000, 9000, 300, 69999, 40001, 9001, 301, 69998, 40002, 9002, 302]
    R, H, n, k = len(seq_l), 64, 70001, 2048
    keys = fp4_round(torch.randn(5, n, 128, generator=g, device=DEV) * 0.1)
    keys[:, :, [5, 60]] *= 6
    k8, ks = encode_e4m3_rows(keys)
    q = fp4_round(torch.randn(R, 1, H, 128, generator=g, device=DEV))
    w = (torch.randn(R, H, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    sel = DecodeSelector(R, n, k, DEV, keep_scores=True)
    assert not sel.one_launch
    want = O.index_score(q.float().cpu().numpy(), k8.float().cpu().numpy(), w.float().cpu().numpy(), seq_l, cls,
                         k_scale=ks.cpu().numpy())
    for rep in range(2):
        print(f"[draft rows {layout}] R {R} call {rep}", flush=True)
        idx = sel(q, k8, w, i64(seq_l), i64(cls), k_scale=ks)
        torch.cuda.synchronize()
        sc = sel.score.cpu().numpy()
        np.testing.assert_array_equal(idx.cpu().numpy()[:, 0], O.topk_indices(sc, k, cls), err_msg=f"call {rep}")
        for b, c in enumerate(cls):
            err = np.abs(sc[b, :c] - want[b, :c]).max() / np.abs(want[b, :c]).max()
            assert err <= 1e-2, (b, err)


@pytest.mark.parametrize("n,cl", [(262145, 262144), (200001, 150000)])
def test_decode_selector_long_row(n, cl):
    """One long row (C4 shape: up to 512 chunks of 512 positions) through the one-launch indexer (forced: by default
    rows past 128 chunks take the multi-launch path) and the multi-launch path: selection bit-exact against the
    oracle on the kernel's own scores, the two paths identical, scores within 1e-2 of the oracle, workspace
    reusable."""
    from dsv41_amd.fused3 import DecodeSelector
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(17)
    H = 64
    keys = fp4_round(torch.randn(2, n, 128, generator=g, device=DEV) * 0.1)
    keys[:, :, [3, 40, 77, 120]] *= 8  # outlier channels
    k8, ks = encode_e4m3_rows(fp4_round(keys))
    q = fp4_round(torch.randn(1, 1, H, 128, generator=g, device=DEV))
    w = (torch.randn(1, H, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    seq = i64([1])
    sel = DecodeSelector(1, n, 2048, DEV, keep_scores=True, max_cl=n - 1, one_launch_max_chunks=512)
    assert sel.one_launch  # (the last row is the spare row)
    for rep in range(2):
        print(f"[selector long row] n {n} cl {cl} call {rep}", flush=True)
        idx = sel(q, k8, w, seq, i64([cl]), k_scale=ks)
        torch.cuda.synchronize()
        assert int(sel.fws[-4].item()) == 0, "row barrier wait gave up"
        sc = sel.score.cpu().numpy()
        np.testing.assert_array_equal(idx.cpu().numpy()[:, 0], O.topk_indices(sc, 2048, [cl]))
    multi = DecodeSelector(1, n, 2048, DEV, max_cl=n - 1)
    assert not multi.one_launch
    np.testing.assert_array_equal(multi(q, k8, w, seq, i64([cl]), k_scale=ks).cpu().numpy(), idx.cpu().numpy())
    want = O.index_score(q.float().cpu().numpy(), k8.float().cpu().numpy(), w.float().cpu().numpy(), [1], [cl],
                         k_scale=ks.cpu().numpy())
    err = np.abs(sc[0, :cl] - want[0, :cl]).max() / np.abs(want[0, :cl]).max()
    assert err <= 1e-2, err


def test_candidate_blocks_select():
    """select_candidate_blocks (dsv41/model.py:256-265) on masked scores: identical masks to the oracle (ties between
    block maxima included), per-row valid counts covering whole, partial, single and empty rows."""
    import dsv41_amd.indexer as I
    r = rng(18)
    R, T = 7, 1000
    sc = r.standard_normal((R, T)).astype(np.float32)
    sc[3] = np.round(sc[3])  # ties between blocks
    cls = [1000, 999, 513, 400, 64, 1, 0]
    for bs, kb in [(8, 16), (64, 4), (16, 1000)]:
        print(f"[candidate blocks] bs {bs} kb {kb}", flush=True)
        want = O.select_candidate_blocks(sc, cls, kb, bs)
        masked = np.where(np.arange(T)[None, :] < np.asarray(cls)[:, None], sc, -np.inf).astype(np.float32)
        got = I.select_candidate_blocks(f32(masked), i64(cls).view(R, 1), kb, bs).cpu().numpy()
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("fmt", ["bf16", "e4m3"])
def test_index_topk_candidates(fmt):
    """Indexer.__call__ with candidate blocks (dsv41/model.py:838-866): the source layer's mask equals the oracle's on
    the kernel's own scores; a consumer layer's selection equals the oracle's top-k on its own masked scores (sparse
    masks: the non-candidates fill the selection, lowest index first)."""
    import dsv41_amd
    r = rng(19)
    b, s, H, D, start, ratio, topk = 1, 80, 64, 128, 900, 4, 64
    T = (start + s) // ratio
    q = _fp4_rows(r, (b, s, H, D), 1.0)
    w = O.bf16(r.standard_normal((b, s, H)).astype(np.float32) * 0.1)
    keys = _fp4_rows(r, (b, T + 10, D))
    if fmt == "bf16":
        kt, ks = bf(keys), None
    else:
        q8, s8 = O.key_encode_fp8(keys)
        kt, ks = torch.from_numpy(q8).to(torch.float8_e4m3fn).to(DEV), f32(s8[..., 0])
    cls = (start + np.arange(s) + 1) // ratio
    idx, score, mask = dsv41_amd.index_topk(bf(q), bf(w), kt, start, ratio, topk, 0, k_scale=ks, return_score=True,
                                            candidate_source=(6, 8))
    sc = score.cpu().numpy()[0]
    sc = np.where(np.arange(T)[None, :] < cls[:, None], sc, -np.inf).astype(np.float32)
    want_mask = O.select_candidate_blocks(sc, cls, 6, 8)
    got_mask = mask.cpu().numpy()[0]
    np.testing.assert_array_equal(got_mask[:, :T], want_mask)
    # a block straddling T extends past it (the reference's repeat_interleave over the key table width); beyond: none
    straddle = (T + 7) // 8 * 8 - T
    np.testing.assert_array_equal(got_mask[:, T:T + straddle], np.repeat(got_mask[:, T - 1:T], straddle, axis=1))
    assert not got_mask[:, T + straddle:].any()
    np.testing.assert_array_equal(idx.cpu().numpy()[0], O.topk_indices(sc, min(topk, T), cls))
    for cand in [mask, torch.from_numpy(r.random((b, s, T + 10)) > 0.95).to(DEV)]:
        idx2, score2 = dsv41_amd.index_topk(bf(q), bf(w), kt, start, ratio, topk, 0, k_scale=ks, return_score=True,
                                            candidates=cand)
        sc2 = score2.cpu().numpy()[0]
        sc2 = np.where(np.arange(T)[None, :] < cls[:, None], sc2, -np.inf).astype(np.float32)
        cm = cand.cpu().numpy()[0, :, :T]
        assert np.all(np.isneginf(sc2[(~cm) & (np.arange(T)[None, :] < cls[:, None])]))
        np.testing.assert_array_equal(sc2[cm & np.isfinite(sc2)], sc[cm & np.isfinite(sc2)])
        np.testing.assert_array_equal(idx2.cpu().numpy()[0], O.topk_indices(sc2, min(topk, T), cls))


def test_decode_candidates():
    """Decode indexer with a candidate mask (dsv41/decode.py:309-315): fused3.index_score(cand=...) scores -inf
    exactly at the non-candidates; the one-launch selector and the two-kernel path select the oracle's top-k of those
    scores (non-candidates as last-resort fillers, lowest index first)."""
    from dsv41_amd.fused3 import DecodeSelector, index_score
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(20)
    R, H, n = 4, 64, 6001
    cls = [6000, 4097, 3000, 100]
    keys = fp4_round(torch.randn(3, n, 128, generator=g, device=DEV) * 0.1)
    k8, ks = encode_e4m3_rows(keys)
    q = fp4_round(torch.randn(R, 1, H, 128, generator=g, device=DEV))
    w = (torch.randn(R, H, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
    seq = i64([0, 2, 1, 2])
    cand = torch.rand(R, 1, n, generator=g, device=DEV) > 0.6
    cand[1, 0, :] = torch.arange(n, device=DEV) % 97 == 0  # row 1: fewer candidates than k
    base = index_score(q, k8, w, seq, i64(cls), k_scale=ks).cpu().numpy()
    sc = index_score(q, k8, w, seq, i64(cls), cand=cand, k_scale=ks).cpu().numpy()
    cm = cand.cpu().numpy()[:, 0]
    for i, c in enumerate(cls):
        np.testing.assert_array_equal(sc[i, :c][cm[i, :c]], base[i, :c][cm[i, :c]])
        assert np.all(np.isneginf(sc[i, :c][~cm[i, :c]]))
    want = O.topk_indices(sc, 2048, cls)
    for one in (True, False):
        sel = DecodeSelector(R, n, 2048, DEV, keep_scores=True, max_cl=n - 1 if one else None)
        if not one:
            sel.one_launch = False
        print(f"[decode candidates] one_launch {sel.one_launch}", flush=True)
        idx = sel(q, k8, w, seq, i64(cls), k_scale=ks, cand=cand)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(idx.cpu().numpy()[:, 0], want)


def test_topk_many_rows_bit_exact():
    """Prefill-shaped selection (many rows of <= 17408 positions: the 256-thread top-k), causal limits per row."""
    import dsv41_amd
    from dsv41_amd._lib import call, ptr
    r = rng(16)
    R, n, k = 600, 16896, 2048
    sc = r.standard_normal((R, n)).astype(np.float32)
    sc[::7] = np.round(sc[::7] * 3) / 3  # tie-heavy rows (the threshold's first-digit bin overflows the list)
    sc[3::11] = np.round(sc[3::11] * 64) / 64  # ties inside a listed bin
    sc[5::13, 100] = 1e30  # one outlier: the first digit spans the range, its threshold bin holds most positions
    start, ratio = 65536 - 4 * 600 + 4 * 16896 - 65536, 4  # rows see (start + i + 1) // 4 positions
    cls = [(start + i + 1) // ratio for i in range(R)]
    out = torch.empty(R, k, dtype=torch.int32, device=DEV)
    call("dsv41_topk_indices", ptr(f32(sc)), n, R, n, k, None, start, ratio, R, 7, ptr(out), k,
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = O.topk_indices(sc, k, cls)
    np.testing.assert_array_equal(out.cpu().numpy(), np.where(want >= 0, want + 7, -1))


@pytest.mark.parametrize("dqk,dv,h", [(576, 512, 64), (512, 512, 64), (576, 512, 40)])
def test_sparse_attn_prefill_shape(dqk, dv, h):
    """Many query rows (the prefill kernel): per-query index lists of window rows + compressed rows with -1 holes
    and out-of-range entries, against the reference's prefill rounding (bf16 QK and PV einsums)."""
    import dsv41_amd
    r = rng(17)
    b, s, n, t = 1, 320, 3000, 700
    q = O.bf16(r.standard_normal((b, s, h, dqk)).astype(np.float32))
    kv = O.bf16(r.standard_normal((b, n, dqk)).astype(np.float32) * 0.1)
    sink = r.standard_normal(h).astype(np.float32)
    idx = r.integers(0, n, (b, s, t)).astype(np.int32)
    idx[:, ::3, 100:180] = -1
    idx[:, 5, :] = -1  # a query with no valid key: output 0
    idx[:, 7, 3] = n + 11
    scale = dqk ** -0.5
    o = host(dsv41_amd.sparse_attn(bf(q), bf(kv), f32(sink), torch.from_numpy(idx).to(DEV), scale, d_v=dv))
    attn_close(o, O.sparse_attn(q, kv, sink, idx, scale, dv=dv), f"prefill {dqk}/{dv} h={h}")


@pytest.mark.parametrize("ratio", [2, 4])
def test_compress_pool_chunks(ratio):
    """Compressor.__call__ / DecodeRuntime.compressor2 (dsv41/model.py:593-660, dsv41/decode.py:243-265) after the
    projections: a sequence fed as prefill chunks (fresh, continuations with and without a partial group, longer than
    the ring) and decode steps of two sequences at once; latents (bf16, rmsnormed) within one bf16 step of the oracle,
    should flags and the fp32 rings exact."""
    import dsv41_amd  # noqa: F401
    from dsv41_amd import compressor as CP
    r = rng(33)
    D, R, S = 512, 8, 2
    w = O.bf16(r.random(D).astype(np.float32) + 0.5)
    rk_t, rs_t = CP.new_rings(S, D, DEV)
    rk = np.zeros((S, R, D), np.float32)
    rs = np.full((S, R, D), -np.inf, np.float32)
    start = 0
    for s in [5, 1, 1, 7, 1, 30, 2, 1, 1, 3]:
        kv = r.standard_normal((S, s, D)).astype(np.float32)
        sc = (2 * r.standard_normal((S, s, D))).astype(np.float32)
        print(f"[compress_pool] ratio {ratio} start {start} chunk {s}", flush=True)
        if s == 1 and start > 0:
            lat, should = CP.compress_pool_decode(f32(kv), f32(sc), i64([start, start + 3]), i64([0, 1]), ratio,
                                                  rk_t, rs_t, bf(w), 1e-6)
            # sequence 1 runs 3 positions ahead (its own ring), as a second slot of the decode batch
            want, wshould, rk, rs = O.compress_pool_decode(kv[:, 0], sc[:, 0], [start, start + 3], [0, 1], ratio, rk,
                                                           rs, w, 1e-6)
            np.testing.assert_array_equal(host(should), wshould)
            np.testing.assert_allclose(host(lat[:, 0]), want, rtol=2 ** -7, atol=1e-5)
        else:
            got = CP.compress_pool(f32(kv[:1]), f32(sc[:1]), start, ratio, rk_t[:1], rs_t[:1], bf(w), 1e-6)
            want, rk[0], rs[0] = O.compress_pool(kv[0], sc[0], start, ratio, rk[0], rs[0], w, 1e-6)
            if want is None:
                assert got is None
            else:
                assert got.shape == (1,) + want.shape
                np.testing.assert_allclose(host(got[0]), want, rtol=2 ** -7, atol=1e-5)
        np.testing.assert_array_equal(host(rk_t), rk)
        np.testing.assert_array_equal(host(rs_t), rs)
        start += s


def test_decode_appends_select_one_launch():
    """dsv41_decode_select (the decode step's cache appends and the one-launch indexer in one launch) == the
    appends launch followed by the indexer launch (dsv41/decode.py:129-164, :270-294): the same top-k indices and
    index keys / compressed rows / scales bit for bit, the ring rows up to rare one-step fp8 flips (the rmsnorm sum
    is reduced in another order), over steps that close a compression group (the new key is scored) and steps that
    do not (spare row), with a candidate mask on one step."""
    from dsv41_amd.decode import DecodeLayer
    from dsv41_amd.workloads import DecodeConfig, make_decode_inputs
    cfg = DecodeConfig("T", [65536, 8192, 40000, 12], topk=2048)
    layers, st = make_decode_inputs(cfg, DEV, seed=3)
    rd = 64
    ang = torch.outer(torch.arange(70000, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    l0 = layers[0]
    mk = lambda: DecodeLayer(l0["ring"].clone(), l0["ckv"].clone(), l0["k8"].clone(), l0["ks"].clone(), st["sink"],  # noqa: E731
                             cos, sin, cfg.ratio, cfg.topk, rd=rd)
    A, B = mk(), mk()
    g = torch.Generator(device=DEV).manual_seed(5)
    for step in range(4):
        pos = st["pos"] + step  # step 0 closes every row's group, 1-3 do not (spare rows), ...
        kv_raw = torch.randn(4, 576, generator=g, device=DEV).to(torch.bfloat16)
        latent = torch.randn(4, 1, 576, generator=g, device=DEV).to(torch.bfloat16)
        k_raw = (torch.randn(4, 128, generator=g, device=DEV) * 2).to(torch.bfloat16)
        q_idx = st["q_idx"] * (1 + step)
        cand = None
        if step == 3:
            cand = torch.rand(4, 1, A.k8.shape[1], generator=g, device=DEV) < 0.7
        print(f"[decode_select] step {step} pos {pos.tolist()}", flush=True)
        A.appends(kv_raw, st["kv_norm"], latent, k_raw, st["k_norm"], pos, st["seq"], q_idx, st["w_idx"])
        cl = torch.div(pos + 1, cfg.ratio, rounding_mode="floor")
        want = A.selector(4, DEV)(q_idx, A.k8, st["w_idx"], st["seq"], cl, k_scale=A.ks, prepared=A._prepared,
                                  cand=cand).clone()
        got = B.appends_select(kv_raw, st["kv_norm"], latent, k_raw, st["k_norm"], pos, st["seq"], q_idx,
                               st["w_idx"], cl=cl, cand=cand).clone()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy(), err_msg=f"step {step}")
        assert int(B.selector(4, DEV).fws[-4].item()) == 0, "row barrier wait gave up"
        np.testing.assert_array_equal(B.k8.view(torch.uint8).cpu().numpy(), A.k8.view(torch.uint8).cpu().numpy())
        np.testing.assert_array_equal(B.ks.cpu().numpy(), A.ks.cpu().numpy())
        np.testing.assert_array_equal(host(B.ckv), host(A.ckv))
        _fp8_close(host(B.ring), host(A.ring), f"decode_select ring step {step}")


@pytest.mark.parametrize("ctx", [[524288, 300000], [1048576]], ids=["two-rows", "C4-shape"])
def test_decode_score_appends_long_rows(ctx):
    """dsv41_decode_score (the decode step's cache appends and the indexer scores with their histogram in one
    launch, rows past the one-launch selection) then the top-k == the appends launch, the score launch and the
    top-k (dsv41/decode.py:129-164, :284-294): the same indices and scores bit for bit, the index keys, scales and
    compressed rows bit for bit, the ring rows up to rare one-step fp8 flips, over a step that closes every row's
    group (the new key is scored by its append workgroup) and one that does not (spare rows), with a candidate
    mask on the second.  The C4 shape (one row of 262144 positions) caps the score grid at the CUs the append
    workgroups leave and covers the rest of the row with one extra tile per wave."""
    from dsv41_amd.decode import DecodeLayer
    from dsv41_amd.workloads import DecodeConfig, make_decode_inputs
    cfg = DecodeConfig("T", ctx, topk=2048)
    R = len(ctx)
    layers, st = make_decode_inputs(cfg, DEV, seed=4)
    rd = 64
    ang = torch.outer(torch.arange(max(ctx) + 16, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    cos, sin = torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)
    l0 = layers[0]
    mk = lambda: DecodeLayer(l0["ring"].clone(), l0["ckv"].clone(), l0["k8"].clone(), l0["ks"].clone(), st["sink"],  # noqa: E731
                             cos, sin, cfg.ratio, cfg.topk, rd=rd)
    A, B = mk(), mk()
    assert not A.selector(R, DEV).one_launch
    g = torch.Generator(device=DEV).manual_seed(6)
    for step in range(2):
        pos = st["pos"] + step  # step 0 closes both rows' groups, step 1 does not
        kv_raw = torch.randn(R, 576, generator=g, device=DEV).to(torch.bfloat16)
        latent = torch.randn(R, 1, 576, generator=g, device=DEV).to(torch.bfloat16)
        k_raw = (torch.randn(R, 128, generator=g, device=DEV) * 2).to(torch.bfloat16)
        q_idx = st["q_idx"] * (1 + step)
        cand = torch.rand(R, 1, A.k8.shape[1], generator=g, device=DEV) < 0.8 if step == 1 else None
        print(f"[decode_score] step {step} pos {pos.tolist()}", flush=True)
        A.appends(kv_raw, st["kv_norm"], latent, k_raw, st["k_norm"], pos, st["seq"], q_idx, st["w_idx"])
        cl = torch.div(pos + 1, cfg.ratio, rounding_mode="floor")
        sa = A.selector(R, DEV)
        want = sa(q_idx, A.k8, st["w_idx"], st["seq"], cl, k_scale=A.ks, prepared=A._prepared, cand=cand).clone()
        got = B.appends_select(kv_raw, st["kv_norm"], latent, k_raw, st["k_norm"], pos, st["seq"], q_idx,
                               st["w_idx"], cl=cl, cand=cand).clone()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy(), err_msg=f"step {step}")
        sb = B.selector(R, DEV)
        for b, c in enumerate(cl.tolist()):
            np.testing.assert_array_equal(sb.score[b, :c].cpu().numpy(), sa.score[b, :c].cpu().numpy(),
                                          err_msg=f"scores row {b} step {step}")
        np.testing.assert_array_equal(B.k8.view(torch.uint8).cpu().numpy(), A.k8.view(torch.uint8).cpu().numpy())
        np.testing.assert_array_equal(B.ks.cpu().numpy(), A.ks.cpu().numpy())
        np.testing.assert_array_equal(host(B.ckv), host(A.ckv))
        _fp8_close(host(B.ring), host(A.ring), f"decode_score ring step {step}")


def test_sparse_attn_two_sources_and_topk_view():
    """kernels.sparse_attn over [window | compressed] read in place (kv2) with the index list in a preallocated
    buffer whose compressed columns index_topk fills (out=) == the reference's torch.cat of both
    (dsv41/model.py:1442-1443), bit for bit; also against the oracle."""
    import dsv41_amd
    from dsv41_amd.indexer import index_topk
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    r = rng(19)
    g = torch.Generator(device=DEV).manual_seed(19)
    h, dqk, dv, s, start, ratio, k = 64, 576, 512, 256, 4000, 4, 300
    n_w, n_c = 200, (start + s) // ratio
    q = bf(r.standard_normal((1, s, h, dqk)).astype(np.float32))
    win = bf(r.standard_normal((1, n_w, dqk)).astype(np.float32) * 0.1)
    ckv = bf(r.standard_normal((1, n_c + 5, dqk)).astype(np.float32) * 0.1)
    sink = f32(r.standard_normal(h).astype(np.float32))
    k8, ks = encode_e4m3_rows(fp4_round(torch.randn(1, n_c + 5, 128, generator=g, device=DEV) * 0.1))
    qi = fp4_round(torch.randn(1, s, 64, 128, generator=g, device=DEV))
    wi = torch.randn(1, s, 64, generator=g, device=DEV) * 0.01
    widx = torch.from_numpy(r.integers(-1, n_w, (1, s, 128)).astype(np.int32)).to(DEV)
    want_c = index_topk(qi, wi, k8, start, ratio, k, n_w, k_scale=ks)
    buf = torch.full((1, s, 128 + k + 9), 12345, dtype=torch.int32, device=DEV)  # wider rows than the index list
    index_topk(qi, wi, k8, start, ratio, k, n_w, k_scale=ks, out=buf[:, :, 128:128 + k])
    buf[:, :, :128] = widx
    np.testing.assert_array_equal(buf[:, :, 128:128 + k].cpu().numpy(), want_c.cpu().numpy())
    idx_cat = torch.cat([widx, want_c], dim=-1)
    scale = dqk ** -0.5
    want = dsv41_amd.sparse_attn(q, torch.cat([win, ckv[:, :n_c]], dim=1), sink, idx_cat, scale, d_v=dv)
    got = dsv41_amd.sparse_attn(q, win, sink, buf[:, :, :128 + k], scale, d_v=dv, kv2=ckv[:, :n_c])
    np.testing.assert_array_equal(host(got), host(want))
    kvc = np.concatenate([host(win), host(ckv)[:, :n_c]], axis=1)
    attn_close(host(got), O.sparse_attn(host(q), kvc, host(sink), idx_cat.cpu().numpy(), scale, dv=dv),
               "sparse_attn two sources")


@pytest.mark.parametrize("M,N,K,gc", [(1, 1280, 5120, 0), (4, 512, 5120, 0), (2, 200, 640, 0), (5, 16, 64, 0),
                                      (1, 4096, 1280, 0), (16, 384, 2048, 0), (20, 200, 640, 0), (70, 256, 1024, 0),
                                      (1, 2048, 1024, 256), (3, 1024, 512, 128), (16, 1040, 640, 0), (1, 3000, 640, 0),
                                      (1, 100, 2048, 0), (4, 700, 1024, 0), (1, 1024, 256, 128)])
def test_fp8_gemm(M, N, K, gc):
    """fp8_gemm_tc / fp8_gemv_m1 (dsv41/cukern.py:116-200): fp32 result within fp32 summation-order error of the
    exact (float64) oracle, bf16 result its rounding; e4m3 codes over the whole range (subnormals included), E8M0
    scales incl. the smallest, column tails (N % 64 != 0), split K, more than 64 rows, block-diagonal; the narrow
    (16-column) and vector (1-4 rows) kernels and, for one row, the split kernel on a 4-byte aligned x."""
    from dsv41_amd.w8 import fp8_gemm_tc
    r = rng(43)
    codes = r.integers(0, 256, (N, K)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x01  # NaN codes -> the smallest subnormal
    s8 = r.integers(100, 140, ((N + 31) // 32, K // 32)).astype(np.uint8)
    s8[0, 0] = 1  # 2^-126
    perm = codes.reshape(N, K // 16, 16)[:, :, O.PERM_K].reshape(N, K)
    G = N // gc if gc else 1
    x = O.bf16(r.standard_normal((M * G, K)).astype(np.float32))
    print(f"[fp8_gemm] M {M} N {N} K {K} group_cols {gc}", flush=True)
    w8 = torch.from_numpy(perm).to(DEV)
    s8t = torch.from_numpy(s8).to(DEV)
    got32 = fp8_gemm_tc(bf(x), w8, s8t, gc, out_dtype=torch.float32).cpu().numpy()
    got16 = host(fp8_gemm_tc(bf(x), w8, s8t, gc))
    want = O.fp8_gemm(x, perm, s8, gc)
    Wd = O.fp8_dequant(perm, s8).astype(np.float64)
    if gc:
        mag = np.concatenate([np.abs(x[g::G]) @ np.abs(Wd[g * gc:(g + 1) * gc]).T for g in range(G)], axis=1)
    else:
        mag = np.abs(x).astype(np.float64) @ np.abs(Wd).T
    err = np.abs(got32 - want)
    assert (err <= 1e-5 * mag + 1e-30).all(), (err / (mag + 1e-30)).max()
    np.testing.assert_array_equal(got16, O.bf16(got32))
    if M * G == 1:  # x only 4-byte aligned: the 64-column split kernel instead of the narrow one, same bound
        xb = torch.zeros(K + 2, dtype=torch.bfloat16, device=DEV)
        xb[2:] = bf(x)[0]
        got_u = fp8_gemm_tc(xb[2:].view(1, K), w8, s8t, gc, out_dtype=torch.float32).cpu().numpy()
        assert (np.abs(got_u - want) <= 1e-5 * mag + 1e-30).all()


@pytest.mark.parametrize("mode,N,K", [(1, 1024, 1280), (2, 512, 8192), (1, 4096, 16384), (2, 300, 128), (1, 5120, 2048)])
def test_fp8_gemv_m1_pre(mode, N, K):
    """fp8_gemv_m1_pre (dsv41/cukern.py:137-158): its prologue (norm_quant, dsv41/fused2.py:251-272; mode 2 the
    fake quantisation alone) equals the oracle's bf16(rmsnorm) -> fake_quant_fp8(32) -> bf16 bit for bit in mode 2
    and up to the last ulp of the fp32 variance sum in mode 1 (at most 0.5 % of the elements, one e4m3 step each);
    the one-launch fp8_gemv_m1_pre (prologue fused into the x staging) equals norm_quant + fp8_gemm_tc bit for bit
    and is within the fp8_gemm bound of the oracle's GEMV of that prologue."""
    from dsv41_amd.fused import norm_quant
    from dsv41_amd.w8 import fp8_gemm_tc, fp8_gemv_m1_pre
    r = rng(53)
    codes = r.integers(0, 256, (N, K)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x01
    s8 = r.integers(110, 130, ((N + 31) // 32, K // 32)).astype(np.uint8)
    perm = codes.reshape(N, K // 16, 16)[:, :, O.PERM_K].reshape(N, K)
    x = O.bf16(r.standard_normal((1, K)).astype(np.float32) * np.float32(3.0))
    x[0, :32] *= np.float32(1e-3)  # a small-magnitude group
    x = O.bf16(x)
    w = O.bf16(1.0 + 0.1 * r.standard_normal(K).astype(np.float32))
    eps = 1e-6
    print(f"[fp8_gemv_m1_pre] mode {mode} N {N} K {K}", flush=True)
    w8, s8t = torch.from_numpy(perm).to(DEV), torch.from_numpy(s8).to(DEV)
    xq = host(norm_quant(bf(x), bf(w) if mode == 1 else None, eps))
    y = O.bf16(O.rmsnorm(x, w, eps)) if mode == 1 else x
    want_q = O.bf16(O.fake_quant_fp8(y, 32))
    diff = xq != want_q
    if mode == 2:
        np.testing.assert_array_equal(xq, want_q)
    else:
        assert diff.mean() <= 5e-3, diff.mean()
        step = np.abs(want_q[diff]) * np.float32(2.0 ** -3) + 1e-30
        assert (np.abs(xq[diff] - want_q[diff]) <= step * 1.01).all()
    got = host(fp8_gemv_m1_pre(bf(x), w8, s8t, bf(w) if mode == 1 else None, eps, mode))
    xb = torch.zeros(K + 2, dtype=torch.bfloat16, device=DEV)  # 4-byte aligned x: the same (64-column) kernel
    xb[2:] = bf(xq)[0]
    np.testing.assert_array_equal(got, host(fp8_gemm_tc(xb[2:].view(1, K), w8, s8t)))  # fused == two launches
    want = O.fp8_gemm(xq, perm, s8)
    mag = np.abs(xq).astype(np.float64) @ np.abs(O.fp8_dequant(perm, s8).astype(np.float64)).T
    assert (np.abs(got - want) <= 1e-5 * mag + np.abs(want) * 2.0 ** -8 + 1e-30).all()


def test_index_key_snapshot_conversion():
    """Cache snapshots (dsv41/engine.py:1072-1230): the reference's bf16 index-key table -> e4m3 + per-row scale ==
    the oracle's key encoding bit for bit, and back == the original table exactly for FP4-grid rows (the reference's
    keys, dsv41/model.py:726); arbitrary bf16 rows round-trip to bf16(e4m3 x scale)."""
    from dsv41_amd.cache import index_keys_to_bf16, index_keys_to_e4m3
    r = rng(47)
    grid = _fp4_rows(r, (3, 40, 128))
    grid[0, 5] = 0.0  # an all-zero row
    any_rows = O.bf16(r.standard_normal((2, 33, 128)).astype(np.float32) * np.float32(3e-3))
    for tag, rows in (("fp4-grid", grid), ("arbitrary", any_rows)):
        k8, ks = index_keys_to_e4m3(bf(rows))
        q, s = O.key_encode_fp8(rows)
        want8 = torch.from_numpy(q).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        np.testing.assert_array_equal(k8.view(torch.uint8).cpu().numpy(), want8, err_msg=tag)
        np.testing.assert_array_equal(ks.cpu().numpy(), s[..., 0], err_msg=tag)
        back = host(index_keys_to_bf16(k8, ks))
        np.testing.assert_array_equal(back, O.bf16(q * s), err_msg=tag)
        if tag == "fp4-grid":
            np.testing.assert_array_equal(back, rows)
