"""The layer-level drop-ins against the oracle's composition: SparseAttention (Attention.__call__ up to the
o-projection, dsv41/model.py:1350-1573) and indexer_query (dsv41/model.py:734-746), at the reference's head geometry
(64 heads x 512 with the rope on the last 64, 32 index heads x 128, ratio 4, top-k 512, window 128) and reduced model
widths, over a fresh prefill chunk, a continuation chunk whose compressed rows exceed top-k, and decode steps.

Bars: attention output max |err| <= 2e-2 and mean <= 2e-3; cache rows bit-exact up to rare
one-step fp8/fp4 flips (bf16 GEMM outputs and rmsnorm sums reduced in another order)."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O
from _layer_weights import layer_weights

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def t(x, dt=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float32))).to(dt).to(DEV)


def host(x):
    return x.float().cpu().numpy()


def close(got, want, tag, mx=2e-2, mean=2e-3):
    err = np.abs(got - want)
    print(f"[{tag}] max {err.max():.3e} mean {err.mean():.3e}", flush=True)
    assert err.max() <= mx and err.mean() <= mean, tag


def rows_close(got, want, tag, frac=5e-3):
    diff = got != want
    print(f"[{tag}] mismatching elements {diff.sum()} ({diff.mean():.2e})", flush=True)
    assert diff.mean() <= frac, tag
    if diff.any():
        rel = np.abs(got[diff] - want[diff]) / np.maximum(np.abs(want[diff]), 1e-30)
        assert rel.max() <= 0.5, (tag, rel.max())


def _w8(rng, N, K):
    """A random FP8 block-scaled weight (e4m3 bytes without NaN codes, E8M0 scales) and its exact dequantisation."""
    from dsv41_amd.w8 import W8
    b = rng.integers(0, 256, (N, K)).astype(np.uint8)
    b = np.where((b & 0x7F) == 0x7F, np.uint8(0x38), b)
    s8 = rng.integers(112, 118, ((N + 31) // 32, K // 32)).astype(np.uint8)
    w = W8(torch.from_numpy(b).to(DEV), torch.from_numpy(s8).to(DEV))
    return w, O.fp8_dequant(b, s8, permuted=False)


def test_indexer_query():
    """a5: q = fq4(rope(linear_fp8(qr, wq_b)), 32), weights = F.linear(x, weights_proj) * d^-1/2 H^-1/2, with a bf16
    and an FP8 (W8) wq_b, at host and device positions."""
    from dsv41_amd.attention import indexer_query
    rng = np.random.default_rng(80)
    b, s, dim, q_rank, HI, rd = 2, 5, 1024, 256, 32, 64
    cos, sin = O.rope_tables(rd, 4096, 0, 10000.0, 1.0, 32, 1)
    x = O.bf16(rng.standard_normal((b, s, dim)).astype(np.float32))
    qr = O.bf16(rng.standard_normal((b, s, q_rank)).astype(np.float32))
    wp = O.bf16(rng.standard_normal((HI, dim)).astype(np.float32) * dim ** -0.5)
    w8, wdq = _w8(rng, HI * 128, q_rank)
    wbf = O.bf16(rng.standard_normal((HI * 128, q_rank)).astype(np.float32) * q_rank ** -0.5)
    for name, wg, wo in (("bf16", t(wbf), wbf), ("w8", w8, wdq)):
        q, w = indexer_query(t(x), t(qr), wg, t(wp), t(cos, torch.float32), t(sin, torch.float32), rd, 300, HI)
        wq, ww = O.indexer_query(x, qr, wo, wp, cos, sin, rd, 300, HI)
        assert q.shape == (b, s, HI, 128) and w.shape == (b, s, HI)
        rows_close(host(q), wq, f"indexer_query q {name}", frac=2e-3)
        np.testing.assert_allclose(host(w), ww, rtol=2 ** -7, atol=1e-6)
    # device positions (rope_dev_): one position per batch row, here both 300 -> the same result
    q2, _ = indexer_query(t(x[:, :1]), t(qr[:, :1]), w8, t(wp), t(cos, torch.float32), t(sin, torch.float32), rd, 0,
                          HI, pos=torch.tensor([300, 300], device=DEV))
    q1, _ = indexer_query(t(x[:, :1]), t(qr[:, :1]), w8, t(wp), t(cos, torch.float32), t(sin, torch.float32), rd, 300,
                          HI)
    np.testing.assert_array_equal(host(q2), host(q1))


@pytest.mark.parametrize("e4m3", [True, False])
def test_sparse_attention_layer(e4m3):
    """a1: SparseAttention.attend against O.AttentionLayer; wq_a is an FP8 (W8) weight.  e4m3: the selection reads
    the e4m3 copy of the index keys, over a fresh 700-token chunk, a 1450-token continuation (537 compressed rows >
    top-k 512: a real selection) and two decode steps; bf16 (the reference's key table): a fresh chunk, a decode step
    and a continuation after it."""
    from dsv41_amd.attention import SparseAttention
    rng = np.random.default_rng(81)
    dim, q_rank, H, D, rd, W, ratio, HI, topk = 1024, 256, 64, 512, 64, 128, 4, 32, 512
    wts = layer_weights(rng, dim, q_rank, H, D, HI)
    w8, wdq = _w8(rng, q_rank, dim)
    wts_o = dict(wts, wq_a=wdq)
    cos, sin = O.rope_tables(rd, 4096, 0, 10000.0, 1.0, 32, 1)
    kw = dict(n_heads=H, head_dim=D, rope_head_dim=rd, window=W, ratio=ratio, index_n_heads=HI, index_topk_k=topk,
              slots=1, cap=560)
    ref = O.AttentionLayer(wts_o, cos=cos, sin=sin, **kw)
    wg = {k: (t(v, torch.float32) if k in ("c_wkv", "c_wgate", "attn_sink") else t(v)) for k, v in wts.items()}
    wg["wq_a"] = w8
    layer = SparseAttention(wg, cos=t(cos, torch.float32), sin=t(sin, torch.float32), e4m3=e4m3, **kw)
    x = O.bf16(rng.standard_normal((1, 2152, dim)).astype(np.float32))
    steps = ((0, 700), (700, 2150), (2150, 2151), (2151, 2152)) if e4m3 else ((0, 700), (700, 701), (701, 1300))
    for a, b in steps:
        print(f"[layer e4m3={e4m3}] positions {a}..{b - 1}", flush=True)
        got = host(layer.attend(t(x[:, a:b]), a))
        want = ref.attend(x[:, a:b], a)
        close(got, want, f"layer e4m3={e4m3} o {a}..{b - 1}")
        rows_close(host(layer.ring), ref.ring, f"ring after {b}")
        rows_close(host(layer.ckv), ref.ckv, f"compressed rows after {b}")
        rows_close(host(layer.index_k), ref.index_k, f"index keys after {b}")
    if e4m3:
        dec = layer.k8.view(torch.float8_e4m3fn).float().cpu().numpy() * layer.ks.cpu().numpy()[..., None]
        np.testing.assert_array_equal(dec, host(layer.index_k))
