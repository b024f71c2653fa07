"""dsv41_decode_step (the whole decode layer-step in one launch: appends, indexer scores + top-k, sparse attention)
against the two-launch path it replaces (dsv41_decode_select then dsv41_sattn2) and against the oracle:
  * the index lists and scores bit-exact against the two-launch path, the selection bit-exact against the oracle's
    top-k of the kernel's own scores;
  * the cache rows (ring, compressed, e4m3 key + scale) bit-exact against the two-launch path;
  * the attention output within the bf16 bar of the oracle's sattn2 over the same selection.
Shapes: C2 (4 slots x 32768 compressed rows, 64 chunks per row), a 16-chunk case with a short row (every valid
position selected), the reference geometry (512-wide rows with rope, 32 index heads, ratio 2, top-k 512), and scores
concentrated in one chunk (the second publication round)."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def host(t):
    return t.float().cpu().numpy()


def _tables(rd, n):
    ang = torch.outer(torch.arange(n, dtype=torch.float32),
                      1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd)))
    return torch.cos(ang).to(DEV), torch.sin(ang).to(DEV)


def _layer_pair(ctx, Dw, HI, ratio, k, seed, hot_chunk=None):
    from dsv41_amd.decode import DecodeLayer
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(seed)
    S = len(ctx)
    cap = max((c + 2) // ratio for c in ctx) + 1  # (room for the steps; the last row is the spare row)
    ring = (torch.randn(S, 128, Dw, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    ckv = (torch.randn(S, cap, Dw, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    kk = torch.randn(S, cap, 128, generator=g, device=DEV) * 0.1
    kk[..., [3, 40, 77, 120]] *= 8
    if hot_chunk is not None:  # one chunk of 512 positions holds the largest keys of every slot
        kk[:, hot_chunk * 512:(hot_chunk + 1) * 512] *= 4
    k8, ks = encode_e4m3_rows(fp4_round(kk))
    rd = 64
    cos, sin = _tables(rd, max(ctx) + 16)
    sink = torch.randn(64, generator=g, device=DEV)
    mk = lambda: DecodeLayer(ring.clone(), ckv.clone(), k8.clone(), ks.clone(), sink, cos, sin, ratio, k, rd=rd,  # noqa: E731
                             dv=512)
    return mk(), mk(), g, cos, sin


@pytest.mark.parametrize("case", ["C2", "short16", "reference", "hot"])
def test_decode_step_one_launch(case):
    from dsv41_amd.workloads import fp4_round
    Dw, HI, ratio, k = 576, 64, 4, 2048
    hot = None
    if case == "C2":
        ctx = [131072] * 4
    elif case == "short16":
        ctx = [32768, 4096, 20000, 130]  # 8192 positions -> 16 chunks; row 1..3 select every valid position
    elif case == "reference":
        Dw, HI, ratio, k, ctx = 512, 32, 2, 512, [16380, 9000, 16380, 700]
    else:
        ctx, hot = [65536, 65536, 65536, 65536], 7
    A, Bl, g, cos, sin = _layer_pair(ctx, Dw, HI, ratio, k, 90 + len(case), hot)
    R = len(ctx)
    if not A.fused_fits(R, 64):
        pytest.skip("the device cannot hold the one-launch grid")
    n_sel = A.k8.shape[1] - 1
    seq = torch.arange(R, dtype=torch.int64, device=DEV)
    kvn = (torch.rand(Dw, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    kn = (torch.rand(128, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    sink = A.sink.cpu().numpy()
    for step in range(3):
        pos_l = [c - 1 + step for c in ctx]  # step 0 closes every group (ratio | ctx), later steps do not
        pos = torch.tensor(pos_l, dtype=torch.int64, device=DEV)
        cl = torch.div(pos + 1, ratio, rounding_mode="floor")
        q = (torch.randn(R, 1, 64, Dw, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
        kv_raw = torch.randn(R, Dw, generator=g, device=DEV).to(torch.bfloat16)
        latent = torch.randn(R, 1, Dw, generator=g, device=DEV).to(torch.bfloat16)
        k_raw = (torch.randn(R, 128, generator=g, device=DEV) * 2).to(torch.bfloat16)
        q_idx = fp4_round(torch.randn(R, 1, HI, 128, generator=g, device=DEV))
        w_idx = (torch.randn(R, HI, generator=g, device=DEV) * (128 ** -0.5 * HI ** -0.5)).to(torch.bfloat16)
        print(f"[step {case}] step {step} pos {pos_l}", flush=True)
        # two-launch path
        sel = Bl.selector(R, DEV)
        sel.keep_scores = True
        idx_b = Bl.appends_select(kv_raw, kvn, latent, k_raw, kn, pos, seq, q_idx, w_idx, cl=cl).clone()
        o_b = Bl.attend(q, idx_b, pos, seq, pos, plim=pos)
        # one launch
        idx_a = torch.full((R, k), 12345, dtype=torch.int32, device=DEV)
        sc_a = torch.full((R, n_sel), float("nan"), dtype=torch.float32, device=DEV)
        o_a = A.step_fused(q, kv_raw, kvn, latent, k_raw, kn, pos, seq, q_idx, w_idx, pos, plim=pos, cl=cl,
                           idx_out=idx_a, score_out=sc_a)
        torch.cuda.synchronize()
        ws = A._attn_ws[("step", R, n_sel, 64, 512 if Dw == 576 else Dw)]
        assert int(ws.view(torch.int32)[0].item()) == 0, "a row-wide wait gave up"
        cls = cl.tolist()
        for b in range(R):
            c = cls[b]
            np.testing.assert_array_equal(host(sc_a[b, :c]), host(sel.score[b, :c]), err_msg=f"scores row {b}")
        np.testing.assert_array_equal(idx_a.cpu().numpy(), idx_b.cpu().numpy()[:, 0], err_msg=f"step {step}")
        np.testing.assert_array_equal(idx_a.cpu().numpy(), O.topk_indices(host(sc_a), k, cls))
        np.testing.assert_array_equal(A.k8.view(torch.uint8).cpu().numpy(), Bl.k8.view(torch.uint8).cpu().numpy())
        np.testing.assert_array_equal(A.ks.cpu().numpy(), Bl.ks.cpu().numpy())
        np.testing.assert_array_equal(host(A.ckv), host(Bl.ckv))
        np.testing.assert_array_equal(host(A.ring), host(Bl.ring))
        # attention against the oracle over the same selection (and the two-launch output)
        rd_out = 0 if Dw == 576 else 64
        want = O.sattn2(host(q), host(A.ring), host(A.ckv), idx_a.cpu().numpy()[:, None], pos_l, list(range(R)),
                        pos_l, pos_l, sink, host(cos), host(sin), rd_out, Dw ** -0.5, dv=512)
        err = np.abs(host(o_a) - want)
        print(f"[step {case}] step {step} attention max {err.max():.3e} mean {err.mean():.3e}; vs two-launch "
              f"{np.abs(host(o_a) - host(o_b)).max():.3e}", flush=True)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3
        assert np.abs(host(o_a) - host(o_b)).max() <= 2e-2
