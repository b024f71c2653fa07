"""GPU parity of the one-launch decode indexer's two selection paths (dsv41_index_select / dsv41_decode_select):
the one-exchange path (every chunk publishes its top keys, every chunk finds the row's k-th largest among them)
and the histogram + candidate exchanges it falls back to when a chunk holds more of the selection than it
published or keys tie at the threshold.  Every call's selection is bit-exact against the oracle's top-k of the
kernel's own scores (the reference's topk_indices, dsv41/fused3.py:65-75, ties lowest index first), whichever path
a row takes, and the workspace stays consistent when calls alternate between the paths.  DSV41_IS_PUB_M forces
the paths: 0 = the two exchanges only, 4 = too few published keys (nearly every row falls back)."""
import numpy as np
import pytest
import torch

from oracle import dsv41_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
CLS = [32768, 32768, 20000, 1500]


def _inputs(kind, seed):
    from dsv41_amd.workloads import encode_e4m3_rows, fp4_round
    g = torch.Generator(device=DEV).manual_seed(seed)
    n = max(CLS) + 1
    keys = torch.randn(3, n, 128, generator=g, device=DEV) * 0.1
    q = fp4_round(torch.randn(len(CLS), 1, 64, 128, generator=g, device=DEV))
    if kind == "clustered":
        # one 512-position chunk of each slot aligned with every row's query: the whole chunk is selected (more than
        # any chunk publishes)
        keys[:, 5120:5632] += q[0, 0].float().mean(0) * 0.5
    elif kind == "ties":
        # every key row is one of 6 rows: each row's scores take at most 6 values, so the k-th largest ties
        keys = keys[:, torch.randint(0, 6, (n,), generator=g, device=DEV) % 6 + 7]
    k8, ks = encode_e4m3_rows(fp4_round(keys))
    w = (torch.randn(len(CLS), 64, generator=g, device=DEV).abs() * 0.01).to(torch.bfloat16)
    return q, k8, ks, w


def _check(sel, q, k8, ks, w, tag):
    seq = torch.tensor([0, 2, 1, 2], dtype=torch.int64, device=DEV)
    cl = torch.tensor(CLS, dtype=torch.int64, device=DEV)
    print(f"[select paths] {tag}", flush=True)
    idx = sel(q, k8, w, seq, cl, k_scale=ks)
    torch.cuda.synchronize()
    sc = sel.score.cpu().numpy()
    np.testing.assert_array_equal(idx.cpu().numpy()[:, 0], O.topk_indices(sc, 2048, CLS), err_msg=tag)
    assert int(sel.fws[-4].item()) == 0, f"{tag}: a row barrier wait gave up"


@pytest.mark.parametrize("pub_m", ["", "0", "4"], ids=["default", "two-exchange", "fallback"])
@pytest.mark.parametrize("kind", ["gauss", "clustered", "ties"])
def test_index_select_paths(pub_m, kind, monkeypatch):
    from dsv41_amd.fused3 import DecodeSelector
    if pub_m:
        monkeypatch.setenv("DSV41_IS_PUB_M", pub_m)
    else:
        monkeypatch.delenv("DSV41_IS_PUB_M", raising=False)
    sel = DecodeSelector(len(CLS), max(CLS) + 1, 2048, DEV, keep_scores=True)
    assert sel.one_launch
    q, k8, ks, w = _inputs(kind, 41)
    for rep in range(2):  # the second call reuses the workspace
        _check(sel, q, k8, ks, w, f"{kind} pub_m={pub_m or 'default'} call {rep}")


def test_index_select_alternating_paths(monkeypatch):
    """Calls that alternate between rows taking the one-exchange path and rows falling back share one workspace:
    every call's selection stays exact (epochs, flags, the histogram left zeroed by the fallback)."""
    from dsv41_amd.fused3 import DecodeSelector
    monkeypatch.delenv("DSV41_IS_PUB_M", raising=False)
    sel = DecodeSelector(len(CLS), max(CLS) + 1, 2048, DEV, keep_scores=True)
    data = {k: _inputs(k, 42 + i) for i, k in enumerate(["gauss", "clustered", "ties"])}
    for i, kind in enumerate(["gauss", "clustered", "gauss", "ties", "ties", "gauss", "clustered", "gauss"]):
        _check(sel, *data[kind], f"alternating call {i} ({kind})")
    assert int(sel.fws[:len(CLS) * 4096].abs().sum().item()) == 0, "row histogram not left zeroed"
