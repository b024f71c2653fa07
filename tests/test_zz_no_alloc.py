"""dsv41_sattn2_noalloc (the sattn2 variant whose split partials and counters live in the library's static device
scratch) against dsv41_sattn2 with a caller workspace, through the C ABI: two calls in a row, the second with
fewer rows and a shorter index list (another counter layout in the shared scratch), bit-identical outputs; a call
whose workspace would exceed the scratch is rejected with hipErrorOutOfMemory."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(g, B, t, H=64, dqk=576, n_c=9000):
    S = B
    q = (torch.randn(B, 1, H, dqk, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    ring = (torch.randn(S, 128, dqk, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    ckv = (torch.randn(S, n_c, dqk, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    idx = torch.stack([torch.sort(torch.randperm(n_c, generator=torch.Generator().manual_seed(b))[:t]).values
                       for b in range(B)]).to(torch.int32).to(DEV)
    idx[:, -7:] = -1
    pos = torch.tensor([4 * n_c - 1 - 3 * b for b in range(B)], dtype=torch.int64, device=DEV)
    seq = torch.arange(B, dtype=torch.int64, device=DEV)
    sink = torch.randn(H, generator=g, device=DEV)
    return q, ring, ckv, idx, pos, seq, sink


def _args(q, ring, ckv, idx, pos, seq, sink, out):
    B, _, H, dqk = q.shape
    z = torch.zeros(1, device=DEV)
    return [q.data_ptr(), ring.data_ptr(), ring.stride(0), ring.shape[1], ckv.data_ptr(), ckv.stride(0), ckv.shape[1],
            idx.data_ptr(), idx.shape[-1], pos.data_ptr(), seq.data_ptr(), pos.data_ptr(), None, sink.data_ptr(),
            z.data_ptr(), z.data_ptr(), 0, dqk ** -0.5, out.data_ptr(), B, H, dqk, 512]


def test_sattn2_noalloc_matches_workspace_entry():
    from dsv41_amd._lib import lib
    L = lib()
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=DEV).manual_seed(71)
    for B, t in ((4, 2048), (2, 600)):
        q, ring, ckv, idx, pos, seq, sink = _inputs(g, B, t)
        want = torch.empty(B, 1, 64, 512, dtype=torch.bfloat16, device=DEV)
        got = torch.full_like(want, 7.0)
        nbytes = L.dsv41_attn_workspace_bytes(B, 64, 128 + t, 512, 0)
        assert 0 < nbytes <= 16 << 20
        ws = torch.zeros(nbytes // 4, dtype=torch.int32, device=DEV)
        print(f"[noalloc] B {B} t {t} workspace {nbytes}", flush=True)
        rc = L.dsv41_sattn2(*_args(q, ring, ckv, idx, pos, seq, sink, want), 0, ws.data_ptr(), nbytes, st)
        assert rc == 0
        rc = L.dsv41_sattn2_noalloc(*_args(q, ring, ckv, idx, pos, seq, sink, got), 0, st)
        assert rc == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())
        assert int(ws[0].item()) == 0
    # 48 rows with the library's split plan need ~60 MB of partials: rejected, nothing launched
    q, ring, ckv, idx, pos, seq, sink = _inputs(g, 48, 2048, n_c=2100)
    out = torch.zeros(48, 1, 64, 512, dtype=torch.bfloat16, device=DEV)
    assert L.dsv41_attn_workspace_bytes(48, 64, 128 + 2048, 512, 0) > 16 << 20
    rc = L.dsv41_sattn2_noalloc(*_args(q, ring, ckv, idx, pos, seq, sink, out), 0, st)
    assert rc == 2  # hipErrorOutOfMemory
    # ... and accepted with fewer splits
    want = torch.empty_like(out)
    nbytes = L.dsv41_attn_workspace_bytes(48, 64, 128 + 2048, 512, 2)
    ws = torch.zeros(max(nbytes, 4) // 4, dtype=torch.int32, device=DEV)
    assert L.dsv41_sattn2(*_args(q, ring, ckv, idx, pos, seq, sink, want), 2, ws.data_ptr(), nbytes, st) == 0
    assert L.dsv41_sattn2_noalloc(*_args(q, ring, ckv, idx, pos, seq, sink, out), 2, st) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())
    assert ctypes.sizeof(ctypes.c_void_p) == 8
