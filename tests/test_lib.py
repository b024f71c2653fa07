"""The C-ABI library loads and exports every symbol include/dsv41_hip.h declares (CPU: no compute calls)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "dsv41_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|long)\s+(dsv41_\w+)\s*\(", txt, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "dsv41_sattn2" in syms and "dsv41_topk_indices" in syms and len(syms) >= 11


def test_library_exports_every_declared_symbol():
    from dsv41_amd import _lib
    L = ctypes.CDLL(str(_lib.LIB_PATH))
    for s in declared_symbols():
        assert hasattr(L, s), s
    assert set(declared_symbols()) == set(_lib.SIGNATURES), "python signatures out of sync with the header"


def test_shims_refuse_cpu_tensors():
    import pytest
    import torch
    import dsv41_amd
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    kv = torch.zeros(1, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        dsv41_amd.sparse_attn(q, kv, torch.zeros(4), torch.zeros(1, 1, 4, dtype=torch.int32), 0.1)


def test_workspace_query_is_pure():
    from dsv41_amd._lib import lib
    L = lib()
    assert L.dsv41_attn_workspace_bytes(2048, 64, 2176, 512, 0) == 0  # many rows: one split per row
    n = L.dsv41_attn_workspace_bytes(4, 64, 2176, 512, 0)
    assert n > 0 and n % 4 == 0
