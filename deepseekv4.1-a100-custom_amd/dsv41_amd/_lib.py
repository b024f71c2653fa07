"""Loader of the HIP library (libdsv41_hip.so, C ABI in include/dsv41_hip.h) and launch helpers.

The library is built in-tree (dsv41_amd/build.py).  There is no fallback: when the library is missing, or the
tensors are not on a GPU, the entry points raise."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("DSV41_HIP_LIB") or Path(__file__).resolve().parent / "libdsv41_hip.so")

_P, _L, _I, _F = ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_float

# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "dsv41_attn_workspace_bytes": [_I, _I, _I, _I, _I],
    "dsv41_sparse_attn": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _L, _I, _F, _I, _P, _L, _P],
    "dsv41_sparse_attn_kv2": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _L, _I, _L, _I, _L, _F, _I, _P, _L, _P],
    "dsv41_sparse_attn2": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _L, _I, _L, _I, _F, _I, _P, _L, _P],
    "dsv41_sattn2": [_P, _P, _L, _I, _P, _L, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P, _I, _I, _I, _I, _I,
                     _P, _L, _P],
    "dsv41_sattn2_noalloc": [_P, _P, _L, _I, _P, _L, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P, _I, _I, _I,
                             _I, _I, _P],
    "dsv41_index_score": [_P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _L, _P, _I, _P, _L, _I, _I, _I, _P, _L, _P,
                          _P, _L, _P],
    "dsv41_select_workspace_bytes": [_I, _I],
    "dsv41_index_select_workspace_bytes": [_I, _I],
    "dsv41_index_select": [_P, _L, _P, _L, _I, _I, _P, _L, _P, _L, _P, _P, _I, _I, _I, _P, _L, _P, _L, _P, _L, _P,
                           _L, _P],
    "dsv41_candidate_blocks_workspace_bytes": [_I, _I, _I, _I],
    "dsv41_candidate_blocks": [_P, _L, _I, _I, _I, _P, _L, _I, _I, _I, _I, _P, _L, _P, _L, _P],
    "dsv41_select_topk": [_P, _L, _I, _I, _I, _P, _I, _P, _L, _P, _L, _P],
    "dsv41_topk_indices": [_P, _L, _I, _I, _I, _P, _L, _I, _I, _I, _P, _L, _P],
    "dsv41_kv_write": [_P, _L, _P, _P, _P, _P, _P, _L, _L, _I, _P, _L, _I, _P, _I, _I, _I, _F, _I, _P],
    "dsv41_window_kv": [_P, _L, _P, _P, _P, _L, _I, _P, _I, _P, _I, _I, _I, _F, _P],
    "dsv41_append_rows": [_P, _L, _P, _F, _P, _P, _I, _P, _L, _L, _L, _P, _I, _P, _L, _P, _L, _I, _I, _P, _L, _P, _L,
                          _I, _I, _P],
    "dsv41_decode_appends": [_P, _P, _P, _L, _I, _I, _P, _P, _L, _I, _P, _P, _P, _L, _P, _L, _P, _L, _I, _I, _P, _P,
                             _P, _I, _P, _P, _I, _F, _P, _P, _I, _P, _P, _I, _P],
    "dsv41_index_qprep": [_P, _P, _I, _I, _P, _P, _P],
    "dsv41_fake_quant": [_P, _P, _L, _I, _I, _I, _P],
    "dsv41_rope": [_P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P],
    "dsv41_rmsnorm": [_P, _P, _P, _L, _I, _F, _P],
    "dsv41_norm_quant": [_P, _P, _F, _P, _L, _I, _P],
    "dsv41_decode_select": [_P, _P, _P, _L, _I, _I, _P, _P, _L, _I, _P, _P, _P, _L, _P, _L, _P, _L, _I, _P, _P, _P, _I,
                            _I, _P, _P, _I, _F, _P, _P, _I, _P, _I, _I, _I, _P, _L, _P, _L, _P, _L, _P, _L, _P],
    "dsv41_decode_score": [_P, _P, _P, _L, _I, _I, _P, _P, _L, _I, _P, _P, _P, _L, _P, _L, _P, _L, _I, _P, _P, _P, _I,
                           _I, _P, _P, _I, _F, _P, _P, _I, _P, _I, _P, _L, _P, _P, _L, _P],
    "dsv41_index_keys_encode": [_P, _L, _P, _P, _P],
    "dsv41_index_keys_decode": [_P, _P, _L, _P, _P],
    "dsv41_fp8_gemm_workspace_bytes": [_I, _I, _I],
    "dsv41_fp8_gemv_m1_pre": [_P, _P, _F, _I, _P, _P, _I, _I, _I, _P, _P, _L, _P],
    "dsv41_fp8_gemm": [_P, _L, _P, _P, _I, _I, _I, _I, _I, _P, _L, _P, _P, _L, _P],
    "dsv41_compress_pool_decode": [_P, _P, _L, _P, _P, _L, _I, _P, _P, _I, _I, _I, _P, _F, _P, _L, _P, _P],
    "dsv41_compress_pool_prefill": [_P, _P, _L, _P, _P, _I, _L, _I, _I, _I, _P, _F, _P, _L, _I, _P],
}
_RESTYPE = {"dsv41_attn_workspace_bytes": _L, "dsv41_select_workspace_bytes": _L,
            "dsv41_index_select_workspace_bytes": _L, "dsv41_candidate_blocks_workspace_bytes": _L,
            "dsv41_fp8_gemm_workspace_bytes": _L}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, argt in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = argt
            f.restype = _RESTYPE.get(name, _I)
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name}: hip error {rc}")


# DSV41_CHECK_ERRORS=1: after launches whose kernels report through a workspace error word (the one-launch indexer's
# row barriers, the decode attention's in-launch split merge), synchronise, read the word, clear it and raise when it
# is set.  Off by default: it costs a host synchronisation per launch and is not legal under graph capture.
CHECK_ERRORS = os.environ.get("DSV41_CHECK_ERRORS", "0") == "1"

_ERR_TEXT = {("index_select", 1): "a row barrier wait gave up (the row's workgroups were not resident together)",
             ("index_select", 2): "a valid count cl exceeded the positions scored (clamped)",
             ("attention", 1): "a split merge stopped waiting for its unit (workgroups not resident together)",
             ("attention", 2): "a split merge ran off its unit's XCD (workgroups not dealt to the XCDs round-robin)"}


def check_error_word(kind: str, word: torch.Tensor) -> None:
    """Read the int32 error word `word` (a one-element view of a workspace), clear it and raise RuntimeError when it
    is set.  Synchronises the word's device."""
    v = int(word.item())
    if v != 0:
        word.zero_()
        raise RuntimeError(f"{kind}: {_ERR_TEXT.get((kind, v), f'error word {v}')}")


def attn_error_word(ws: torch.Tensor | None, R: int, H: int, nbytes: int):
    """The error word of an attention workspace, or None when the launch has none (no split, or the 64-head kernel,
    whose splits are merged by a separate launch).  The decode kernel runs when R * ceil(H / 64) < 16."""
    if ws is None or nbytes <= 0 or R * ((H + 63) // 64) >= 16:
        return None
    return ws.view(torch.int32)[:1]


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def require_gpu(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"dsv41_amd kernels need GPU tensors (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def as_i64(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """Index tensors (pos, seq, cl, ...) as contiguous int64 on the launch device."""
    if t.device != dev or t.dtype != torch.int64 or not t.is_contiguous():
        t = t.to(device=dev, dtype=torch.int64, non_blocking=True).contiguous()
    return t

