"""Drop-in for the FP8 block-scaled projections around the attention path: dsv41/w8.py (weight container and byte
order) and the fp8_gemm_tc / fp8_gemv_m1 / fp8_gemv_m1_pre operators of dsv41/cukern.py:116-200.  Weights are e4m3
bytes [N, K] with every 16-k group in the PERM_K byte order and E8M0 scales per [32 x 32] block; x is bf16; the
products are exact (e4m3 x power of two in bf16) and accumulate in fp32 (dsv41_fp8_gemm)."""
from __future__ import annotations

import torch

from ._lib import call, lib, ptr, require_gpu, stream

# Byte order of every 16-k group in memory (dsv41/w8.py:23): position p holds k = PERM_K[p].
PERM_K = [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15]
_INV_PERM_K = [PERM_K.index(i) for i in range(16)]


def permute_k(w8: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K] natural k order -> the in-memory order of the fp8 kernels (dsv41/w8.py:27-31)."""
    N, K = w8.shape
    assert K % 16 == 0
    return w8.view(N, K // 16, 16)[:, :, PERM_K].reshape(N, K).contiguous()


def unpermute_k(w8: torch.Tensor) -> torch.Tensor:
    N, K = w8.shape
    return w8.view(N, K // 16, 16)[:, :, _INV_PERM_K].reshape(N, K).contiguous()


class W8:
    """dsv41/w8.py:39-60: e4m3 bits [N, K] (natural k order unless permuted=True) + E8M0 scales [ceil(N/32), K/32]."""
    __slots__ = ("w8", "s8", "shape", "device")

    def __init__(self, w8: torch.Tensor, s8: torch.Tensor, permuted: bool = False):
        assert w8.dtype == torch.uint8 and s8.dtype == torch.uint8 and w8.dim() == 2
        self.w8 = w8.contiguous() if permuted else permute_k(w8)
        self.s8 = s8.contiguous()
        self.shape = tuple(w8.shape)
        self.device = w8.device

    @property
    def dtype(self):
        return torch.bfloat16

    def bf16(self) -> torch.Tensor:
        """The dequantised weight (exact): e4m3 value x 2^(scale - 127) per block, bf16 [N, K]."""
        N, K = self.shape
        w = unpermute_k(self.w8).view(torch.float8_e4m3fn).float()
        e = self.s8.to(torch.int32) - 127
        sc = torch.ldexp(torch.ones_like(e, dtype=torch.float32), e)
        sc = sc.repeat_interleave(32, 0)[:N].repeat_interleave(32, 1)[:, :K]
        return (w * sc).to(torch.bfloat16)

    @staticmethod
    def cat(ws: list) -> "W8":
        """Concatenate along N (row counts must be multiples of 32), dsv41/w8.py."""
        assert all(w.shape[0] % 32 == 0 for w in ws)
        return W8(torch.cat([w.w8 for w in ws], 0), torch.cat([w.s8 for w in ws], 0), permuted=True)


_WS: dict = {}


def _workspace(dev, M, N, K):
    n = lib().dsv41_fp8_gemm_workspace_bytes(M, N, K)
    if n <= 0:
        return None, 0
    key = (dev, M, N, K)
    ws = _WS.get(key)
    if ws is None:  # zeroed once: every launch leaves its split counters at zero
        ws = _WS[key] = torch.zeros((n + 3) // 4, dtype=torch.int32, device=dev)
    return ws, n


def fp8_gemm_tc(x: torch.Tensor, w8: torch.Tensor, s8: torch.Tensor, group_cols: int = 0,
                out_dtype=torch.bfloat16) -> torch.Tensor:
    """dsv41/cukern.py:164-200: x bf16 [M, K]; w8 uint8 (e4m3 bits) [N, K] in the PERM_K byte order; s8 uint8 (E8M0)
    [ceil(N/32), K/32] -> x @ dequant(w8, s8)^T as [M, N] (fp32 accumulation, rounded to out_dtype: bf16 or fp32).
    group_cols > 0: block-diagonal (x: [B * N/group_cols, K]; output row b, column n uses x row
    b * (N/group_cols) + n // group_cols) -> [B, N]."""
    dev = require_gpu(x, w8, s8)
    K = x.shape[-1]
    N = w8.shape[0]
    xc = x.reshape(-1, K)
    if xc.dtype != torch.bfloat16:
        xc = xc.to(torch.bfloat16)
    xc = xc.contiguous()
    assert w8.dtype == torch.uint8 and w8.is_contiguous() and s8.is_contiguous() and w8.shape[1] == K
    Mo = xc.shape[0] // (N // group_cols) if group_cols else xc.shape[0]
    out = torch.empty(Mo, N, device=dev, dtype=torch.bfloat16)
    outf = torch.empty(Mo, N, device=dev, dtype=torch.float32) if out_dtype == torch.float32 else None
    ws, n = _workspace(dev, Mo, N, K)
    call("dsv41_fp8_gemm", ptr(xc), K, ptr(w8), ptr(s8), Mo, N, K, s8.shape[1], int(group_cols), ptr(out), N,
         ptr(outf), ptr(ws), n, stream(dev))
    return outf if outf is not None else out


def fp8_gemv_m1(x: torch.Tensor, w8: torch.Tensor, s8: torch.Tensor, group_cols: int = 0,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """dsv41/cukern.py:116-134: one row (or the block-diagonal rows of one token) -> bf16 [1, N]."""
    y = fp8_gemm_tc(x, w8, s8, group_cols)
    if out is not None:
        out.copy_(y.view_as(out))
        return out
    return y


def fp8_gemv_m1_pre(x_raw: torch.Tensor, w8: torch.Tensor, s8: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                    mode: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """dsv41/cukern.py:137-158: the GEMV with its activation prologue: mode 1 = rmsnorm(x_raw) * norm_w then per-32
    fp8 fake quant, mode 2 = fake quant only; one launch (the prologue is applied while the x row is staged)."""
    if mode not in (1, 2):
        raise ValueError(f"fp8_gemv_m1_pre: mode {mode} (1: rmsnorm + fake quant, 2: fake quant)")
    if mode == 1 and norm_w is None:
        raise ValueError("fp8_gemv_m1_pre: mode 1 needs norm_w")
    dev = require_gpu(x_raw, w8, s8)
    K = x_raw.shape[-1]
    N = w8.shape[0]
    xc = x_raw.reshape(-1).contiguous()
    if xc.dtype != torch.bfloat16:
        xc = xc.to(torch.bfloat16)
    if xc.data_ptr() % 16:
        xc = xc.clone()
    assert xc.numel() == K and w8.dtype == torch.uint8 and w8.is_contiguous() and s8.is_contiguous()
    wn = None
    if mode == 1:
        wn = norm_w.to(torch.bfloat16).contiguous()
        if wn.data_ptr() % 16:
            wn = wn.clone()
    direct = out is not None and out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == N
    y = out if direct else torch.empty(1, N, device=dev, dtype=torch.bfloat16)
    ws, n = _workspace(dev, 1, N, K)
    call("dsv41_fp8_gemv_m1_pre", ptr(xc), ptr(wn), float(eps), int(mode), ptr(w8), ptr(s8), N, K, s8.shape[1],
         ptr(y), ptr(ws), n, stream(dev))
    if out is not None and not direct:
        out.copy_(y.view_as(out))
    return out if out is not None else y
