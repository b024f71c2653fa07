"""Seeded synthetic workloads of the benchmark configurations (random data of the real shapes; no checkpoint).

C1  CPU plumbing: 1 slot, ctx 4096, ratio 4 -> 1024 compressed rows x 576 bf16, k 512, W 128, 64 x 128 indexer.
C2  decode: 4 slots x 131072 ctx -> 32768 compressed rows per slot, k 2048 (the headline decode config).
C3  chunked prefill: 2048 queries after 65536 prior tokens (16384 + own compressed rows), k 2048.
C4  long-context decode: 1 slot x 1048576 ctx -> 262144 compressed rows, k 2048.
C5  ragged batched decode + speculative verify: 8 slots x 6 query rows.

All values N(0,1)*0.1 from torch.Generator seeds (CPU, then copied to the device); index keys and index queries are
FP4-rounded per 32 like the reference stores them (dsv41/model.py:726, :738) and carry a few x8 outlier channels;
the index-key table is kept as e4m3 + per-row fp32 scale.  The BASELINE configs use absorbed-MLA rows (576 = 512
latent + 64 rope, V = latent), 64 index heads and ratio 4; the reference geometry (head_dim 512 with in-row rope,
32 index heads, ratio 2, top-k 512) is built by the parity tests of tests/test_gpu_coverage.py themselves."""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

H, DQK, DV, HI, DI, WIN = 64, 576, 512, 64, 128, 128
OUTLIER_CH = (3, 40, 77, 120)


@dataclass
class DecodeConfig:
    name: str
    ctx: list                     # context length (tokens) per slot
    rows_per_slot: int = 1        # query rows per slot (1 + MTP drafts)
    ratio: int = 4
    topk: int = 2048
    spare: int = 1                # spare capacity rows (the reference's dummy row)
    extra: dict = field(default_factory=dict)

    @property
    def slots(self):
        return len(self.ctx)

    def n_c(self, s):
        return self.ctx[s] // self.ratio


CONFIGS = {
    "C1": DecodeConfig("C1", [4096], topk=512),
    "C2": DecodeConfig("C2", [131072] * 4),
    "C4": DecodeConfig("C4", [1048576]),
    "C5": DecodeConfig("C5", [524288, 131072, 131072, 131072, 65536, 32768, 8192, 2048], rows_per_slot=6),
}


def fp4_round(x: torch.Tensor, block: int = 32) -> torch.Tensor:
    """E2M1 values with a power-of-two scale per `block` (the reference's fake_quant_fp4, dsv41/quant.py:75-87),
    torch on any device; used only to synthesise inputs."""
    shp = x.shape
    g = x.float().reshape(-1, block)
    amax = g.abs().amax(-1, keepdim=True).clamp_min(6 * 2.0 ** -126)
    m, e = torch.frexp(amax / 6.0)
    s = torch.exp2((e - (m == 0.5).to(e.dtype)).float())
    v = (g / s).clamp(-6, 6)
    a = v.abs()
    r = torch.where(a < 2, torch.round(a * 2) / 2, torch.where(a < 4, torch.round(a), torch.round(a / 2) * 2))
    return (torch.copysign(r.clamp(max=6), v) * s).reshape(shp).to(torch.bfloat16)


def encode_e4m3_rows(k: torch.Tensor):
    """bf16 rows -> (float8_e4m3fn rows, fp32 per-row pow2 scale): exact for FP4-grid rows."""
    kf = k.float()
    amax = kf.abs().amax(-1, keepdim=True).clamp_min(1e-30)
    m, e = torch.frexp(amax / 448.0)
    s = torch.exp2((e - (m == 0.5).to(e.dtype)).float().clamp_min(-126))
    q = (kf / s).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q, s[..., 0]


def _randn(g, *shape, scale=0.1):
    return torch.randn(*shape, generator=g) * scale


def make_decode_inputs(cfg: DecodeConfig, device, seed: int = 0, cache_copies: int = 1):
    """Caches (cache_copies independent copies, to rotate past the 256 MB last-level cache) and per-step inputs."""
    g = torch.Generator().manual_seed(seed)
    S = cfg.slots
    cap = max(cfg.n_c(s) for s in range(S)) + cfg.spare
    R = S * cfg.rows_per_slot
    layers = []
    for c in range(cache_copies):
        ckv = torch.empty(S, cap, DQK, dtype=torch.bfloat16, device=device)
        k8 = torch.empty(S, cap, DI, dtype=torch.float8_e4m3fn, device=device)
        ks = torch.empty(S, cap, dtype=torch.float32, device=device)
        for s in range(S):
            gs = torch.Generator(device=device).manual_seed(seed * 1000 + c * 64 + s) if device != "cpu" else g
            n = cap
            ckv[s] = (torch.randn(n, DQK, generator=gs, device=device) * 0.1).to(torch.bfloat16)
            kk = torch.randn(n, DI, generator=gs, device=device) * 0.1
            kk[:, list(OUTLIER_CH)] *= 8
            q8, sc = encode_e4m3_rows(fp4_round(kk))
            k8[s] = q8
            ks[s] = sc
        ring = (_randn(g, S, WIN, DQK)).to(torch.bfloat16).to(device)
        layers.append(dict(ckv=ckv, k8=k8, ks=ks, ring=ring))
    pos, seq, pmax = [], [], []
    for s in range(S):
        for j in range(cfg.rows_per_slot):
            pos.append(cfg.ctx[s] - cfg.rows_per_slot + j)
            seq.append(s)
            pmax.append(cfg.ctx[s] - 1)
    step = dict(
        q=_randn(g, R, 1, H, DQK).to(torch.bfloat16).to(device),
        q_idx=fp4_round(_randn(g, R, 1, HI, DI, scale=1.0)).to(device),
        w_idx=(_randn(g, R, HI) * (DI ** -0.5 * HI ** -0.5)).to(torch.bfloat16).to(device),
        kv_raw=_randn(g, R, DQK, scale=1.0).to(torch.bfloat16).to(device),
        latent=_randn(g, R, 1, DQK, scale=1.0).to(torch.bfloat16).to(device),
        k_raw=_randn(g, R, DI, scale=1.0).to(torch.bfloat16).to(device),
        kv_norm=(torch.rand(DQK, generator=g) + 0.5).to(torch.bfloat16).to(device),
        k_norm=(torch.rand(DI, generator=g) + 0.5).to(torch.bfloat16).to(device),
        sink=_randn(g, H, scale=1.0).to(device),
        pos=torch.tensor(pos, dtype=torch.int64, device=device),
        seq=torch.tensor(seq, dtype=torch.int64, device=device),
        pmax=torch.tensor(pmax, dtype=torch.int64, device=device),
    )
    return layers, step


@dataclass
class PrefillConfig:
    name: str = "C3"
    chunk: int = 2048        # query tokens in the chunk
    prior: int = 65536       # tokens before the chunk
    ratio: int = 4
    topk: int = 2048
    extra: dict = field(default_factory=dict)

    @property
    def end(self):
        return self.prior + self.chunk

    @property
    def n_c(self):  # compressed rows visible to the last query
        return self.end // self.ratio


PREFILL = {"C3": PrefillConfig()}


def make_prefill_inputs(cfg: PrefillConfig, device, seed: int = 1):
    """One layer's chunked-prefill inputs: queries, index queries/weights, the compressed-KV table and e4m3 index keys
    covering the prior context plus the chunk's own groups, the SWA history + chunk rows, and the per-query index
    lists in the reference's layout (window indices into [history | chunk] followed by compressed indices + offset,
    dsv41/model.py:1442-1443)."""
    g = torch.Generator(device=device).manual_seed(seed)
    S, T = cfg.chunk, cfg.n_c
    hist = min(cfg.prior, WIN - 1)
    q = (torch.randn(1, S, H, DQK, generator=g, device=device) * 0.1).to(torch.bfloat16)
    q_idx = fp4_round(torch.randn(1, S, HI, DI, generator=g, device=device))
    w_idx = (torch.randn(1, S, HI, generator=g, device=device) * (DI ** -0.5 * HI ** -0.5)).to(torch.bfloat16)
    kk = torch.randn(1, T, DI, generator=g, device=device) * 0.1
    kk[..., list(OUTLIER_CH)] *= 8
    kbf = fp4_round(kk)
    k8, ks = encode_e4m3_rows(kbf)
    ckv = (torch.randn(1, T, DQK, generator=g, device=device) * 0.1).to(torch.bfloat16)
    win = (torch.randn(1, hist + S, DQK, generator=g, device=device) * 0.1).to(torch.bfloat16)
    qq = hist + torch.arange(S, device=device).unsqueeze(1)
    widx = (qq - WIN + 1).clamp_min(0) + torch.arange(WIN, device=device).unsqueeze(0)
    widx = torch.where(widx <= qq, widx, -1).to(torch.int32).unsqueeze(0)
    return dict(q=q, q_idx=q_idx, w_idx=w_idx, kbf=kbf, k8=k8, ks=ks, ckv=ckv, win=win, widx=widx, hist=hist)
