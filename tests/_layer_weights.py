"""Random weights of one attention layer (bf16-valued numpy arrays; the compressor's projections fp32) for the
layer-level parity tests: the reference's geometry at reduced widths."""
import numpy as np

from oracle import dsv41_oracle as O


def layer_weights(rng, dim, q_rank, H, D, HI, scale_sink=1.0):
    def w(n, k, s=None):
        return O.bf16(rng.standard_normal((n, k)).astype(np.float32) * (s if s is not None else k ** -0.5))
    return {
        "wq_a": w(q_rank, dim), "q_norm_w": O.bf16(rng.random(q_rank).astype(np.float32) + 0.5),
        "wq_b": w(H * D, q_rank), "wkv": w(D, dim), "kv_norm_w": O.bf16(rng.random(D).astype(np.float32) + 0.5),
        "attn_sink": (rng.standard_normal(H) * scale_sink).astype(np.float32),
        "c_wkv": (rng.standard_normal((D, dim)) * dim ** -0.5).astype(np.float32),
        "c_wgate": (rng.standard_normal((D, dim)) * dim ** -0.5).astype(np.float32),
        "c_norm_w": O.bf16(rng.random(D).astype(np.float32) + 0.5),
        "i_wq_b": w(HI * 128, q_rank), "i_weights_proj": w(HI, dim), "i_wk": w(128, D),
        "i_k_norm_w": O.bf16(rng.random(128).astype(np.float32) + 0.5),
    }
