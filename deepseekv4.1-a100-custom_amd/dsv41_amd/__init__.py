"""dsv41_amd: MI355X-native (gfx950 HIP) implementation of DeepSeek-V4.1's sparse-attention path as the dsv41 runtime
runs it -- lightning indexer (score + top-k), sparse latent attention over the selected compressed rows plus the SWA
ring, the cache appends and the compressor pooling.  Python entry points keep the reference's call signatures (dsv41/fused.py,
dsv41/fused2.py, dsv41/fused3.py, dsv41/kernels.py); the compute is the C-ABI library libdsv41_hip.so."""
from .fused import (fake_quant, fake_quant_fp4, fake_quant_fp8, rmsnorm, rope_, rope_dev_, sparse_attn_decode,
                    sparse_attn_decode2, sparse_attn_decode_split)
from .fused2 import kv_write, sattn2
from .fused3 import index_score, topk_indices
from .kernels import sparse_attn
from .indexer import index_topk
from . import cache, compressor

__all__ = ["fake_quant", "fake_quant_fp4", "fake_quant_fp8", "rmsnorm", "rope_", "rope_dev_", "sparse_attn_decode",
           "sparse_attn_decode2", "sparse_attn_decode_split", "kv_write", "sattn2", "index_score", "topk_indices",
           "sparse_attn", "index_topk", "cache", "compressor"]
