"""aetherkv — MI355X-native (gfx950) compressed-KV hot path of Aether-2B decode.

Drop-in modules (same names and signatures as the reference):
  aetherkv.turbo_quant       <- aether_2b/turbo_quant.py        (_wht, PolarQuant)
  aetherkv.sparse_attention  <- aether_kernels/sparse_attention.py
  aetherkv.loader            <- aether_kernels/loader.py
  aetherkv.backends          <- aether_pipeline/serving.py backend protocol
New fused decode path over quantised KV:
  aetherkv.decode            csa_indexer_topk_quant, quant_sink_attention, csa_decode, hca_decode
  aetherkv.cache             the engine's cache state types and quant helpers (drop-in), and CodeRing:
                             preallocated code storage appended in place and read by csa_decode_ring /
                             hca_decode_ring
  aetherkv.storage           paged-allocator pages and prefix-cache files holding codes + scales
  aetherkv.attention_io      query prep, window entry and the output's inverse RoPE (one launch each)
                             and the grouped output projection
  aetherkv.prefill           chunked prefill through the quantised reader: every target of a chunk
                             scored and attended in one launch each (csa_prefill, hca_prefill)
All compute runs in libaetherkv.so (hand-written HIP for gfx950, C ABI in include/aetherkv.h).
"""
from .loader import cuda_build_environment, cuda_extension_unavailable_reason, load_aether_cuda_kernels
from .sparse_attention import csa_indexer_topk, hca_compress, sparse_sink_attention, tiled_prefill_attention
from .turbo_quant import PolarQuant, _wht

__all__ = [
    "PolarQuant",
    "_wht",
    "cuda_build_environment",
    "cuda_extension_unavailable_reason",
    "load_aether_cuda_kernels",
    "sparse_sink_attention",
    "tiled_prefill_attention",
    "csa_indexer_topk",
    "hca_compress",
]
