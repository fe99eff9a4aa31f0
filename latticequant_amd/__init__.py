"""LatticeQuant compressed-KV hot path for AMD Instinct MI355X (gfx950).

E8 lattice quantisation, bit-wise rANS coding, dequantisation and the fused
merge / decode-attention step, as hand-written HIP kernels behind a C ABI
(liblatticequant_amd.so).  Host code mirrors the reference's Python modules:

  latticequant_amd.core.e8_quantizer       (core/e8_quantizer.py)
  latticequant_amd.core.entropy_coder      (core/entropy_coder.py)
  latticequant_amd.core.compact_storage    (core/compact_storage.py)
  latticequant_amd.core.gpu_ans            (core/gpu_ans.py)
  latticequant_amd.core.triton_dequant     (core/triton_dequant.py)
  latticequant_amd.core.pipeline           (core/pipeline.py, RHT)
  latticequant_amd.llm.compressed_kv_cache (llm/compressed_kv_cache.py)
  latticequant_amd.llm.fused_triton_merge  (llm/fused_triton_merge.py)
  latticequant_amd.llm.triton_kv_integration (llm/triton_kv_integration.py)
  latticequant_amd.llm.decode_attention     (decode step over the compressed prefix)
"""
__version__ = "0.1.0"
