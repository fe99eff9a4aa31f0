"""KV-cache integration: CompressedKVCache and the fused merge paths."""
