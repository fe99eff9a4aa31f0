"""KV-cache integration: CompressedKVCache (HF Cache), fixed-rate merge paths, decode attention."""
