"""Per-layer bit allocation hook of the cache (reference allocation/eval_alloc.py)."""
