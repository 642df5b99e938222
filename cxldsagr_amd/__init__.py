"""MI355X-native DeepSeek-V3.2 sparse-attention (DSA) prefill path.

Host operators mirror the reference's operator API; every operator launches
hand-written gfx950 kernels from libdsa_gfx950.so (see include/dsa_gfx950.h).
"""

__all__ = ["attention", "contracts", "indexer", "kv_transfer", "layer", "ops", "token_pool"]
