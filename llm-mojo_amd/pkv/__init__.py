"""pkv -- MI355X-native paged KV-cache attention (host side over libpkv.so)."""
from .engine import (BF16, F32, LayerSpec, LSABucketCache, PagedKVCache,
                     attention_window_start, lsa_expand_buckets, make_params, paged_attention_layer, q4_matmul,
                     ring_row)
from .lib import PkvError, load

__all__ = [
    "BF16", "F32", "LayerSpec", "LSABucketCache", "PagedKVCache", "PkvError", "attention_window_start", "load",
    "lsa_expand_buckets", "make_params", "paged_attention_layer", "q4_matmul", "ring_row",
]
