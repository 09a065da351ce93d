from engine.cache.block_table import BlockTable
from engine.cache.kv_cache import KVCacheConfig, PagedKVCache, StepBatch, block_table_tensor, kv_append

__all__ = ["PagedKVCache", "BlockTable", "KVCacheConfig", "block_table_tensor", "kv_append", "StepBatch"]
