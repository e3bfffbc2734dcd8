"""mitten_amd — MI355X-native paged-KV hot path of the mitten inference engine.

Device side (libmitten_kv.so, hand-written gfx950 HIP):
    DeviceKvPool      the device KV pool and its operations (append, gather,
                      copy_blocks, decode_attention, extend_attention, and
                      qk_norm_rope_append, the fused norm + RoPE + append
                      step before attention)
Host side (libmitten_kvhost.so, C++):
    KvCachePool, PageTable, RadixCache, BlockManager
                      the engine's page allocator, radix prefix cache and
                      block-table bookkeeping (inference-engine/src/*.rs)
"""
from .device_pool import (  # noqa: F401
    BackendError,
    DeviceIndexError,
    DeviceKvPool,
    EngineError,
    OutOfKvPages,
    PoolDesc,
    required_bytes,
    rope_inv_freq,
    validate_block_tables,
    validate_copy_pairs,
    validate_slots,
)

__version__ = "0.1.0"
