"""MI355X-native paged KV-cache hot path behind PagedCore's allocator/attention API.

Modules:
  engine_types  request/block ids, KVReservation, CapacityCounts (boundary records)
  config        pool-sizing configuration
  kv_cache      allocate_kv_pool, KVAllocator (LIFO blocks, staged decode, block gather)
  attention     paged_attention / paged_attention_batch on the HIP kernels
  _hip          ctypes binding of libpagedcore_hip.so (include/pagedcore_hip.h)
"""
