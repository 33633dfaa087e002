"""kvx: MI355X-native KV-block copy path (libkvx HIP kernels behind a C ABI).

Module layout mirrors the reference package it drops into:
  kvx.layers.attention.store_kvcache        <- nanovllm.layers.attention.store_kvcache
  kvx.engine.cpu_prefix_cache.CPUBlockCache <- nanovllm.engine.cpu_prefix_cache.CPUBlockCache
  kvx.engine.block_manager.BlockManager     <- nanovllm.engine.block_manager.BlockManager
  kvx.ops                                   the operator API (codec, block lists, test hooks)
"""

__version__ = "0.1.0"
