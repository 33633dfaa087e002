"""kvx: MI355X-native KV-block copy path (libkvx HIP kernels behind a C ABI).

Module layout mirrors the reference package it drops into:
  kvx.layers.attention.store_kvcache        <- nanovllm.layers.attention.store_kvcache
  kvx.engine.cpu_prefix_cache.CPUBlockCache <- nanovllm.engine.cpu_prefix_cache.CPUBlockCache
  kvx.engine.block_manager.BlockManager     <- nanovllm.engine.block_manager.BlockManager
  kvx.engine.scheduler.Scheduler            <- nanovllm.engine.scheduler.Scheduler
  kvx.engine.llm_engine.LLMEngine           <- nanovllm.engine.llm_engine.LLMEngine (model-free)
  kvx.engine.kv_handoff                     <- nanovllm.engine.kv_handoff
  kvx.engine.handoff_timing                 <- nanovllm.engine.handoff_timing
  kvx.ops                                   the operator API (codec, block lists, test hooks)
"""

__version__ = "0.1.0"
