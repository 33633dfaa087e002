"""kvx: MI355X-native KV-block copy path (libkvx HIP kernels behind a C ABI).

Drop-ins for the reference package's copy path:
  kvx.ops.store_kvcache                     <- nanovllm.layers.attention.store_kvcache
  kvx.engine.cpu_prefix_cache.CPUBlockCache <- nanovllm.engine.cpu_prefix_cache.CPUBlockCache
  kvx.engine.kv_handoff                     <- nanovllm.engine.kv_handoff (plus an FP8 payload)
  kvx.ops                                   the operator API (codec, block lists, token copies, test hooks)
Callers of the copy path, with the reference's hook contract and signatures:
  kvx.engine.block_manager.BlockManager, kvx.engine.scheduler.Scheduler,
  kvx.engine.llm_engine.LLMEngine (model-free), kvx.engine.slot_mapping
"""

__version__ = "0.2.0"
