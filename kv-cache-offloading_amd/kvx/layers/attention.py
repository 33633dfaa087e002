"""The paged KV write a model's attention layer calls each step.

store_kvcache is the drop-in for nanovllm/layers/attention.py:33-40 (the
Triton store_kvcache_kernel at :10-30 becomes libkvx's HIP kernel).
"""

from kvx.ops import store_kvcache

__all__ = ["store_kvcache"]
