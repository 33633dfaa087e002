"""The reference's CPU copy path, expressed with the torch operations it uses.

TEST INFRASTRUCTURE ONLY: bench.py times it as the CPU baseline and
tests/golden/make_golden.py uses it to write fixtures from torch's own
conversion routines (independent of kvx_oracle.c's table search).

When CPUBlockCache's pool lives on the CPU, the reference saves a block with
fp8_quantize (or a byte copy) straight into its slab slot and restores with
fp8_dequantize (or a byte copy) straight into the pool
(nanovllm/engine/cpu_prefix_cache.py:323-326, 394-397). The codec is four
torch calls (:20-28); they are repeated here in the same order with the same
dtypes, because bit-exactness is defined by that sequence of roundings.
"""

import torch

FP8_MAX = 448.0


def fp8_quantize(source: torch.Tensor, payload: torch.Tensor, scale: torch.Tensor):
    """cpu_prefix_cache.py:20-24: per-row scale in scale's dtype, then e4m3fn payload."""
    row_max = source.abs().amax(-1, keepdim=True).float()
    scale.copy_((row_max / FP8_MAX).clamp_min(1e-30))
    payload.copy_((source.float() / scale.float()).clamp_(-FP8_MAX, FP8_MAX))


def fp8_dequantize(payload: torch.Tensor, scale: torch.Tensor, target: torch.Tensor):
    """cpu_prefix_cache.py:27-28."""
    torch.mul(payload.to(target.dtype), scale, out=target)


def save_block(pool: torch.Tensor, block_id: int, payload: torch.Tensor, scale: torch.Tensor | None):
    """One CPU-pool save (cpu_prefix_cache.py:323-326)."""
    source = pool[:, :, block_id]
    if scale is not None:
        fp8_quantize(source, payload, scale)
    else:
        payload.copy_(source)


def restore_block(pool: torch.Tensor, block_id: int, payload: torch.Tensor, scale: torch.Tensor | None):
    """One CPU-pool restore (cpu_prefix_cache.py:394-397)."""
    target = pool[:, :, block_id]
    if scale is not None:
        fp8_dequantize(payload, scale, target)
    else:
        target.copy_(payload)
