"""Slot mappings for store_kvcache: where each token of a step writes its K/V in the pool.

Slot s addresses row s of a layer's [num_blocks * block_size, H * hd] cache
view: block_table[position // block_size] * block_size + position % block_size
(nanovllm/engine/model_runner.py:156-166 for prefill, :186 for decode; -1
pads a captured graph's batch, :211). The producers build int32 numpy
arrays with vectorised arithmetic (a 65K-token prefill is one pass, not a
Python loop per token); `upload` moves one to the device without waiting
for the GPU, as the reference's runner does with a pinned host copy and a
non-blocking host-to-device copy (:173, 189). Here a kernel on the current
stream reads the pinned copy (kvx.ops.upload): a DMA copy there would queue
behind the restore stream's bulk host-to-device copies, delaying the step by
as long as the restores in flight take.
"""

import numpy as np
import torch


def prefill_slot_mapping(seqs, block_size: int) -> np.ndarray:
    """Slots of every scheduled prefill token, request after request (requests without blocks add none)."""
    parts = []
    for seq in seqs:
        if not seq.block_table or not seq.num_scheduled_tokens:
            continue
        positions = np.arange(seq.num_cached_tokens, seq.num_cached_tokens + seq.num_scheduled_tokens,
                              dtype=np.int64)
        table = np.asarray(seq.block_table, dtype=np.int64)
        parts.append(table[positions // block_size] * block_size + positions % block_size)
    if not parts:
        return np.empty(0, dtype=np.int32)
    return np.concatenate(parts).astype(np.int32)


def decode_slot_mapping(seqs, block_size: int, padded_to: int | None = None) -> np.ndarray:
    """The slot of each request's newest token; with padded_to, -1 fills the batch to that size."""
    n = len(seqs) if padded_to is None else padded_to
    if n < len(seqs):
        raise ValueError("padded_to is smaller than the batch")
    slots = np.full(n, -1, dtype=np.int32)
    for i, seq in enumerate(seqs):
        slots[i] = seq.block_table[-1] * block_size + seq.last_block_num_tokens - 1
    return slots


def upload(values: np.ndarray, device: torch.device) -> torch.Tensor:
    """A device copy of a host array, read from pinned memory by a kernel on the current stream."""
    from kvx import ops

    return ops.upload(values, device)
