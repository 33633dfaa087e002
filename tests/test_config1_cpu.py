"""Config 1 on the CPU: the reference's own CPU path (its torch codec on a CPU pool) against the C oracle.

Qwen3-0.6B block geometry [2, 28, *, 256, 8, 128] bf16 ~ N(0, 1); 16 seeded blocks are saved to FP8 (fp32
scales) and restored into 16 other seeded blocks, as nanovllm/engine/cpu_prefix_cache.py:323-326, 394-397 do for
a CPU pool. The pool holds 40 blocks instead of 512 (the per-block work is identical; 40 keeps host memory small).
"""

import numpy as np
import torch

from helpers import bf16_bits
from workloads import block_selection
from oracle import kvx_oracle as oracle
from oracle import torch_path


def test_reference_cpu_path_matches_the_oracle_on_16_qwen3_0_6b_blocks():
    g = torch.Generator().manual_seed(0)
    pool = torch.randn((2, 28, 40, 256, 8, 128), generator=g).to(torch.bfloat16)
    order = block_selection(40, 32, seed=1)
    sources, dests = order[:16], order[16:]
    before = bf16_bits(pool)
    shape = (2, 28, 256, 8, 128)
    for src, dst in zip(sources, dests):
        payload = torch.empty(shape, dtype=torch.float8_e4m3fn)
        scale = torch.empty((*shape[:-1], 1), dtype=torch.float32)
        torch_path.save_block(pool, src, payload, scale)
        codes, scales = oracle.save_block_fp8(before, src, True)
        assert np.array_equal(payload.view(torch.uint8).numpy(), codes)
        assert np.array_equal(scale.numpy(), scales)
        torch_path.restore_block(pool, dst, payload, scale)
        assert np.array_equal(bf16_bits(pool[:, :, dst]), oracle.dequantize(codes, scales, True))
        source = torch.from_numpy(before[:, :, src].view(np.int16)).view(torch.bfloat16).float()
        restored = pool[:, :, dst].float()
        assert torch.all((restored - source).abs() <= source.abs().amax(-1, keepdim=True) / 16)
