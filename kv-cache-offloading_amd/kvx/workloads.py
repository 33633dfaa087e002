"""Seeded synthetic KV pools and block selections for benchmarks and tests.

Shapes follow the pool layout [2, L, NB, BS, H, hd] (nanovllm/engine/model_runner.py:120).
Values are generated on the pool's device, one (K/V, layer) plane at a time,
with a torch.Generator seeded per plane so any plane can be regenerated.
"""

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class PoolShape:
    layers: int
    num_blocks: int
    block_size: int = 256
    kv_heads: int = 8
    head_dim: int = 128

    @property
    def shape(self) -> tuple[int, ...]:
        return (2, self.layers, self.num_blocks, self.block_size, self.kv_heads, self.head_dim)

    @property
    def block_elems(self) -> int:
        return 2 * self.layers * self.block_size * self.kv_heads * self.head_dim

    @property
    def block_bytes_bf16(self) -> int:
        return 2 * self.block_elems

    @property
    def rows_per_block(self) -> int:
        return 2 * self.layers * self.block_size * self.kv_heads


# Qwen3 KV geometry (8 KV heads, head_dim 128, 256-token blocks).
QWEN3_8B = PoolShape(layers=36, num_blocks=320)
QWEN3_0_6B = PoolShape(layers=28, num_blocks=512)


def _plane_generator(device, seed: int, kv: int, layer: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed((seed * 1_000_003 + kv * 4099 + layer) & 0x7FFFFFFFFFFFFFFF)
    return g


def fill_normal(pool: torch.Tensor, seed: int = 0):
    """pool <- bf16(N(0, 1)), plane by plane."""
    for kv in range(2):
        for layer in range(pool.shape[1]):
            g = _plane_generator(pool.device, seed, kv, layer)
            plane = pool[kv, layer]
            plane.copy_(torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32))
    return pool


def fill_student_t(pool: torch.Tensor, seed: int = 0, df: int = 4, scale: float = 0.5,
                   outlier_channels: int = 4, outlier_gain: float = 20.0):
    """pool <- bf16(scale * t_df) with `outlier_channels` seeded channels per (K/V, layer, head) x gain.

    t_df = z / sqrt(chi2_df / df) with chi2_df a sum of df squared normals.
    """
    heads, hd = pool.shape[4], pool.shape[5]
    for kv in range(2):
        for layer in range(pool.shape[1]):
            g = _plane_generator(pool.device, seed, kv, layer)
            plane = pool[kv, layer]
            z = torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32)
            chi2 = torch.zeros_like(z)
            for _ in range(df):
                chi2.add_(torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32).square_())
            t = z.div_(chi2.div_(df).sqrt_()).mul_(scale)
            del chi2
            gain = torch.ones((heads, hd), device=pool.device, dtype=torch.float32)
            for h in range(heads):
                channels = torch.randperm(hd, generator=g, device=pool.device)[:outlier_channels]
                gain[h, channels] = outlier_gain
            plane.copy_(t.mul_(gain))
    return pool


def block_selection(num_blocks: int, count: int, seed: int, exclude=()) -> list[int]:
    """`count` distinct seeded block ids from [0, num_blocks) minus `exclude`."""
    g = torch.Generator().manual_seed(seed)
    excluded = set(exclude)
    order = [b for b in torch.randperm(num_blocks, generator=g).tolist() if b not in excluded]
    if count > len(order):
        raise ValueError(f"cannot pick {count} of {len(order)} blocks")
    return order[:count]
