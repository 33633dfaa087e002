"""Shared test helpers: bit-pattern conversions and seeded inputs."""

import numpy as np
import torch


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16 tensor (copied to the host)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_tensor(bits: np.ndarray, device=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    return t if device is None else t.to(device)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def scale_bits(t: torch.Tensor) -> np.ndarray:
    """Scale tensor as raw bytes (fp32 or bf16), for bit-exact comparison."""
    return u8(t)


def finite_bf16_rows(rows: int, hd: int, seed: int) -> np.ndarray:
    """Finite bf16 bit patterns covering every exponent, both signs and subnormals.

    Half of the rows are confined to a random exponent window so the row amax
    does not dominate every element.
    """
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 16, size=(rows, hd), dtype=np.uint32).astype(np.uint16)
    narrow = rng.random(rows) < 0.5
    window = rng.integers(0x0080, 0x7E00, size=rows).astype(np.uint32)
    low = (bits.astype(np.uint32) & 0x807F) | ((window[:, None] + (bits.astype(np.uint32) & 0x0380)) & 0x7F80)
    bits[narrow] = low[narrow].astype(np.uint16)
    bits[(bits & 0x7F80) == 0x7F80] &= 0xBFFF  # fold inf/NaN patterns into finite ones
    return bits


def student_t_rows(rows: int, hd: int, seed: int, outliers: int = 4) -> np.ndarray:
    """bf16 bits of 0.5 * t(df=4) rows with `outliers` channels scaled by 20."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn((rows, hd), generator=g) / torch.randn((rows, hd, 4), generator=g).square().mean(-1).sqrt()
    t = t * 0.5
    t[:, :outliers] *= 20
    return bf16_bits(t.to(torch.bfloat16))
