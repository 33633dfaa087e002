"""Writes fp8_codec.npz: FP8 codec fixtures computed by torch's CPU kernels.

Inputs are seeded bf16 rows plus hand-built edge rows; expected outputs come
from the reference's four codec calls (nanovllm/engine/cpu_prefix_cache.py:20-28)
run with torch on the CPU (oracle/torch_path.py), i.e. from torch's own
division, bf16 and float8_e4m3fn conversion routines. Tests compare both
kvx_oracle.c and the HIP kernels against these arrays.

Run from the repository root: python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import torch_path  # noqa: E402

OUT = Path(__file__).resolve().with_name("fp8_codec.npz")


def edge_rows(hd: int) -> torch.Tensor:
    """Rows whose codes exercise clamping, ties, subnormals and the scale floor."""
    rows = []
    r = torch.zeros(hd)
    rows.append(r.clone())                                   # all zero: scale = 1e-30
    r = torch.zeros(hd); r[hd // 2] = -3.0; rows.append(r)   # single value: -> -448
    # amax 448 -> scale exactly 1: ties between e4m3 neighbours round to even.
    specials = [448.0, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -(2.0 ** -10), 232.0, 0.0, -0.0]
    r = torch.full((max(hd, len(specials)),), 1.0625)
    r[:len(specials)] = torch.tensor(specials)
    rows.append(r[:hd] if hd >= len(specials) else torch.tensor([448.0, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10]))
    r = torch.linspace(-1e-30, 1e-30, hd); rows.append(r)    # amax below 448e-30: scale floor
    r = torch.linspace(-1e38, 1e38, hd); rows.append(r)      # huge magnitudes
    r = torch.full((hd,), -3.3895313892515355e38); r[-1] = 1.0; rows.append(r)  # bf16 max (0xFF7F)
    r = torch.full((hd,), 1e-38); r[0] = 2.0 ** -133; rows.append(r)  # bf16 subnormals
    return torch.stack(rows)


def main():
    g = torch.Generator().manual_seed(20261201)
    out = {}
    for hd, n_random in ((128, 48), (64, 16), (256, 8), (4, 16)):
        normal = torch.randn((n_random // 2, hd), generator=g)
        t = torch.randn((n_random - n_random // 2, hd), generator=g) / (
            torch.randn((n_random - n_random // 2, hd, 4), generator=g).square().mean(-1).sqrt()) * 0.5
        t[:, : max(1, hd // 32)] *= 20.0
        rows = torch.cat([normal, t, edge_rows(hd)]).to(torch.bfloat16)
        out[f"x_hd{hd}"] = rows.view(torch.int16).numpy().view(np.uint16)
        for name, dtype in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
            payload = torch.empty(rows.shape, dtype=torch.float8_e4m3fn)
            scale = torch.empty((rows.shape[0], 1), dtype=dtype)
            torch_path.fp8_quantize(rows, payload, scale)
            back = torch.empty_like(rows)
            torch_path.fp8_dequantize(payload, scale, back)
            out[f"codes_hd{hd}_{name}"] = payload.view(torch.uint8).numpy()
            out[f"scale_hd{hd}_{name}"] = (scale.numpy() if dtype == torch.float32
                                           else scale.view(torch.int16).numpy().view(np.uint16))
            out[f"back_hd{hd}_{name}"] = back.view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
