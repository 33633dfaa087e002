"""Plane ranges of the token copies and the handoff's plane groups (CPU only: layout arithmetic, no copies)."""

import pytest
import torch

from kvx import ops
from kvx.engine import kv_handoff

QWEN3_8B = (2, 36, 320, 256, 8, 128)


def test_a_plane_range_is_the_pool_layout_with_fewer_planes_from_the_first_ones_address():
    pool = torch.empty((2, 3, 5, 16, 2, 8), dtype=torch.bfloat16)
    layout = ops.pool_layout(pool)
    address, sub, lead = ops._plane_range(pool, layout, (1, 4))
    assert address == pool.data_ptr() + 1 * 5 * 16 * 2 * 8 * 2 == pool[0, 1].data_ptr()
    assert (sub.planes, lead) == (3, (3,))
    for name, _ in ops.BlockLayout._fields_:
        if name != "planes":
            assert getattr(sub, name) == getattr(layout, name)
    assert ops._plane_range(pool, layout, None) == (pool.data_ptr(), layout, (2, 3))
    # Plane 3 (V, layer 0) starts at pool[1, 0].
    assert ops._plane_range(pool, layout, (3, 6))[0] == pool[1, 0].data_ptr()


@pytest.mark.parametrize("planes", [(0, 0), (3, 2), (-1, 2), (0, 7), (6, 7)])
def test_plane_ranges_outside_the_pool_are_refused(planes):
    pool = torch.empty((2, 3, 5, 16, 2, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="plane range"):
        ops._plane_range(pool, ops.pool_layout(pool), planes)


@pytest.mark.parametrize("kv_dtype,scale_dtype,group", [(torch.bfloat16, None, 4),
                                                         (torch.float8_e4m3fn, torch.float32, 7),
                                                         (torch.float8_e4m3fn, torch.bfloat16, 7)])
def test_plane_groups_cover_every_plane_once_within_the_staging(kv_dtype, scale_dtype, group):
    pool = torch.empty(QWEN3_8B, dtype=torch.bfloat16, device="meta")
    groups = kv_handoff._plane_groups(pool, 32767, kv_dtype, scale_dtype)
    assert groups[0] == (0, group) and groups[-1][1] == 72
    assert [p for first, end in groups for p in range(first, end)] == list(range(72))
    row = 128 * kv_dtype.itemsize + (scale_dtype.itemsize if scale_dtype else 0)
    assert all((end - first) * 32767 * 8 * row <= kv_handoff._STAGING_BYTES for first, end in groups)


def test_a_plane_larger_than_the_staging_still_moves_alone():
    pool = torch.empty(QWEN3_8B, dtype=torch.bfloat16, device="meta")
    groups = kv_handoff._plane_groups(pool, 1 << 20, torch.bfloat16, None)  # 2 GiB planes
    assert groups == [(p, p + 1) for p in range(72)]
