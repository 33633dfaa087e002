"""kvx_upload: a step's inputs copied from pinned host memory by a kernel on the caller's stream.

The copy is byte-exact for any size and alignment; sources that are not one
pinned allocation covering the whole range are refused before any launch;
uploads queued faster than the stream runs reuse their pinned buffers only
after the kernel that read them has run; and an upload does not wait behind
host-to-device DMA queued on another stream.
"""

import ctypes

import numpy as np
import pytest
import torch

from kvx import _lib, ops
from kvx._lib import check, lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.uint8, np.float32])
@pytest.mark.parametrize("count", [1, 3, 16, 17, 4099, 1 << 18])
def test_upload_copies_every_byte(gpu, dtype, count):
    rng = np.random.default_rng(count)
    host = rng.integers(-2**31, 2**31 - 1, size=count, dtype=np.int64).astype(dtype)
    print(f"upload {count} x {np.dtype(dtype).name}", flush=True)
    got = ops.upload(host, gpu)
    assert got.device == gpu and got.shape == host.shape
    assert np.array_equal(got.cpu().numpy().view(np.uint8), host.view(np.uint8))


@pytest.mark.parametrize("src_offset,dst_offset,nbytes", [(1, 0, 100), (0, 3, 64), (7, 5, 1000), (16, 16, 33)])
def test_upload_of_unaligned_ranges_through_the_c_abi(gpu, src_offset, dst_offset, nbytes):
    src = torch.arange(4096, dtype=torch.int32).view(torch.uint8).pin_memory()
    dst = torch.full((8192,), 0x5A, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    check(lib().kvx_upload(dst.data_ptr() + dst_offset, src.data_ptr() + src_offset, nbytes, stream), "upload")
    out = dst.cpu().numpy()
    assert np.array_equal(out[dst_offset:dst_offset + nbytes], src.numpy()[src_offset:src_offset + nbytes])
    assert np.all(out[:dst_offset] == 0x5A) and np.all(out[dst_offset + nbytes:] == 0x5A)


def test_upload_refuses_sources_that_are_not_one_pinned_allocation(gpu):
    dst = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    pageable = np.arange(1024, dtype=np.uint8)
    with pytest.raises(ValueError, match="pinned"):
        check(lib().kvx_upload(dst.data_ptr(), pageable.ctypes.data, pageable.nbytes, stream), "upload")
    with pytest.raises(ValueError, match="pinned"):
        check(lib().kvx_upload(dst.data_ptr(), dst.data_ptr(), 1024, stream), "upload")  # device memory
    small = torch.zeros(4096, dtype=torch.uint8).pin_memory()
    with pytest.raises(ValueError):
        check(lib().kvx_upload(dst.data_ptr(), small.data_ptr(), 512 << 20, stream), "upload")  # runs past it
    with pytest.raises(IndexError, match="largest upload"):
        check(lib().kvx_upload(dst.data_ptr(), small.data_ptr(), _lib.UPLOAD_MAX_BYTES + 1, stream), "upload")
    with pytest.raises(ValueError, match="negative"):
        check(lib().kvx_upload(dst.data_ptr(), small.data_ptr(), -1, stream), "upload")
    torch.cuda.synchronize(gpu)
    assert int(dst.count_nonzero()) == 0


def test_uploads_queued_behind_a_busy_stream_keep_their_bytes(gpu):
    """More uploads than pinned buffers while the stream is held: each buffer is rewritten only after its
    reader ran, so every result holds its own array."""
    ops.sleep(20_000, device=gpu)  # 20 ms on the current stream
    arrays = [np.full(1000 + i, i, dtype=np.int32) for i in range(40)]
    outs = [ops.upload(a, gpu) for a in arrays]
    for a, out in zip(arrays, outs):
        assert np.array_equal(out.cpu().numpy(), a)


def test_upload_into_a_given_tensor(gpu):
    out = torch.zeros(300, dtype=torch.int64, device=gpu)
    host = np.arange(300, dtype=np.int64) * 3
    assert ops.upload(host, gpu, out=out) is out
    assert np.array_equal(out.cpu().numpy(), host)
    with pytest.raises(ValueError, match="out must be"):
        ops.upload(host.astype(np.int32), gpu, out=out)


def test_upload_does_not_wait_for_dma_queued_on_another_stream(gpu):
    """Every buffer exists before the DMA is queued, so no allocation can hold the host back. The DMA's stream
    is chosen as the copy engine chooses its streams: one that runs beside the current stream (two streams on
    one hardware queue run in queue order, whatever they hold)."""
    from kvx.engine.cpu_prefix_cache import _copy_streams

    nbytes = 1 << 30
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dev = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    (other,), concurrent = _copy_streams(gpu, 1)
    assert concurrent
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    slots = torch.arange(65536, dtype=torch.int32).pin_memory()
    got = torch.zeros(65536, dtype=torch.int32, device=gpu)
    current = torch.cuda.current_stream(gpu)
    torch.cuda.synchronize(gpu)
    start = torch.cuda.Event(enable_timing=True)
    dma_done = torch.cuda.Event(enable_timing=True)
    upload_done = torch.cuda.Event(enable_timing=True)
    start.record(other)
    for off in range(0, nbytes, 64 << 20):
        assert hip.hipMemcpyAsync(dev.data_ptr() + off, host.data_ptr() + off, 64 << 20, 1, other.cuda_stream) == 0
    dma_done.record(other)
    check(lib().kvx_upload(got.data_ptr(), slots.data_ptr(), 65536 * 4, current.cuda_stream), "upload")
    upload_done.record(current)
    torch.cuda.synchronize(gpu)
    assert torch.equal(got.cpu(), slots)
    dma_ms, upload_ms = start.elapsed_time(dma_done), start.elapsed_time(upload_done)
    print(f"1 GiB H2D DMA {dma_ms:.2f} ms; 256 KiB upload done at {upload_ms:.2f} ms", flush=True)
    assert upload_ms < dma_ms / 2


def test_a_captured_upload_reads_the_pinned_source_at_each_replay(gpu):
    """A graph holding kvx_upload (as a decode graph would hold its static inputs' copies): the host rewrites the
    pinned source between replays, with eager work in between, and every replay lands the current contents."""
    src = torch.zeros(4096, dtype=torch.int32).pin_memory()
    dst = torch.full((4096,), -1, dtype=torch.int32, device=gpu)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize(gpu)
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream(gpu).cuda_stream
        check(lib().kvx_upload(dst.data_ptr(), src.data_ptr(), src.numel() * 4, stream), "upload")
    scratch = torch.empty(1 << 20, device=gpu)
    for replay in range(5):
        src.copy_(torch.arange(4096, dtype=torch.int32) * (replay + 3))
        graph.replay()
        scratch.mul_(2).add_(1)  # eager work between replays
        torch.cuda.synchronize(gpu)
        assert torch.equal(dst.cpu(), src), f"replay {replay}"
