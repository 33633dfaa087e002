#!/usr/bin/env python3
"""FP8 save + restore of Qwen3-8B-shaped KV blocks on one MI355X through libkvx.

Workload (config 2): a [2, 36, 320, 256, 8, 128] bf16 pool holding
0.5 * t(df=4) values with 4 seeded outlier channels (x20) per (K/V, layer,
KV head). One step saves 128 seeded blocks into pinned host slab slots
(gather + per-(token, head) e4m3 quantisation into device staging, then
DMA; fp32 scales) on the save stream while 128 host entries are restored
into 128 other seeded blocks (DMA into staging, then dequantisation +
scatter) on the restore stream: the two directions of the host link overlap.

`value` is logical KV throughput of that step: BF16-equivalent bytes saved +
restored per second (37,748,736 B per block and direction). `host_link`
prices the step's entry bytes against the PCIe link (spec and a measured
pinned-memcpy ceiling). `roofline` prices the dominant kernel's algorithmic
HBM bytes (57,212,928 B per block: 36 MiB bf16 read, 18 MiB e4m3 + 576 KiB
fp32 scales written, or the reverse) per launch against 8 TB/s, timed with
HIP events on its stream in the same save + restore with entries in HBM
(`kernels`). `cpu_baseline` times the reference's CPU path (its torch codec
on CPU tensors) on a bounded sample of the same blocks.

Run: python bench.py [--steps 50] [--warmup 5] [--blocks 128]
"""

import argparse
import ctypes
import json
import os
import subprocess
import sys
import time
from contextlib import contextmanager
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kv-cache-offloading_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "KV GB/s FP8 save+restore, Qwen3-8B blocks (% HBM & host-link roofline)"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
PCIE_PEAK_GBS = 63.0        # PCIe 5.0 x16, per direction (raw 64 GT/s x16 after 128b/130b)
BF16_BLOCK_BYTES = 37_748_736


def log(*args):
    print(*args, file=sys.stderr, flush=True)


@contextmanager
def marked(name: str):
    """A named range in rocprofv3's marker trace (roctx, through torch.cuda.nvtx), to split traces by leg."""
    import torch

    try:
        torch.cuda.nvtx.range_push(name)
        pushed = True
    except Exception:  # no marker library: the range is only a label
        pushed = False
    try:
        yield
    finally:
        if pushed:
            torch.cuda.nvtx.range_pop()


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--blocks", type=int, default=128, help="blocks saved and restored per step")
    p.add_argument("--scale", choices=("fp32", "bf16"), default="fp32")
    p.add_argument("--skip-host-link", action="store_true")
    p.add_argument("--skip-sdma-probe", action="store_true",
                   help="skip the host-link probe that queues HSA copies on explicit SDMA engines (it also skips "
                        "itself when a profiler tool is loaded)")
    p.add_argument("--skip-cpu-baseline", action="store_true")
    p.add_argument("--skip-store", action="store_true", help="skip the store_kvcache leg")
    p.add_argument("--skip-store-concurrency", action="store_true",
                   help="skip the store_kvcache leg's run beside concurrent FP8 saves")
    p.add_argument("--skip-tp-rank", action="store_true",
                   help="skip config 2 at one TP=8 rank's share of the pool (1 KV head)")
    p.add_argument("--skip-store-decode", action="store_true",
                   help="skip store_kvcache in the decode regime (1-512 tokens per step)")
    p.add_argument("--skip-hybrid", action="store_true", help="skip the hybrid-admission calibration leg")
    p.add_argument("--skip-agents", action="store_true", help="skip the agent-pressure leg")
    p.add_argument("--skip-handoff", action="store_true", help="skip the KV handoff leg")
    p.add_argument("--skip-microbench", action="store_true", help="skip the copy-path microbenchmark leg")
    p.add_argument("--skip-reference-gpu", action="store_true",
                   help="skip timing the reference's torch codec chain on the GPU")
    p.add_argument("--skip-configs", action="store_true",
                   help="skip the Qwen3-0.6B FP8 and Qwen3-8B BF16 legs")
    p.add_argument("--host-reps", type=int, default=3)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="after timing, gather the same blocks once with the BF16 copy kernel (known bytes), "
                        "to scale HBM counters read under rocprofv3 --pmc")
    return p.parse_args()


def pmc_traffic(kernel_prefix: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary, if one matches."""
    path = ROOT / "profiles" / "fp8_save_restore_qwen3_8b.traffic.json"
    if not path.exists():
        return None, None
    data = json.loads(path.read_text())
    for name, entry in data["kernels"].items():
        if name.startswith(kernel_prefix):
            return entry["total_bytes"], data["source"]
    return None, None


def kernel_leg(torch, ops, pool, sources, dests, scale_dtype, steps, warmup, block_bytes=BF16_BLOCK_BYTES,
               label="kernel leg"):
    """HBM-resident save + restore; returns timings and algorithmic byte counts (`block_bytes`: one pool block)."""
    layout = ops.pool_layout(pool, scale_dtype)
    logical, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    n = len(sources)
    staging = torch.empty(n * stride, dtype=torch.uint8, device=pool.device)
    entries = [staging.data_ptr() + i * stride for i in range(n)]
    stream = torch.cuda.current_stream(pool.device)

    def step(events=None):
        if events:
            events[0].record(stream)
        ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)
        if events:
            events[1].record(stream)
        ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, scale_dtype)
        if events:
            events[2].record(stream)

    for _ in range(warmup):
        step()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with marked(f"{label}: timed steps"):
        for ev in events:
            step(ev)
        torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    save_ms = sum(e[0].elapsed_time(e[1]) for e in events) / steps
    restore_ms = sum(e[1].elapsed_time(e[2]) for e in events) / steps
    hbm_bytes = n * (block_bytes + logical)  # per launch, either direction
    return dict(elapsed=elapsed, save_ms=save_ms, restore_ms=restore_ms, hbm_bytes=hbm_bytes,
                logical_entry=logical, entry_stride=stride)


def store_leg(torch, ops, pool, reps=5, concurrency=True):
    """store_kvcache over all layers for a ragged batch of 16 sequences (lengths U[1, 8192], seeded).

    K is contiguous; V is a strided view of a fused QKV output (row stride
    (32 + 2H) * hd, as Qwen3-8B's). The headline slots are distinct random
    pool slots, token by token (the worst case for the writes); the batch is
    padded to a multiple of 256 with -1 slots. `paged_blocks` times the same
    batch with the slot layout a model runner produces (model_runner.py:156-166):
    each sequence gets seeded random distinct blocks and fills them in order.
    `contiguous_slots` writes the batch to consecutive slots (streaming
    destinations). `writes_only` prices each slot pattern alone: the same
    kernel with K and V expanded from one row (row stride 0), so every token's
    source is one cached 4 KiB row and HBM sees only the destination rows.
    """
    import numpy as np

    _, layers, nb, bs, heads, hd = pool.shape
    rng = np.random.default_rng(7)
    lengths = rng.integers(1, 8193, size=16)
    total = int(min(lengths.sum(), nb * bs))
    padded = -(-total // 256) * 256
    slots = np.full(padded, -1, dtype=np.int32)
    slots[:total] = rng.permutation(nb * bs)[:total]
    g = torch.Generator(device=pool.device).manual_seed(8)
    qkv = torch.randn((padded, (32 + 2 * heads) * hd), generator=g, device=pool.device).to(torch.bfloat16)
    key = qkv[:, 32 * hd:(32 + heads) * hd].contiguous().view(padded, heads, hd)
    value = qkv[:, (32 + heads) * hd:].view(padded, heads, hd)
    stream = torch.cuda.current_stream(pool.device)
    row = heads * hd * 2

    def timed(slot_map, tokens, sources=(key, value)):
        mapping = torch.from_numpy(slot_map).to(pool.device)

        def run():
            for layer in range(layers):
                ops.store_kvcache(*sources, pool[0, layer], pool[1, layer], mapping)

        run()
        times = []
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            run()
            end.record(stream)
            end.synchronize()
            times.append(start.elapsed_time(end) / 1000)
        t = sorted(times)[len(times) // 2]
        per_launch = tokens * 4 * row + padded * 4  # K and V rows read and written, plus the slot map
        gbs = layers * per_launch / t / 1e9
        return t, per_launch, gbs

    t, per_launch, gbs = timed(slots, total)
    traffic, _ = pmc_traffic("store_kv_vec<")
    out = {"tokens": total, "padded_tokens": padded, "layers": layers, "ms_all_layers": round(1000 * t, 4),
           "algorithmic_bytes_per_launch": per_launch, "hbm_gbs": round(gbs, 1),
           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}

    paged = np.full(padded, -1, dtype=np.int32)
    blocks = iter(rng.permutation(nb).tolist())
    pos = 0
    for length in lengths.tolist():
        need = -(-length // bs)
        if pos + length > padded or need > nb:
            break
        table = [next(blocks, None) for _ in range(need)]
        if None in table:
            break
        seq_slots = (np.asarray(table, dtype=np.int64)[:, None] * bs + np.arange(bs)).reshape(-1)[:length]
        paged[pos:pos + length] = seq_slots
        pos += length
    t, per_launch, gbs = timed(paged, pos)
    out["paged_blocks"] = {"tokens": pos, "ms_all_layers": round(1000 * t, 4),
                           "algorithmic_bytes_per_launch": per_launch, "hbm_gbs": round(gbs, 1),
                           "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # The same kernel and batch with the destinations in slot order (a prefill into fresh, consecutive blocks):
    # the rate the kernel reaches when its writes stream, against which the random 2 KiB rows are priced.
    contiguous = np.full(padded, -1, dtype=np.int32)
    contiguous[:total] = np.arange(total, dtype=np.int32)
    t, per_launch, gbs = timed(contiguous, total)
    out["contiguous_slots"] = {"tokens": total, "ms_all_layers": round(1000 * t, 4), "hbm_gbs": round(gbs, 1),
                               "frac": round(gbs / HBM_PEAK_GBS, 4)}
    out["random_vs_contiguous"] = round(out["hbm_gbs"] / gbs, 4)
    one_row = (key[:1].expand(padded, heads, hd), value[:1].expand(padded, heads, hd))
    written = {}
    for name, slot_map, tokens in (("random", slots, total), ("paged_blocks", paged, pos),
                                   ("contiguous", contiguous, total)):
        t, _, _ = timed(slot_map, tokens, one_row)
        wgbs = layers * (tokens * 2 * row + padded * 4) / t / 1e9
        written[name] = {"ms_all_layers": round(1000 * t, 4), "write_gbs": round(wgbs, 1),
                         "frac": round(wgbs / HBM_PEAK_GBS, 4)}
    out["writes_only"] = written
    if concurrency:
        out["with_concurrent_saves"] = store_beside_saves(torch, ops, pool, key, value, lengths, reps)
    return out


def store_decode_leg(torch, ops, pool, batches=(1, 8, 64, 256, 512), reps=100):
    """store_kvcache in the decode regime: one new token per running request, every layer, per step.

    The reference's decode step calls it once per layer with N = the batch
    (padded to a captured size), inside a CUDA graph for batches up to 512
    (model_runner.py:201-262, attention.py:59-63). For each N: the host time
    of one eager ops.store_kvcache call (all checks and the C call), of the
    bare C call with its arguments prepared, the device time per step of a
    HIP graph replaying the step's calls, and the device time per step of
    the same calls issued eagerly back to back. K is contiguous; V is a
    strided view of a fused QKV row ((32 + 2H) * hd elements), as in
    Qwen3-8B; slots are distinct random pool slots.
    """
    import ctypes as c

    import numpy as np

    from kvx._lib import lib

    _, layers, nb, bs, heads, hd = pool.shape
    rng = np.random.default_rng(11)
    stream = torch.cuda.current_stream(pool.device)
    out = {"layers": layers, "reps": reps}
    for n in batches:
        g = torch.Generator(device=pool.device).manual_seed(n)
        qkv = torch.randn((n, (32 + 2 * heads) * hd), generator=g, device=pool.device).to(torch.bfloat16)
        key = qkv[:, 32 * hd:(32 + heads) * hd].view(n, heads, hd)
        value = qkv[:, (32 + heads) * hd:].view(n, heads, hd)
        mapping = torch.from_numpy(rng.permutation(nb * bs)[:n].astype(np.int32)).to(pool.device)
        k_caches = [pool[0, layer] for layer in range(layers)]
        v_caches = [pool[1, layer] for layer in range(layers)]

        def step():
            for layer in range(layers):
                ops.store_kvcache(key, value, k_caches[layer], v_caches[layer], mapping)

        raw_args = [(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_caches[layer].data_ptr(),
                     v_caches[layer].data_ptr(), mapping.data_ptr(), n, heads, hd, 2,
                     k_caches[layer].numel() // (heads * hd), c.c_void_p(stream.cuda_stream))
                    for layer in range(layers)]
        fn = lib().kvx_store_kvcache

        def raw_step():
            for args in raw_args:
                fn(*args)

        res = {}
        for name, issue in (("eager_call", step), ("bare_c_call", raw_step)):
            issue()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                issue()
            host = time.perf_counter() - t0
            torch.cuda.synchronize()
            res[f"{name}_host_us"] = round(1e6 * host / (reps * layers), 2)
        # Device time per step: the step's calls replayed from a captured graph, and issued eagerly after a
        # long delay kernel so the queue is full before the device reaches them.
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(pool.device)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            step()
        stream.wait_stream(side)
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with marked(f"store decode: graph, {n} tokens"):
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
            e1.synchronize()
        res["graph_step_us"] = round(1000 * e0.elapsed_time(e1) / reps, 2)
        ops.sleep(20_000, stream=stream, device=pool.device)
        with marked(f"store decode: eager, {n} tokens"):
            e0.record(stream)
            for _ in range(20):
                step()
            e1.record(stream)
            e1.synchronize()
        res["eager_step_us_queued"] = round(1000 * e0.elapsed_time(e1) / 20, 2)
        res["device_us_per_call"] = round(res["graph_step_us"] / layers, 3)
        res["host_over_device"] = round(res["eager_call_host_us"] / res["device_us_per_call"], 2)
        res["algorithmic_bytes_per_call"] = n * (4 * heads * hd * 2 + 4)
        del graph
        out[str(n)] = res
        log(f"store decode {n} tokens: {json.dumps(res)}")
    return out


def store_beside_saves(torch, ops, pool, key, value, lengths, reps):
    """The same batch written while FP8 saves of 64 seeded evicted blocks run on the save stream.

    The batch's slots avoid the evicted blocks (a block being saved is not
    rewritten). The saves are queued first, one call per block (as the
    reference's BlockManager issues them) or as one batched call, then the
    36 store launches on the compute stream. The stores are timed on the
    compute stream from their first launch; the saves on the save stream from
    before they were queued; the host time spent queueing the saves is
    reported beside them.
    """
    import numpy as np
    from types import SimpleNamespace

    from kvx.engine.block_manager import BlockManager
    from kvx.engine.cpu_prefix_cache import CPUBlockCache
    from workloads import block_selection

    _, layers, nb, bs, heads, hd = pool.shape
    evicted = block_selection(nb, 64, seed=6)
    excluded = set(evicted)
    free_slots = np.array([b * bs + i for b in range(nb) if b not in excluded for i in range(bs)])
    total = int(min(lengths.sum(), free_slots.size))
    padded = key.shape[0]
    slots = np.full(padded, -1, dtype=np.int32)
    slots[:total] = np.random.default_rng(9).permutation(free_slots)[:total]
    mapping = torch.from_numpy(slots).to(pool.device)
    manager = BlockManager(nb, bs)
    keys = []
    for i, b in enumerate(evicted):
        tokens = [5000 + i] * bs
        h = BlockManager.compute_hash(tokens)
        manager.blocks[b].update(h, tokens)
        manager.hash_to_block_id[h] = b
        keys.append(h)
    runner = SimpleNamespace(world_size=1, block_size=bs, kv_cache=pool)
    entry = pool[:, :, 0].numel() + pool[:, :, 0].numel() // hd * 4
    cache = CPUBlockCache(runner, manager, 64 * entry, split_streams=True, fp8=True, scale_dtype=torch.float32,
                          preallocate=True)
    compute = torch.cuda.current_stream(pool.device)
    row = heads * hd * 2
    per_launch = total * 4 * row + padded * 4
    out = {"tokens": total, "saved_blocks": 64}
    try:
        for mode in ("alone", "per_block_saves", "batched_saves"):
            store_ms, save_ms, issue_ms = [], [], []
            for _ in range(reps + 1):
                cache.clear()
                torch.cuda.synchronize()
                start, store_start, store_end, save_end = (torch.cuda.Event(enable_timing=True) for _ in range(4))
                start.record(compute)
                t0 = time.perf_counter()
                if mode == "per_block_saves":
                    for k in keys:
                        cache.save_block(k)
                elif mode == "batched_saves":
                    with cache.coalesce():
                        for k in keys:
                            cache.save_block(k)
                issue_ms.append(1000 * (time.perf_counter() - t0))
                store_start.record(compute)
                for layer in range(layers):
                    ops.store_kvcache(key, value, pool[0, layer], pool[1, layer], mapping)
                store_end.record(compute)
                save_end.record(cache._copy_stream)
                torch.cuda.synchronize()
                store_ms.append(store_start.elapsed_time(store_end))
                save_ms.append(start.elapsed_time(save_end))
            store_t = sorted(store_ms[1:])[reps // 2] / 1000
            res = {"store_ms": round(1000 * store_t, 3), "store_hbm_gbs": round(layers * per_launch / store_t / 1e9, 1)}
            if mode != "alone":
                save_t = sorted(save_ms[1:])[reps // 2] / 1000
                res.update({"saves_done_ms": round(1000 * save_t, 3),
                            "save_link_gbs": round(64 * cache.block_bytes / save_t / 1e9, 2),
                            "save_issue_host_ms": round(sorted(issue_ms[1:])[reps // 2], 3)})
            out[mode] = res
    finally:
        cache.close()
    return out


def microbench_leg(torch, blocks=64, matmul_iters=200):
    """The reference's copy-path microbenchmark (bench/cpu_cache_microbench.py:59-163) on this path.

    Same workload and measurements: a Qwen3-0.6B-shaped pool of 2 * blocks
    blocks; pinned memcpy ceilings (:91-98); the cost of a pinned allocation
    per save (:101-106) and of a synchronous pageable save (:109-116); per-block
    save_block / restore_block through the cache (:119-127); and whether saves
    on the copy stream slow concurrent compute, 4096^2 bf16 matmuls (:130-155).
    Issue time is host time until the calls return, total adds the device wait.
    The reference runs its default (BF16) cache; the FP8 cache runs as well.
    """
    from types import SimpleNamespace

    from kvx.engine.block_manager import BlockManager
    from kvx.engine.cpu_prefix_cache import CPUBlockCache
    from workloads import QWEN3_0_6B

    n = blocks
    shape = (2, QWEN3_0_6B.layers, 2 * n, *QWEN3_0_6B.shape[3:])
    g = torch.Generator(device="cuda").manual_seed(0)
    pool = torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16)
    bs = shape[3]
    block_shape = (2, shape[1], *shape[3:])
    block_bytes = pool[:, :, 0].numel() * pool.element_size()
    runner = SimpleNamespace(world_size=1, block_size=bs, kv_cache=pool)

    def timed(fn):
        torch.cuda.synchronize()
        start = time.perf_counter()
        fn()
        issued = time.perf_counter()
        torch.cuda.synchronize()
        return issued - start, time.perf_counter() - start

    def per_block(issue_s, total_s, nbytes=block_bytes):
        return {"issue_ms_per_block": round(1000 * issue_s / n, 4), "ms_per_block": round(1000 * total_s / n, 4),
                "gb_per_s": round(n * nbytes / total_s / 1e9, 2)}

    def published():
        manager = BlockManager(2 * n, bs)
        hashes = []
        for i in range(n):
            tokens = [i] * bs
            h = BlockManager.compute_hash(tokens)
            manager.blocks[i].update(h, tokens)
            manager.hash_to_block_id[h] = i
            hashes.append(h)
        return manager, hashes

    out = {"pool": list(shape), "blocks": n, "block_bytes": block_bytes}
    flat_gpu = torch.empty(n * block_bytes // 2, dtype=torch.bfloat16, device="cuda")
    flat_host = torch.empty_like(flat_gpu, device="cpu", pin_memory=True)
    flat_host.copy_(flat_gpu)
    out["pinned_memcpy_d2h"] = per_block(*timed(lambda: flat_host.copy_(flat_gpu, non_blocking=True)))
    out["pinned_memcpy_h2d"] = per_block(*timed(lambda: flat_gpu.copy_(flat_host, non_blocking=True)))
    del flat_gpu, flat_host

    def pinned_allocs():
        return [torch.empty(block_shape, dtype=pool.dtype, pin_memory=True) for _ in range(n)]

    _, total = timed(pinned_allocs)
    out["per_save_pinned_alloc"] = {"ms_per_block": round(1000 * total / n, 4)}

    def pageable_saves():
        keep = []
        for i in range(n):
            payload = torch.empty(block_shape, dtype=pool.dtype)
            torch.cuda.synchronize()
            payload.copy_(pool[:, :, i], non_blocking=False)
            keep.append(payload)

    out["pageable_sync_save"] = per_block(*timed(pageable_saves))

    x = torch.randn(4096, 4096, dtype=torch.bfloat16, device="cuda")

    def matmuls():
        for _ in range(matmul_iters):
            torch.mm(x, x)

    matmuls()  # library warm-up
    _, compute_s = timed(matmuls)
    for name, fp8 in (("bf16", False), ("fp8", True)):
        manager, hashes = published()
        kw = dict(fp8=True, scale_dtype=torch.float32) if fp8 else {}
        start = time.perf_counter()
        cache = CPUBlockCache(runner, manager, n * block_bytes, preallocate=True, **kw)
        res = {"slab_preallocate_s": round(time.perf_counter() - start, 3)}
        entry = cache.block_bytes
        try:
            with marked(f"microbench {name}: slab saves"):
                res["slab_save"] = per_block(*timed(lambda: [cache.save_block(h) for h in hashes]), entry)
            for h in hashes:
                block = manager.blocks[manager.hash_to_block_id.pop(h)]
                block.hash, block.token_ids = -1, []
            with marked(f"microbench {name}: slab restores"):
                res["slab_restore"] = per_block(*timed(lambda: [cache.restore_block(h) for h in hashes]), entry)
        finally:
            cache.close()
        manager, hashes = published()
        cache = CPUBlockCache(runner, manager, n * block_bytes, preallocate=True, **kw)
        try:
            _, copy_s = timed(lambda: [cache.save_block(h) for h in hashes])
            cache.clear()

            def both():
                for h in hashes:  # saves first: each waits for the compute queued before it
                    cache.save_block(h)
                matmuls()

            _, both_s = timed(both)
        finally:
            cache.close()
        res["overlap"] = {"compute_alone_s": round(compute_s, 5), "saves_alone_s": round(copy_s, 5),
                          "together_s": round(both_s, 5), "serial_sum_s": round(compute_s + copy_s, 5),
                          "hidden_fraction": round((compute_s + copy_s - both_s) / min(compute_s, copy_s), 3)}
        out[name] = res
    return out


# Recompute cost coefficients the reference's replay harness defaults to
# (bench/agent_replay.py:283-286); they describe the model, not this path.
RECOMPUTE_S_PER_TOKEN = 6.87e-6
RECOMPUTE_S_PER_TOKEN2 = 9.3e-10


def hybrid_leg(torch, pool, scale_dtype, prefix_blocks=128):
    """The hybrid-admission calibration loop (bench/agent_replay.py:387-391) on this path.

    Measures the restore cost per block (H2D DMA plus dequantisation) with
    CPUBlockCache.measure_restore_s_per_block, sets cache.hybrid from it, and
    reports the split plan_split picks for a 32,768-token prefix.
    """
    from types import SimpleNamespace

    from kvx.engine.block_manager import BlockManager, plan_split
    from kvx.engine.cpu_prefix_cache import CPUBlockCache

    _, _, nb, bs, _, _ = pool.shape
    runner = SimpleNamespace(world_size=1, block_size=bs, kv_cache=pool)
    out = {"prefix_blocks": prefix_blocks, "recompute_s_per_token": RECOMPUTE_S_PER_TOKEN,
           "recompute_s_per_token2": RECOMPUTE_S_PER_TOKEN2}
    for name, fp8 in (("fp8", True), ("bf16", False)):
        cache = CPUBlockCache(runner, BlockManager(nb, bs), 1 << 30, automatic=True, fp8=fp8,
                              scale_dtype=scale_dtype if fp8 else None)
        try:
            restore_s = cache.measure_restore_s_per_block()
            cache.hybrid = (restore_s, RECOMPUTE_S_PER_TOKEN, RECOMPUTE_S_PER_TOKEN2)
            split = plan_split(prefix_blocks, bs, *cache.hybrid)
        finally:
            cache.close()
        tokens = split * bs
        recompute = tokens * RECOMPUTE_S_PER_TOKEN + tokens * tokens * RECOMPUTE_S_PER_TOKEN2
        out[name] = {"restore_ms_per_block": round(1000 * restore_s, 4),
                     "restore_gbs": round(cache.block_bytes / restore_s / 1e9, 2),
                     "recompute_blocks": split, "restored_blocks": prefix_blocks - split,
                     "admission_ms": round(1000 * max(recompute, (prefix_blocks - split) * restore_s), 3),
                     "restore_only_ms": round(1000 * prefix_blocks * restore_s, 3)}
    return out


def agent_leg(torch, pool, scale_dtype, h2d_gbs=None):
    """Agent pressure through the whole engine: 4 agents x 32,768-token contexts, 12 turns of 2,048 new tokens.

    FP8 saves of evicted blocks into an 8 GiB pinned budget, restores and
    prefetch restores of each returning agent's prefix, KV written by
    store_kvcache. Run with split save/restore streams, with one copy stream,
    and with split streams but one engine call per block (the call pattern of
    the reference's BlockManager, which has no coalesce()); link GB/s is
    entry bytes moved over the run's wall time
    (engine, scheduling and the synthetic model included). Each cache pins its
    whole budget when it is created (the reference's preallocate option), so
    neither run's time includes page-locking host memory.

    The CPU tier never evicts: once the 8 GiB budget (441 entries) is full, a
    save is dropped and counted as a budget skip (cpu_prefix_cache.py:297-298,
    334-340), and from then on the run only restores. `budget_for_all` repeats
    the split-stream run with a budget that holds every agent's blocks, so
    saves continue through every turn.

    Each agent's request hints the next agent's prefix with
    prefetch_prefix(defer=True): the engine starts those restores right after
    the request's admission, so they overlap its compute. `hints_after_first_step`
    repeats the split-stream run hinting after the request's first step, the
    only time a client of the reference engine can hint (its hints are dropped
    while a request waits). With `h2d_gbs` (the copy engine's measured H2D rate
    for batched restores), each run reports the time its H2D bytes need at
    that rate and its wall time over it.
    """
    from contextlib import nullcontext

    from kvx.engine.llm_engine import LLMEngine
    from workloads import SyntheticKVRunner, run_agent_pressure

    out = {"agents": 4, "context_tokens": 32768, "turns": 12, "append_tokens": 2048, "host_budget_bytes": 8 << 30}
    # The first (untimed, one-turn) run grows torch's allocator for the synthetic model, so no timed run pays it.
    budget = 8 << 30
    blocks_per_agent = -(-(32768 + 12 * (2048 + 1)) // pool.shape[3])
    entry = 2 * pool.shape[1] * pool.shape[3] * pool.shape[4] * (pool.shape[5] + scale_dtype.itemsize)
    budget_for_all = -(-4 * blocks_per_agent * entry // (1 << 30)) << 30  # every agent's blocks, in whole GiB
    runs = (("warm-up", True, 1, True, budget, "deferred"), ("split_streams", True, 12, True, budget, "deferred"),
            ("hints_after_first_step", True, 12, True, budget, "after_first_step"),
            ("one_copy_stream", False, 12, True, budget, "deferred"),
            ("per_block_calls", True, 12, False, budget, "deferred"),
            ("budget_for_all", True, 12, True, budget_for_all, "deferred"))
    for name, split, turns, batched, max_bytes, hints in runs:
        engine = LLMEngine(SyntheticKVRunner(pool), max_num_batched_tokens=16384, max_num_seqs=4, eos=-1,
                           kvcache_block_size=pool.shape[3], num_kvcache_blocks=pool.shape[2])
        cache = engine.create_cpu_prefix_cache(max_bytes, automatic=True, prefetch=True, split_streams=split,
                                               fp8=True, scale_dtype=scale_dtype, preallocate=True)
        if not batched:
            cache.coalesce = nullcontext  # the block manager then issues one engine call per block
        try:
            with marked(f"agents: {name}"):
                r = run_agent_pressure(engine, agents=4, context=32768, turns=turns, append=2048, verify=False,
                                       hints=hints)
            copy_stats = cache.copy_stats
        finally:
            engine.exit()
        if name == "warm-up":
            continue
        out[name] = {"wall_s": round(r.wall_s, 3), "saved_blocks": r.saved_blocks,
                     "restored_blocks": r.restored_blocks, "prefetched_blocks": r.prefetched_blocks,
                     "d2h_bytes": r.d2h_bytes, "h2d_bytes": r.h2d_bytes, "link_gbs": round(r.link_gbs, 2),
                     "host_blocked_s": round(r.host_blocked_s, 3), "drain_s": round(r.drain_s, 4),
                     "budget_skips": r.budget_skips, "host_budget_bytes": max_bytes, "hints": hints,
                     "dma_copies": {k: copy_stats[k] for k in ("d2h_copies", "h2d_copies")}}
        if h2d_gbs:
            floor = r.h2d_bytes / (h2d_gbs * 1e9)
            out[name].update(h2d_floor_s=round(floor, 3), wall_over_h2d_floor=round(r.wall_s / floor, 3))
        log(f"agents {name}: {json.dumps(out[name])}")
    if h2d_gbs:
        out["h2d_gbs_for_floor"] = h2d_gbs
    out["deferred_hint_speedup"] = round(out["hints_after_first_step"]["wall_s"] / out["split_streams"]["wall_s"], 3)
    out["split_speedup"] = round(out["one_copy_stream"]["wall_s"] / out["split_streams"]["wall_s"], 3)
    out["batching_speedup"] = round(out["per_block_calls"]["wall_s"] / out["split_streams"]["wall_s"], 3)
    return out


def timed_pair(torch, first, second, reps=10):
    """Median event times (s) of two launches queued back to back on the current stream."""
    stream = torch.cuda.current_stream()
    first(), second()
    t1, t2 = [], []
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        ev[0].record(stream)
        first()
        ev[1].record(stream)
        second()
        ev[2].record(stream)
        ev[2].synchronize()
        t1.append(ev[0].elapsed_time(ev[1]) / 1000)
        t2.append(ev[1].elapsed_time(ev[2]) / 1000)
    return sorted(t1)[reps // 2], sorted(t2)[reps // 2]


def reference_gpu_leg(torch, pool, sources, dests, scale_dtype, kvx_step_ms, reps=3):
    """The reference's own implementation of this path, run on this GPU for comparison.

    Per block, the reference quantises into device staging with four torch
    calls (fp8_quantize, cpu_prefix_cache.py:20-24, via _quantize :225-231)
    and dequantises into the pool with two (fp8_dequantize :27-28, via
    _dequantize :236-243). Here the same calls run over the same 128 + 128
    blocks with every entry staged in HBM (no host copies), exactly the work
    the kvx step times.
    """
    _, layers, _, bs, heads, hd = pool.shape
    block = (2, layers, bs, heads, hd)
    n = len(sources)
    payload = torch.empty((n, *block), dtype=torch.float8_e4m3fn, device=pool.device)
    scale = torch.empty((n, *block[:-1], 1), dtype=scale_dtype, device=pool.device)

    def save():
        for i, b in enumerate(sources):
            source = pool[:, :, b]
            row_max = source.abs().amax(-1, keepdim=True).float()
            scale[i].copy_((row_max / 448.0).clamp_min(1e-30))
            payload[i].copy_((source.float() / scale[i].float()).clamp_(-448.0, 448.0))

    def restore():
        for i, d in enumerate(dests):
            torch.mul(payload[i].to(pool.dtype), scale[i], out=pool[:, :, d])

    save_s, restore_s = timed_pair(torch, save, restore, reps=reps)
    step_ms = 1000 * (save_s + restore_s)
    return {"blocks_saved": n, "blocks_restored": len(dests), "save_ms": round(1000 * save_s, 3),
            "restore_ms": round(1000 * restore_s, 3), "step_ms": round(step_ms, 3),
            "logical_kv_gbs": round(2 * n * BF16_BLOCK_BYTES / (step_ms / 1000) / 1e9, 1),
            "kvx_speedup": round(step_ms / kvx_step_ms, 2)}


def reference_link_leg(torch, pool, sources, dests, scale_dtype, reps=3):
    """The reference's host path for FP8 blocks, run on this GPU for comparison with the host-link leg.

    Per block, a save quantises into the stream's one device staging pair and
    queues two non-blocking D2H copies (payload, scales) on the copy stream
    (cpu_prefix_cache.py:225-234, 306-322); a restore copies both back into
    staging and dequantises into the pool (:236-243, 374-393). Save and
    restore streams are chosen like the kvx cache's (concurrent queues), so
    only the implementation differs. Returns link GB/s of logical entry bytes.
    """
    from kvx.engine.cpu_prefix_cache import _copy_streams

    (save_stream, restore_stream), _ = _copy_streams(pool.device, 2)
    _, layers, _, bs, heads, hd = pool.shape
    block, rows = (2, layers, bs, heads, hd), (2, layers, bs, heads, 1)
    n = len(sources)
    host_payload = torch.empty((2 * n, *block), dtype=torch.float8_e4m3fn, pin_memory=True)
    host_scale = torch.empty((2 * n, *rows), dtype=scale_dtype, pin_memory=True)
    stage = [(torch.empty(block, dtype=torch.float8_e4m3fn, device=pool.device),
              torch.empty(rows, dtype=scale_dtype, device=pool.device)) for _ in range(2)]

    def quantize(source, payload, scale):
        row_max = source.abs().amax(-1, keepdim=True).float()
        scale.copy_((row_max / 448.0).clamp_min(1e-30))
        payload.copy_((source.float() / scale.float()).clamp_(-448.0, 448.0))

    def save(first):
        payload, scale = stage[0]
        with torch.cuda.stream(save_stream):
            for i, b in enumerate(sources):
                quantize(pool[:, :, b], payload, scale)
                host_payload[first + i].copy_(payload, non_blocking=True)
                host_scale[first + i].copy_(scale, non_blocking=True)

    def restore():
        payload, scale = stage[1]
        with torch.cuda.stream(restore_stream):
            for i, d in enumerate(dests):
                payload.copy_(host_payload[i], non_blocking=True)
                scale.copy_(host_scale[i], non_blocking=True)
                torch.mul(payload.to(pool.dtype), scale, out=pool[:, :, d])

    def timed(*fns):
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for fn in fns:
                fn()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return best

    save(0)  # entries for the restores to read
    torch.cuda.synchronize()
    link = n * (host_payload[0].numel() + host_scale[0].numel() * host_scale.element_size())
    save_s = timed(lambda: save(n))
    restore_s = timed(restore)
    both_s = timed(lambda: save(n), restore)
    return {"bytes_per_direction": link, "save_d2h_gbs": round(link / save_s / 1e9, 2),
            "restore_h2d_gbs": round(link / restore_s / 1e9, 2), "duplex_gbs": round(2 * link / both_s / 1e9, 2)}


def handoff_leg(torch, pool, reps=3):
    """KV handoff of one 32,767-token request (128 blocks) on the Qwen3-8B pool: export and import, BF16 and FP8.

    kvx: export_kv's and import_kv's copy (kv_handoff.copy_tokens: a group of
    (K/V, layer) planes at a time through 256 MiB of device staging, the token
    gather or scatter, quantising or dequantising for FP8, and one DMA per
    tensor and group), each waited for. Beside
    them, the reference's BF16 copies for the same request on this GPU
    (kv_handoff.py:46-55: index_select, pack, .cpu(); :112-118: .to(device),
    one copy_ per block). `wire_gbs` counts payload bytes (what crosses the
    link), `logical_kv_gbs` the BF16 bytes of the request's KV.
    """
    from kvx.engine.kv_handoff import copy_tokens
    from workloads import block_selection

    _, layers, nb, bs, heads, hd = pool.shape
    count = 128 * bs - 1
    table = block_selection(nb, 128, seed=1)
    dest = block_selection(nb, 128, seed=2)
    shape = (2, layers, count, heads, hd)
    logical = 2 * layers * count * heads * hd * pool.element_size()
    device = pool.device

    def timed(fn):
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return best

    bf16 = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
    codes = torch.empty(shape, dtype=torch.float8_e4m3fn, pin_memory=True)
    scales = torch.empty((*shape[:-1], 1), dtype=torch.float32, pin_memory=True)
    fp8_bytes = codes.numel() + scales.numel() * scales.element_size()

    def kvx_export():
        copy_tokens(True, pool, table, count, bf16)

    def kvx_import():
        copy_tokens(False, pool, dest, count, bf16)

    def kvx_export_fp8():
        copy_tokens(True, pool, table, count, codes, scales)

    def kvx_import_fp8():
        copy_tokens(False, pool, dest, count, codes, scales)

    ids = torch.tensor(table, dtype=torch.int64, device=device)
    held = {}

    def reference_export():
        held["kv"] = pool.index_select(2, ids).flatten(2, 3)[:, :, :count].contiguous().cpu()

    def reference_import():
        payload = held["kv"].to(device=device)
        for logical_block, physical in enumerate(dest):
            start = logical_block * bs
            end = min(start + bs, count)
            pool[:, :, physical, :end - start].copy_(payload[:, :, start:end])

    out = {"tokens": count, "bf16_payload_bytes": logical, "fp8_payload_bytes": fp8_bytes}
    for name, fn, wire in (("kvx_export", kvx_export, logical), ("kvx_import", kvx_import, logical),
                           ("kvx_export_fp8", kvx_export_fp8, fp8_bytes), ("kvx_import_fp8", kvx_import_fp8, fp8_bytes),
                           ("reference_export", reference_export, logical),
                           ("reference_import", reference_import, logical)):
        seconds = timed(fn)
        out[name] = {"ms": round(1000 * seconds, 2), "wire_gbs": round(wire / seconds / 1e9, 2),
                     "logical_kv_gbs": round(logical / seconds / 1e9, 2)}
    return out


def bf16_leg(torch, ops, pool, reps, link=True):
    """BF16 storage mode on the Qwen3-8B pool: byte gather of 200 seeded blocks into entries and scatter into
    200 other seeded blocks (HBM-resident), then the same 200 blocks over the host link: saved to pinned host
    slots and restored into those 200 destinations, which overlap the sources (restores into a block being
    saved wait for its save kernel)."""
    from workloads import block_selection

    nb = pool.shape[2]
    sources = block_selection(nb, 200, seed=3)
    dests = block_selection(nb, 200, seed=4)
    layout = ops.pool_layout(pool)
    logical, _, stride = ops.entry_layout(layout, ops.FORMAT_RAW)
    staging = torch.empty(len(sources) * stride, dtype=torch.uint8, device=pool.device)
    entries = [staging.data_ptr() + i * stride for i in range(len(sources))]
    gather_s, scatter_s = timed_pair(torch, lambda: ops.save_blocks(pool, sources, entries, ops.FORMAT_RAW),
                                     lambda: ops.restore_blocks(pool, dests, entries, ops.FORMAT_RAW))
    del staging
    moved = len(sources) * 2 * BF16_BLOCK_BYTES  # read + written per launch
    link = host_link_leg(torch, pool, layout, sources, dests, reps, fmt=ops.FORMAT_RAW,
                         ceilings=False) if link else None
    return {"blocks": len(sources), "algorithmic_bytes_per_launch": moved,
            "gather": {"ms": round(1000 * gather_s, 4), "hbm_gbs": round(moved / gather_s / 1e9, 1),
                       "frac": round(moved / gather_s / 1e9 / HBM_PEAK_GBS, 4)},
            "scatter": {"ms": round(1000 * scatter_s, 4), "hbm_gbs": round(moved / scatter_s / 1e9, 1),
                        "frac": round(moved / scatter_s / 1e9 / HBM_PEAK_GBS, 4)},
            "host_link_200_blocks": link}


def qwen3_0_6b_leg(torch, ops, scale_dtype):
    """FP8 save of 16 seeded Qwen3-0.6B blocks and restore into 16 other seeded blocks, HBM-resident."""
    from workloads import QWEN3_0_6B, block_selection, fill_normal

    pool = torch.empty(QWEN3_0_6B.shape, dtype=torch.bfloat16, device="cuda")
    fill_normal(pool, seed=0)
    order = block_selection(QWEN3_0_6B.num_blocks, 32, seed=1)
    sources, dests = order[:16], order[16:]
    layout = ops.pool_layout(pool, scale_dtype)
    logical, _, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    staging = torch.empty(16 * stride, dtype=torch.uint8, device=pool.device)
    entries = [staging.data_ptr() + i * stride for i in range(16)]
    save_s, restore_s = timed_pair(
        torch, lambda: ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype),
        lambda: ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, scale_dtype), reps=20)
    block = pool[:, :, 0].numel() * 2
    moved = 16 * (block + logical)
    del staging, pool
    return {"pool": list(QWEN3_0_6B.shape), "blocks": 16, "algorithmic_bytes_per_launch": moved,
            "logical_kv_gbs": round(2 * 16 * block / (save_s + restore_s) / 1e9, 1),
            "save": {"ms": round(1000 * save_s, 4), "hbm_gbs": round(moved / save_s / 1e9, 1)},
            "restore": {"ms": round(1000 * restore_s, 4), "hbm_gbs": round(moved / restore_s / 1e9, 1)}}


def host_link_leg(torch, pool, layout, sources, dests, reps, fmt=None, ceilings=True):
    """Saves to / restores from pinned host slabs through the copy engine; D2H, H2D, both at once."""
    from kvx import ops
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    n = len(sources)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8 if fmt is None else fmt, split=True)
    try:
        stride = engine.entry_stride
        link_bytes = n * engine.logical_bytes
        t = time.perf_counter()
        slab = torch.empty(2 * n * stride, dtype=torch.uint8, pin_memory=True)
        pin_s = time.perf_counter() - t
        save_staging = torch.empty(n * stride, dtype=torch.uint8, device=pool.device)
        restore_staging = torch.empty(n * stride, dtype=torch.uint8, device=pool.device)
        engine.add_slab(slab, 2 * n)
        engine.set_staging(save_staging, restore_staging, n)
        compute = torch.cuda.current_stream(pool.device).cuda_stream
        low, high = list(range(n)), list(range(n, 2 * n))
        # DMA copies queued per phase (the engine's counters, or the pieces a memcpy phase queues): a memory-copy
        # trace of the phase must hold exactly this many records per direction.
        copies = {}

        def timed(fn, label="host link", pieces_per_rep=None):
            best = None
            before = engine.dma_counters()
            with marked(label):
                for _ in range(reps):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    fn()
                    engine.synchronize()
                    torch.cuda.synchronize()
                    dt = time.perf_counter() - t0
                    best = dt if best is None else min(best, dt)
            after = engine.dma_counters()
            copies[label] = {k: after[k] - before[k] for k in ("d2h_copies", "h2d_copies")}
            if pieces_per_rep:
                for k, v in pieces_per_rep.items():
                    copies[label][k] += reps * v
            return best

        engine.save(sources, low, compute)  # fill the restore source slots
        engine.synchronize()
        save_s = timed(lambda: engine.save(sources, high, compute), "host link: saves alone")
        restore_s = timed(lambda: engine.restore(low, dests, False, compute), "host link: restores alone")

        def both():
            engine.save(sources, high, compute)
            engine.restore(low, dests, False, compute)

        both_s = timed(both, "host link: both")

        # What CPUBlockCache does: one engine call per block, with its default staging.
        from kvx.engine.cpu_prefix_cache import _MAX_BATCH, _STAGING_BYTES

        engine.set_staging(save_staging, restore_staging, max(1, min(_MAX_BATCH, _STAGING_BYTES // stride)))

        def calls_of(k):
            def save_each():
                for i in range(0, n, k):
                    engine.save(sources[i:i + k], high[i:i + k], compute)

            def restore_each():
                for i in range(0, n, k):
                    engine.restore(low[i:i + k], dests[i:i + k], False, compute)

            def both_each():
                for i in range(0, n, k):
                    engine.save(sources[i:i + k], high[i:i + k], compute)
                    engine.restore(low[i:i + k], dests[i:i + k], False, compute)

            save_s_k = timed(save_each, f"host link: saves, calls of {k}")
            restore_s_k = timed(restore_each, f"host link: restores, calls of {k}")
            both_s_k = timed(both_each, f"host link: both, calls of {k}")
            return {"save_d2h_gbs": round(gbs(link_bytes, save_s_k), 2),
                    "restore_h2d_gbs": round(gbs(link_bytes, restore_s_k), 2),
                    "duplex_gbs": round(gbs(2 * link_bytes, both_s_k), 2)}

        gbs = lambda nbytes, s: nbytes / s / 1e9  # noqa: E731
        # One block per call (the reference's BlockManager), and four (a small batch, as kvx's BlockManager
        # issues from its admission and release loops).
        per_block, per_4_blocks = calls_of(1), calls_of(4)

        # An admission under memory pressure (block_manager.py:97-116, 290-302): the victims are saved, then
        # CPU entries are restored into those same blocks, waited for. Each restore chunk waits only for the
        # save kernel that read its destinations, so the restores' copies overlap the saves' transfers.
        victims_saved = timed(lambda: engine.save(sources, high, compute), "host link: recycle, saves alone")
        restored_alone = timed(lambda: engine.restore(low, sources, True, compute),
                               "host link: recycle, restores alone")

        def recycle():
            engine.save(sources, high, compute)
            engine.restore(low, sources, True, compute)

        recycled = timed(recycle, "host link: recycle, save victims then restore into them")
        recycle = {"staging_entries": max(1, min(_MAX_BATCH, _STAGING_BYTES // stride)),
                   "save_s": round(victims_saved, 5), "restore_s": round(restored_alone, 5),
                   "both_s": round(recycled, 5), "duplex_gbs": round(gbs(2 * link_bytes, recycled), 2),
                   "overlap_fraction": round((victims_saved + restored_alone - recycled)
                                             / min(victims_saved, restored_alone), 3)}
        engine.set_staging(save_staging, restore_staging, n)

        ceil_d2h = ceil_h2d = ceil_both = None
        if ceilings:
            # Ceiling: pinned hipMemcpyAsync each way, and both at once on the
            # engine's two streams (the runtime torch loaded), interleaved in pieces
            # (one multi-GB copy per stream does not always overlap with the other
            # direction); the best of several piece sizes is the ceiling.
            hip = ctypes.CDLL("libamdhip64.so.7")
            hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                           ctypes.c_void_p]
            flat_dev = torch.empty(link_bytes, dtype=torch.uint8, device=pool.device)
            flat_dev2 = torch.empty_like(flat_dev)
            host_a, host_b = slab.data_ptr(), slab.data_ptr() + n * stride
            s1, s2 = engine.save_stream.cuda_stream, engine.restore_stream.cuda_stream

            def pieces(piece):
                return [(off, min(piece, link_bytes - off)) for off in range(0, link_bytes, piece)]

            def d2h(piece):
                for off, size in pieces(piece):
                    assert hip.hipMemcpyAsync(host_a + off, flat_dev.data_ptr() + off, size, 2, s1) == 0

            def h2d(piece):
                for off, size in pieces(piece):
                    assert hip.hipMemcpyAsync(flat_dev2.data_ptr() + off, host_b + off, size, 1, s2) == 0

            def both_ways(piece):
                for (off, size) in pieces(piece):
                    assert hip.hipMemcpyAsync(host_a + off, flat_dev.data_ptr() + off, size, 2, s1) == 0
                    assert hip.hipMemcpyAsync(flat_dev2.data_ptr() + off, host_b + off, size, 1, s2) == 0

            piece_sizes = (8 << 20, 16 << 20, 32 << 20, 64 << 20, -(-link_bytes // 16))
            ceil_d2h = min(timed(lambda: d2h(p), f"memcpy d2h, {p} B pieces", {"d2h_copies": len(pieces(p))})
                           for p in piece_sizes)
            ceil_h2d = min(timed(lambda: h2d(p), f"memcpy h2d, {p} B pieces", {"h2d_copies": len(pieces(p))})
                           for p in piece_sizes)
            ceil_both = min(timed(lambda: both_ways(p), f"memcpy both, {p} B pieces",
                                  {"d2h_copies": len(pieces(p)), "h2d_copies": len(pieces(p))})
                            for p in piece_sizes)
        overlap = (save_s + restore_s - both_s) / min(save_s, restore_s)
        duplex = gbs(2 * link_bytes, both_s)
        out = {
            "bytes_per_direction": link_bytes,
            "save_d2h_gbs": round(gbs(link_bytes, save_s), 2),
            "restore_h2d_gbs": round(gbs(link_bytes, restore_s), 2),
            "duplex_gbs": round(duplex, 2),
            "overlap_fraction": round(overlap, 3),
            "peak_per_direction_gbs": PCIE_PEAK_GBS,
            "frac_duplex_of_spec": round(duplex / (2 * PCIE_PEAK_GBS), 3),
            "pin_seconds": round(pin_s, 2),
            "recycle": recycle,
            "logical_kv_gbs": round(2 * n * BF16_BLOCK_BYTES / both_s / 1e9, 2),
            "streams_concurrent": engine.streams_concurrent,
            "per_block_calls": per_block,
            "calls_of_4_blocks": per_4_blocks,
            "dma_copies_by_phase": copies,
        }
        if ceilings:
            out.update({
                "ceiling_memcpy_d2h_gbs": round(gbs(link_bytes, ceil_d2h), 2),
                "ceiling_memcpy_h2d_gbs": round(gbs(link_bytes, ceil_h2d), 2),
                "ceiling_memcpy_duplex_gbs": round(gbs(2 * link_bytes, ceil_both), 2),
                "frac_duplex_of_measured_ceiling": round(duplex / gbs(2 * link_bytes, ceil_both), 3),
            })
        return out
    finally:
        engine.close()


def gpu_pci_address(device_index: int = 0):
    """The GPU's PCI address ("0000:xx:yy.z") as the HIP runtime torch loaded reports it."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    buf = ctypes.create_string_buffer(64)
    hip.hipDeviceGetPCIBusId.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
    if hip.hipDeviceGetPCIBusId(buf, 64, device_index) != 0:
        return None
    return buf.value.decode().lower()


def pcie_path(bdf):
    """Negotiated and maximum link speed/width of the GPU's PCI function and every bridge above it (sysfs)."""
    import re

    if bdf is None:
        return []
    path = os.path.realpath(f"/sys/bus/pci/devices/{bdf}")
    hops = []
    while re.fullmatch(r"[0-9a-f]{4}:[0-9a-f]{2}:[0-9a-f]{2}\.[0-7]", os.path.basename(path)):
        hop = {"bdf": os.path.basename(path)}
        for key in ("current_link_speed", "current_link_width", "max_link_speed", "max_link_width"):
            try:
                hop[key] = Path(path, key).read_text().strip()
            except OSError:
                hop[key] = None
        hops.append(hop)
        path = os.path.dirname(path)
    return hops


def _cpu_list(text):
    """CPU ids of a sysfs cpulist ("0-3,8,10-11")."""
    cpus = set()
    for part in text.strip().split(","):
        if part:
            lo, _, hi = part.partition("-")
            cpus.update(range(int(lo), int(hi or lo) + 1))
    return cpus


def pages_by_node(address, maps_path="/proc/self/maps", numa_maps_path="/proc/self/numa_maps"):
    """{node: pages} of the mapping that holds `address`, from numa_maps (None if not found)."""
    try:
        start = None
        with open(maps_path) as maps:
            for line in maps:
                lo, hi = (int(x, 16) for x in line.split()[0].split("-"))
                if lo <= address < hi:
                    start = lo
                    break
        if start is None:
            return None
        with open(numa_maps_path) as numa:
            for line in numa:
                fields = line.split()
                if int(fields[0], 16) == start:
                    return {f[1:f.index("=")]: int(f[f.index("=") + 1:]) for f in fields
                            if f[0] == "N" and "=" in f and f[1:f.index("=")].isdigit()}
    except (OSError, ValueError):
        return None
    return None


def numa_placement(torch, bdf, sysfs="/sys"):
    """Where the host link's ends sit: the GPU's NUMA node (its PCI function), the nodes of the CPUs this
    process may run on, and the nodes holding the pages of a fresh pinned allocation (as the cache's slabs are
    made). -1 or None where the kernel does not say."""
    out = {"nodes": {}, "gpu_numa_node": None, "affinity_cpus_by_node": {}, "pinned_pages_by_node": None}
    try:
        node_dirs = sorted(p for p in Path(sysfs, "devices/system/node").glob("node[0-9]*"))
    except OSError:
        node_dirs = []
    affinity = os.sched_getaffinity(0)
    for d in node_dirs:
        try:
            cpus = _cpu_list(Path(d, "cpulist").read_text())
        except OSError:
            continue
        node = d.name[4:]
        out["nodes"][node] = len(cpus)
        mine = sorted(cpus & affinity)
        if mine:
            out["affinity_cpus_by_node"][node] = len(mine)
    if bdf:
        try:
            out["gpu_numa_node"] = int(Path(sysfs, "bus/pci/devices", bdf, "numa_node").read_text())
        except (OSError, ValueError):
            pass
    if torch is not None:
        probe = torch.ones(64 << 20, dtype=torch.uint8, pin_memory=True)
        out["pinned_pages_by_node"] = pages_by_node(probe.data_ptr())
        del probe
    return out


def host_inventory(torch):
    """What the CPU baseline and the host link run on (the reference records the same: bench/inventory.py:79-105)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        limit, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if limit != "max":
            quota = int(limit) / int(period)
    except (OSError, ValueError):
        pass
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = affinity if quota is None else max(1, min(affinity, int(quota)))

    def command(*argv):
        try:
            return subprocess.run(argv, capture_output=True, text=True, timeout=10, check=True).stdout
        except (OSError, subprocess.SubprocessError):
            return ""

    lscpu = {k.strip(): v.strip() for k, _, v in (line.partition(":") for line in command("lscpu").splitlines())}
    nproc = command("nproc").strip()
    bdf = gpu_pci_address(0)
    return {"nproc": int(nproc) if nproc.isdigit() else None, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": affinity, "cgroup_cpu_quota": quota, "cpu_model": model,
            "lscpu_model": lscpu.get("Model name"), "lscpu_cpus": lscpu.get("CPU(s)"),
            "lscpu_sockets": lscpu.get("Socket(s)"),
            "usable_cpus": usable, "torch_threads_default": torch.get_num_threads(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "gpu": torch.cuda.get_device_name(0),
            "gpu_pci": bdf, "pcie_path": pcie_path(bdf), "numa": numa_placement(torch, bdf)}


def headline_leg(torch, pool, layout, sources, dests, steps, warmup, label="headline"):
    """Config 2 end to end: each step saves the sources into pinned host slots and restores as many host entries
    into the destinations, overlapped on the copy engine's save and restore streams (the C ABI calls the cache
    makes: one kvx_cache_save and one kvx_cache_restore of 128 blocks)."""
    from kvx import ops
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    n = len(sources)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8, split=True)
    try:
        stride = engine.entry_stride
        slab = torch.empty(2 * n * stride, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(n * stride, dtype=torch.uint8, device=pool.device) for _ in range(2)]
        engine.add_slab(slab, 2 * n)
        engine.set_staging(*staging, n)
        compute = torch.cuda.current_stream(pool.device).cuda_stream
        restored_slots, saved_slots = list(range(n)), list(range(n, 2 * n))
        engine.save(sources, restored_slots, compute)  # the host entries the steps restore
        engine.synchronize()

        def step():
            engine.save(sources, saved_slots, compute)
            engine.restore(restored_slots, dests, False, compute)

        for _ in range(warmup):
            step()
        engine.synchronize()
        torch.cuda.synchronize()
        with marked(f"{label}: timed steps"):
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            engine.synchronize()
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - t0
        return {"elapsed": elapsed, "link_bytes_per_step": 2 * n * engine.logical_bytes,
                "streams_concurrent": engine.streams_concurrent}
    finally:
        engine.close()


def tp_rank_leg(torch, ops, scale_dtype, steps, warmup, tp=8, blocks=128):
    """Config 2 at one tensor-parallel rank's share of the pool.

    Under TP each rank's pool holds num_kv_heads // tp heads (model_runner.py:110): at TP=8 Qwen3-8B's pool is
    [2, 36, 320, 256, 1, 128] per rank, and each rank saves and restores its head slice of every block over its
    own host link. Same values, seeds and 128 + 128 blocks as the headline: the FP8 kernels with entries in HBM
    (per-launch algorithmic bytes as the headline's, for the rank's block), then the overlapped pinned-slab step.
    """
    from workloads import PoolShape, block_selection, fill_student_t

    shape = PoolShape(layers=36, num_blocks=320, kv_heads=8 // tp)
    pool = torch.empty(shape.shape, dtype=torch.bfloat16, device="cuda")
    fill_student_t(pool, seed=0)
    order = block_selection(shape.num_blocks, 2 * blocks, seed=1)
    sources, dests = order[:blocks], order[blocks:]
    layout = ops.pool_layout(pool, scale_dtype)
    k = kernel_leg(torch, ops, pool, sources, dests, scale_dtype, steps, warmup, block_bytes=shape.block_bytes_bf16,
                   label=f"tp{tp} rank kernel leg")
    h = headline_leg(torch, pool, layout, sources, dests, steps, warmup, label=f"tp{tp} rank")
    step_s = h["elapsed"] / steps
    link_gbs = h["link_bytes_per_step"] / step_s / 1e9
    kernels = {}
    for name in ("save", "restore"):
        gbs = k["hbm_bytes"] / (k[f"{name}_ms"] / 1000) / 1e9
        kernels[name] = {"ms": round(k[f"{name}_ms"], 4), "hbm_gbs": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    del pool
    return {"tp": tp, "pool": list(shape.shape), "blocks_saved": blocks, "blocks_restored": blocks,
            "block_bytes_bf16": shape.block_bytes_bf16, "entry_bytes": k["logical_entry"],
            "kernels": dict(kernels, algorithmic_bytes_per_launch=k["hbm_bytes"]),
            "pinned_step": {"ms": round(1000 * step_s, 4),
                            "logical_kv_gbs": round(2 * blocks * shape.block_bytes_bf16 / step_s / 1e9, 2),
                            "link_gbs": round(link_gbs, 2), "link_frac_of_spec": round(link_gbs / (2 * PCIE_PEAK_GBS), 4),
                            "streams_concurrent": h["streams_concurrent"]}}


def profiler_tool_loaded(maps_path="/proc/self/maps"):
    """The rocprofiler-sdk library mapped into this process, if one is (a rocprofv3 run loads it), else None."""
    try:
        with open(maps_path) as maps:
            for line in maps:
                if "librocprofiler-sdk" in line:
                    return line.split()[-1]
    except OSError:
        return None
    return None


# Copiers whose copies may still be in flight after a timed-out wait: their buffers and signals must outlive them.
_ABANDONED_COPIERS = []


class SdmaCopier:
    """Copies between a device buffer and pinned host memory on explicitly chosen SDMA engines, through HSA's
    hsa_amd_memory_async_copy_on_engine, bypassing the HIP runtime's choice of engine (it runs device-to-host
    hipMemcpyAsync copies as blit kernels). `unavailable` names why it cannot run here, if it cannot.

    The copier owns one hsa_init reference and every signal it creates. close() (or leaving a `with` block)
    destroys the signals and calls hsa_shut_down, so the process never ends with HSA state of the probe's
    making. A copy that fails to queue leaves no signal behind: the pieces queued before it are waited for
    first. A wait that times out leaves its copies possibly in flight, so their signals and buffers are then
    kept until the process ends, and HSA stays initialised.

    It refuses to run under a profiler tool (rocprofiler-sdk mapped into the process): a traced run that
    queued these copies ended in a segmentation fault during the tool's teardown, and the tracer intercepts
    exactly these HSA calls.
    """

    def __init__(self, torch, nbytes, piece=64 << 20):
        import re

        self.unavailable = None
        self.hsa = None
        self.abandoned = False
        self._live = []
        self.nbytes, self.piece = nbytes, piece
        tool = profiler_tool_loaded()
        if tool:
            self.unavailable = f"a profiler tool is loaded ({tool}); explicit SDMA copies are not run under it"
            return
        try:
            hsa = ctypes.CDLL("libhsa-runtime64.so.1")
        except OSError as error:
            self.unavailable = f"libhsa-runtime64 not loadable: {error}"
            return
        u64, u32 = ctypes.c_uint64, ctypes.c_uint32
        hsa.hsa_init.restype = ctypes.c_int
        hsa.hsa_shut_down.restype = ctypes.c_int
        hsa.hsa_iterate_agents.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hsa.hsa_agent_get_info.argtypes = [u64, ctypes.c_int, ctypes.c_void_p]
        hsa.hsa_signal_create.argtypes = [ctypes.c_int64, u32, ctypes.c_void_p, ctypes.POINTER(u64)]
        hsa.hsa_signal_destroy.argtypes = [u64]
        hsa.hsa_signal_load_scacquire.argtypes = [u64]
        hsa.hsa_signal_load_scacquire.restype = ctypes.c_int64
        hsa.hsa_signal_subtract_screlease.argtypes = [u64, ctypes.c_int64]
        hsa.hsa_amd_memory_copy_engine_status.argtypes = [u64, u64, ctypes.POINTER(u32)]
        hsa.hsa_amd_memory_async_copy_on_engine.argtypes = [ctypes.c_void_p, u64, ctypes.c_void_p, u64,
                                                            ctypes.c_size_t, u32, ctypes.c_void_p, u64, ctypes.c_int,
                                                            ctypes.c_bool]
        if hsa.hsa_init() != 0:
            self.unavailable = "hsa_init failed"
            return
        self.hsa = hsa
        HSA_AGENT_INFO_DEVICE, HSA_AMD_AGENT_INFO_BDFID = 17, 0xA006
        agents = {"cpu": [], "gpu": []}
        callback_type = ctypes.CFUNCTYPE(ctypes.c_int, u64, ctypes.c_void_p)

        def visit(agent, _):
            kind = u32()
            hsa.hsa_agent_get_info(agent, HSA_AGENT_INFO_DEVICE, ctypes.byref(kind))
            if kind.value == 0:
                agents["cpu"].append(agent)
            elif kind.value == 1:
                bdf = u32()
                hsa.hsa_agent_get_info(agent, HSA_AMD_AGENT_INFO_BDFID, ctypes.byref(bdf))
                agents["gpu"].append((agent, bdf.value))
            return 0

        callback = callback_type(visit)
        hsa.hsa_iterate_agents(ctypes.cast(callback, ctypes.c_void_p), None)
        address = gpu_pci_address(0)
        m = re.fullmatch(r"[0-9a-f]{4}:([0-9a-f]{2}):([0-9a-f]{2})\.([0-7])", address or "")
        want = (int(m.group(1), 16) << 8) | (int(m.group(2), 16) << 3) | int(m.group(3)) if m else None
        gpu = next((a for a, bdf in agents["gpu"] if bdf == want), None)
        if gpu is None and len(agents["gpu"]) == 1:
            gpu = agents["gpu"][0][0]  # the only GPU this process sees
        if gpu is None or not agents["cpu"]:
            self.unavailable = f"no HSA agent matches the GPU at {address} ({len(agents['gpu'])} GPU agents)"
            return
        self.cpu, self.gpu = agents["cpu"][0], gpu
        self.masks = {}
        for name, (dst, src) in {"d2h": (self.cpu, gpu), "h2d": (gpu, self.cpu)}.items():
            mask = u32()
            status = hsa.hsa_amd_memory_copy_engine_status(dst, src, ctypes.byref(mask))
            self.masks[name] = mask.value if status == 0 else 0
        engines = {name: [1 << i for i in range(16) if mask & (1 << i)] for name, mask in self.masks.items()}
        self.engines = {"d2h": engines["d2h"][:2]}
        self.engines["h2d"] = [e for e in engines["h2d"] if e not in self.engines["d2h"]][:2]
        if not self.engines["d2h"] or not self.engines["h2d"]:
            self.unavailable = f"not enough distinct SDMA engines (masks {self.masks})"
            return
        self.dev_src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        self.dev_dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        self.host_dst = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        self.host_src = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True)
        torch.cuda.synchronize()
        self.pieces = [(off, min(piece, nbytes - off)) for off in range(0, nbytes, piece)]

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def start(self, directions, spread=1):
        """Queues every piece of each direction ("d2h", "h2d"), alternating over `spread` engines per direction;
        returns the completion signals. If a piece fails to queue, the copies queued so far are waited for
        and every signal of the call is destroyed before the error is raised."""
        if self.unavailable or self.abandoned:
            raise RuntimeError(f"SDMA copier cannot queue copies: {self.unavailable or 'a wait timed out'}")
        hsa, signals = self.hsa, []
        try:
            for direction in directions:
                sig = ctypes.c_uint64()
                if hsa.hsa_signal_create(len(self.pieces), 0, None, ctypes.byref(sig)) != 0:
                    raise RuntimeError("hsa_signal_create failed")
                signals.append(sig.value)
                self._live.append(sig.value)
                engines = self.engines[direction][:spread]
                for i, (off, size) in enumerate(self.pieces):
                    engine = engines[i % len(engines)]
                    if direction == "d2h":
                        rc = hsa.hsa_amd_memory_async_copy_on_engine(self.host_dst.data_ptr() + off, self.cpu,
                                                                     self.dev_src.data_ptr() + off, self.gpu, size,
                                                                     0, None, sig.value, engine, True)
                    else:
                        rc = hsa.hsa_amd_memory_async_copy_on_engine(self.dev_dst.data_ptr() + off, self.gpu,
                                                                     self.host_src.data_ptr() + off, self.cpu, size,
                                                                     0, None, sig.value, engine, True)
                    if rc != 0:
                        # The pieces not queued never decrement the signal: take them off its count.
                        hsa.hsa_signal_subtract_screlease(sig.value, len(self.pieces) - i)
                        raise RuntimeError(f"hsa_amd_memory_async_copy_on_engine ({direction}) returned {rc}")
        except BaseException:
            if signals:
                self.wait(signals)  # copies already queued still write the buffers
            raise
        return signals

    def wait(self, signals, limit_s=30.0):
        """Waits for the signals to reach zero, then destroys them. On a timeout the copies may still run: the
        signals are kept and the copier takes no more work."""
        deadline = time.perf_counter() + limit_s
        while any(self.hsa.hsa_signal_load_scacquire(sig) > 0 for sig in signals):
            if time.perf_counter() > deadline:
                self.abandoned = True
                raise RuntimeError(f"SDMA copies did not finish within {limit_s} s")
            time.sleep(20e-6)
        for sig in signals:
            self.hsa.hsa_signal_destroy(sig)
            self._live.remove(sig)

    def run(self, directions, spread=1):
        t0 = time.perf_counter()
        self.wait(self.start(directions, spread))
        return time.perf_counter() - t0

    def close(self):
        """Destroys the remaining signals and balances hsa_init, unless a wait timed out (see the class)."""
        if self.hsa is None:
            return
        if self.abandoned:
            _ABANDONED_COPIERS.append(self)
            return
        for sig in self._live:
            self.hsa.hsa_signal_destroy(sig)
        self._live.clear()
        for name in ("dev_src", "dev_dst", "host_dst", "host_src"):
            self.__dict__.pop(name, None)
        hsa, self.hsa = self.hsa, None
        hsa.hsa_shut_down()


def sdma_probe(torch, nbytes, reps=3):
    """Plain DMA duplex over the host link on explicit SDMA engines: D2H alone, H2D alone, both at once, each on
    one engine and spread over two. GB/s, or why it could not run."""
    with SdmaCopier(torch, nbytes) as copier:
        if copier.unavailable:
            return {"skipped": copier.unavailable}
        out = {"bytes_per_direction": nbytes, "piece_bytes": copier.piece, "engines": copier.engines,
               "engine_masks": copier.masks}
        try:
            for name, directions, spread in (("d2h", ["d2h"], 1), ("h2d", ["h2d"], 1),
                                             ("duplex", ["d2h", "h2d"], 1), ("d2h_2_engines", ["d2h"], 2),
                                             ("h2d_2_engines", ["h2d"], 2),
                                             ("duplex_2_engines_each", ["d2h", "h2d"], 2)):
                best = min(copier.run(directions, spread) for _ in range(reps))
                out[f"{name}_gbs"] = round(len(directions) * nbytes / best / 1e9, 2)
        except RuntimeError as error:
            out["error"] = str(error)
        return out


def interference_leg(torch, nbytes=1 << 30, reps=20, kvx_kernels=None):
    """How a host-link copy slows HBM-bound kernels on another stream.

    The kernels: `reps` elementwise adds over 512 MiB of bf16 (torch), and
    each of `kvx_kernels` ({name: callable queuing kvx work on the current
    stream}), on a stream checked to run beside the copy stream. Each runs
    alone, then beside 1 GiB moved by the runtime's device-to-host
    hipMemcpyAsync (which it runs as blit kernels), its host-to-device copy
    (DMA), and an SDMA-engine device-to-host copy queued through HSA.
    """
    from kvx.engine.cpu_prefix_cache import _copy_streams

    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    (copy_stream, work_stream), concurrent = _copy_streams(torch.device("cuda", 0), 2)
    dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    a = torch.randn(1 << 28, device="cuda").to(torch.bfloat16)
    b = torch.empty_like(a)
    piece = 64 << 20
    copier = SdmaCopier(torch, nbytes)

    def adds():
        for _ in range(reps):
            torch.add(a, 1, out=b)

    def kernels_ms(start=None, finish=None, work=adds):
        torch.cuda.synchronize()
        handle = start() if start else None
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(work_stream):
            e0.record(work_stream)
            work()
            e1.record(work_stream)
        if finish:
            finish(handle)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def runtime_copy(kind):
        def start():
            for off in range(0, nbytes, piece):
                dst, src = (host, dev) if kind == 2 else (dev, host)
                assert hip.hipMemcpyAsync(dst.data_ptr() + off, src.data_ptr() + off, piece, kind,
                                          copy_stream.cuda_stream) == 0
        return start

    out = {"streams_concurrent": concurrent, "copy_bytes": nbytes,
           "sdma": copier.unavailable or "available"}
    with copier:
        for name, work in {f"{reps} x torch.add over 512 MiB bf16": adds, **(kvx_kernels or {})}.items():
            kernels_ms(work=work)
            res = {"alone_ms": round(kernels_ms(work=work), 3)}
            with marked(f"interference: {name} beside runtime D2H"):
                res["beside_runtime_d2h_ms"] = round(kernels_ms(runtime_copy(2), work=work), 3)
            with marked(f"interference: {name} beside runtime H2D"):
                res["beside_runtime_h2d_ms"] = round(kernels_ms(runtime_copy(1), work=work), 3)
            if not copier.unavailable:
                with marked(f"interference: {name} beside SDMA D2H"):
                    res["beside_sdma_d2h_ms"] = round(kernels_ms(lambda: copier.start(["d2h"]), copier.wait,
                                                                 work), 3)
            out[name] = res
    return out


def cpu_baseline_leg(torch, pool, sources, dests, scale_dtype, inventory, pairs=128, runs=5):
    """The reference's CPU path on this host: its torch codec and byte copies on CPU tensors, the branches
    CPUBlockCache takes for a CPU pool (cpu_prefix_cache.py:20-28, 323-326, 394-397).

    Threads: the CPUs the process may run on at once (affinity, capped by the
    cgroup quota). Each measurement is 1 warm-up and the median of `runs`
    runs (time.perf_counter). Samples: `pairs` of the Qwen3-8B workload's
    Student-t blocks (copied from the GPU pool) saved to FP8 and restored into
    other blocks, the same `pairs` in BF16 mode, and config 1 as written: 16
    N(0, 1) blocks of a 512-block Qwen3-0.6B host pool saved and restored into
    16 other seeded blocks. Only the blocks the workload touches are written;
    the rest of the 15 GB pool is allocated but never touched, so its pages
    are not materialised.
    """
    from workloads import QWEN3_0_6B, block_selection

    from oracle import torch_path

    threads = inventory["usable_cpus"]
    torch.set_num_threads(threads)
    _, layers, _, bs, heads, hd = pool.shape

    def median_s(fn):
        fn()
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return sorted(times)[runs // 2]

    def codec(host, src, dst, fmt_scale):
        entry = (len(src), 2, host.shape[1], *host.shape[3:])
        payload = torch.empty(entry, dtype=torch.float8_e4m3fn if fmt_scale else host.dtype)
        scale = torch.empty((*entry[:-1], 1), dtype=fmt_scale) if fmt_scale else None

        def save():
            for i, b in enumerate(src):
                torch_path.save_block(host, b, payload[i], None if scale is None else scale[i])

        def restore():
            for i, b in enumerate(dst):
                torch_path.restore_block(host, b, payload[i], None if scale is None else scale[i])

        return median_s(save), median_s(restore)

    host = torch.empty((2, layers, 2 * pairs, bs, heads, hd), dtype=pool.dtype)
    host[:, :, :pairs] = pool[:, :, sources[:pairs]].cpu()
    src, dst = list(range(pairs)), list(range(pairs, 2 * pairs))
    fp8_save, fp8_restore = codec(host, src, dst, scale_dtype)
    raw_save, raw_restore = codec(host, src, dst, None)
    del host
    small = torch.empty(QWEN3_0_6B.shape, dtype=torch.bfloat16)
    order = block_selection(QWEN3_0_6B.num_blocks, 32, seed=1)
    g = torch.Generator(device="cuda").manual_seed(0)
    for b in order:
        small[:, :, b] = torch.randn(small[:, :, b].shape, generator=g, device="cuda").to(torch.bfloat16).cpu()
    c1_save, c1_restore = codec(small, order[:16], order[16:], torch.float32)
    small_block = small[:, :, 0].numel() * 2
    del small
    logical = lambda n, per, s: round(n * per / s / 1e9, 3)  # noqa: E731
    value = logical(2 * pairs, BF16_BLOCK_BYTES, fp8_save + fp8_restore)
    return {
        "value": value,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{pairs} Qwen3-8B blocks of the bench's pool saved to FP8 ({str(scale_dtype)[6:]} scales) and "
                  f"restored into {pairs} others through torch's CPU codec (cpu_prefix_cache.py:20-28, 323-326, "
                  f"394-397); median of {runs} runs after a warm-up, save and restore timed separately",
        "fp8_qwen3_8b": {"blocks": pairs, "save_s": round(fp8_save, 4), "restore_s": round(fp8_restore, 4),
                         "save_gbs": logical(pairs, BF16_BLOCK_BYTES, fp8_save),
                         "restore_gbs": logical(pairs, BF16_BLOCK_BYTES, fp8_restore)},
        "bf16_qwen3_8b": {"blocks": pairs, "save_s": round(raw_save, 4), "restore_s": round(raw_restore, 4),
                          "save_gbs": logical(pairs, BF16_BLOCK_BYTES, raw_save),
                          "restore_gbs": logical(pairs, BF16_BLOCK_BYTES, raw_restore)},
        "fp8_qwen3_0_6b_16_blocks": {"pool": list(QWEN3_0_6B.shape), "save_s": round(c1_save, 4),
                                     "restore_s": round(c1_restore, 4),
                                     "logical_kv_gbs": logical(32, small_block, c1_save + c1_restore)},
        "threads_basis": "sched_getaffinity capped by the cgroup CPU quota",
        "torch_threads": torch.get_num_threads(),
        "host": {key: inventory.get(key) for key in ("nproc", "affinity_cpus", "cgroup_cpu_quota", "cpu_model",
                                                      "lscpu_model", "torch_threads_default", "omp_num_threads")},
        "runs": runs,
        "warmup_runs": 1,
    }


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the KV copy path is per GPU and this build runs on a single "
              f"MI355X (asked for --gpus {args.gpus}, WORLD_SIZE {world})", file=sys.stderr)
        sys.exit(2)

    import torch

    from kvx import ops
    from workloads import QWEN3_8B, block_selection, fill_student_t

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a ROCm GPU")
    device = torch.device("cuda", 0)
    scale_dtype = torch.float32 if args.scale == "fp32" else torch.bfloat16
    shape = QWEN3_8B.shape
    inventory = host_inventory(torch)
    log(f"pool {shape} bf16 on {inventory['gpu']} at {inventory['gpu_pci']}; {inventory['usable_cpus']} usable CPUs")
    log(f"PCIe path: {json.dumps(inventory['pcie_path'])}")
    pool = torch.empty(shape, dtype=torch.bfloat16, device=device)
    fill_student_t(pool, seed=0)
    torch.cuda.synchronize()
    order = block_selection(QWEN3_8B.num_blocks, 2 * args.blocks, seed=1)
    sources, dests = order[:args.blocks], order[args.blocks:]
    layout = ops.pool_layout(pool, scale_dtype)
    n = args.blocks

    log("config 2: saves to and restores from pinned host slabs, overlapped")
    h = headline_leg(torch, pool, layout, sources, dests, args.steps, args.warmup)
    ms_per_step = 1000 * h["elapsed"] / args.steps
    value = 2 * n * BF16_BLOCK_BYTES / (ms_per_step / 1000) / 1e9
    link_gbs = h["link_bytes_per_step"] / (ms_per_step / 1000) / 1e9
    log(f"step {ms_per_step:.3f} ms: {value:.1f} GB/s logical KV, {link_gbs:.2f} GB/s over the host link")

    k = kernel_leg(torch, ops, pool, sources, dests, scale_dtype, args.steps, args.warmup)
    save_gbs = k["hbm_bytes"] / (k["save_ms"] / 1000) / 1e9
    restore_gbs = k["hbm_bytes"] / (k["restore_ms"] / 1000) / 1e9
    dominant = "save" if k["save_ms"] >= k["restore_ms"] else "restore"
    achieved = min(save_gbs, restore_gbs)
    scale_flag = "true" if args.scale == "bf16" else "false"
    kernel_name = (f"fp8_save_kernel<128, 2, 128, {scale_flag}, false>" if dominant == "save"
                   else f"fp8_restore_kernel<128, 2, 64, {scale_flag}, false>")
    traffic, traffic_source = pmc_traffic(kernel_name)
    hbm_step_ms = 1000 * k["elapsed"] / args.steps
    log(f"entries in HBM: step {hbm_step_ms:.3f} ms; save {k['save_ms']:.3f} ms ({save_gbs:.0f} GB/s), "
        f"restore {k['restore_ms']:.3f} ms ({restore_gbs:.0f} GB/s)")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-8b-kv-fp8-save-restore-pinned-host-slabs",
            "pool": list(shape),
            "blocks_saved": n,
            "blocks_restored": n,
            "scale_dtype": args.scale,
            "storage": "bf16 pool -> e4m3fn payload + per-(token, kv-head) scale",
            "dtype_note": "the codec computes in fp32 (amax / 448, x / scale, code * scale); values are stored "
                          "as bf16 in the pool and e4m3fn + scale in the entries",
            "values": "bf16 0.5*t(df=4), 4 outlier channels x20 per (kv, layer, head)",
            "residency": "pool in HBM; saves write pinned host slabs (D2H), restores read pinned host slabs "
                         "(H2D); the two directions overlap on the save and restore streams",
        },
        "blocks_per_s": round(2 * n / (ms_per_step / 1000), 1),
        "host_link": {
            "bound": "pcie",
            "achieved": round(link_gbs, 2),
            "peak": 2 * PCIE_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(link_gbs / (2 * PCIE_PEAK_GBS), 4),
            "bytes_per_step": h["link_bytes_per_step"],
            "streams_concurrent": h["streams_concurrent"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "workload": f"the same {n} + {n} blocks with entries in HBM, one launch each, HIP events on the "
                        "launching stream",
        },
        "kernels": {
            "save": {"ms": round(k["save_ms"], 4), "hbm_gbs": round(save_gbs, 1),
                     "frac": round(save_gbs / HBM_PEAK_GBS, 4)},
            "restore": {"ms": round(k["restore_ms"], 4), "hbm_gbs": round(restore_gbs, 1),
                        "frac": round(restore_gbs / HBM_PEAK_GBS, 4)},
            "algorithmic_bytes_per_launch": k["hbm_bytes"],
            "hbm_resident_step": {"ms": round(hbm_step_ms, 4),
                                  "logical_kv_gbs": round(2 * n * BF16_BLOCK_BYTES / (hbm_step_ms / 1000) / 1e9, 1)},
        },
        "inventory": inventory,
    }
    if not args.skip_tp_rank:
        log("config 2 at one TP=8 rank's share of the pool")
        result["tp8_rank_shape"] = tp_rank_leg(torch, ops, scale_dtype, args.steps, args.warmup)
        log(f"tp8 rank: {json.dumps(result['tp8_rank_shape'])}")
    if not args.skip_store:
        log("store_kvcache leg")
        result["store_kvcache"] = store_leg(torch, ops, pool, concurrency=not args.skip_store_concurrency)
    if not args.skip_store_decode:
        log("store_kvcache decode leg")
        result["store_kvcache_decode"] = store_decode_leg(torch, ops, pool)
    if args.calibrate_copy:
        raw_layout = ops.pool_layout(pool)
        _, _, raw_stride = ops.entry_layout(raw_layout, ops.FORMAT_RAW)
        raw = torch.empty(n * raw_stride, dtype=torch.uint8, device=device)
        ops.save_blocks(pool, sources, [raw.data_ptr() + i * raw_stride for i in range(n)], ops.FORMAT_RAW)
        torch.cuda.synchronize()
        result["calibration_copy"] = {"kernel": "raw_copy_kernel", "read_bytes": n * BF16_BLOCK_BYTES,
                                      "write_bytes": n * BF16_BLOCK_BYTES}
        del raw
    if not args.skip_host_link:
        log("host link leg")
        legs = host_link_leg(torch, pool, layout, sources, dests, args.host_reps)
        link = result["host_link"]
        link["legs"] = legs
        ceiling = legs.get("ceiling_memcpy_duplex_gbs")
        if ceiling:
            link["measured_ceiling"] = ceiling
            link["frac_of_measured_ceiling"] = round(link_gbs / ceiling, 4)
        if not args.skip_sdma_probe:
            log("host link: explicit SDMA engines")
            link["sdma_probe"] = sdma_probe(torch, legs["bytes_per_direction"])
            log("host link: copies beside HBM-bound kernels")
            hbm_entries = torch.empty(n * k["entry_stride"], dtype=torch.uint8, device=device)
            entries = [hbm_entries.data_ptr() + i * k["entry_stride"] for i in range(n)]
            ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)
            link["interference"] = interference_leg(torch, kvx_kernels={
                f"kvx FP8 restore of {n} blocks (entries in HBM)":
                    lambda: ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, scale_dtype),
                f"kvx FP8 save of {n} blocks (entries in HBM)":
                    lambda: ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)})
            del hbm_entries
            log(f"interference: {json.dumps(link['interference'])}")
        log(f"host link legs: D2H {legs['save_d2h_gbs']}, H2D {legs['restore_h2d_gbs']}, duplex {legs['duplex_gbs']} "
            f"GB/s (memcpy ceiling {ceiling}); SDMA probe {json.dumps(link.get('sdma_probe'))}")
    if not args.skip_reference_gpu:
        log("reference torch codec on the GPU")
        result["reference_torch_gpu"] = reference_gpu_leg(torch, pool, sources, dests, scale_dtype, hbm_step_ms)
        if not args.skip_host_link:
            log("reference host path on the GPU")
            result["reference_torch_gpu"]["host_link"] = reference_link_leg(torch, pool, sources, dests, scale_dtype)
    if not args.skip_configs:
        log("bf16 leg")
        result["bf16_qwen3_8b"] = bf16_leg(torch, ops, pool, args.host_reps, link=not args.skip_host_link)
        log("qwen3-0.6b leg")
        result["fp8_qwen3_0_6b"] = qwen3_0_6b_leg(torch, ops, scale_dtype)
    if not args.skip_handoff:
        log("kv handoff leg")
        result["kv_handoff"] = handoff_leg(torch, pool)
    if not args.skip_microbench:
        log("copy-path microbench leg")
        result["microbench"] = microbench_leg(torch)
    if not args.skip_hybrid:
        log("hybrid calibration leg")
        result["hybrid_admission"] = hybrid_leg(torch, pool, scale_dtype)
    if not args.skip_agents:
        log("agent pressure leg")
        h2d_gbs = result["host_link"].get("legs", {}).get("restore_h2d_gbs")
        result["agent_pressure"] = agent_leg(torch, pool, scale_dtype, h2d_gbs)
    if not args.skip_cpu_baseline:
        log("cpu baseline leg")
        result["cpu_baseline"] = cpu_baseline_leg(torch, pool, sources, dests, scale_dtype, inventory)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
