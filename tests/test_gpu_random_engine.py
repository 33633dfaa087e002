"""Seeded request streams through the whole engine on the GPU, every finished request's blocks verified.

LLMEngine with the synthetic KV runner (store_kvcache writes K/V that are a function of each token and its
position) and a real CPUBlockCache on libkvx: requests drawn from documents that share leading blocks arrive at
random steps, so admissions hit GPU blocks, restore CPU entries (waited, split or prefetched), recycle and save
victims, and decode into fresh blocks; hints are started at once or, deferred, after a step's admissions. When a
request finishes, each of its published full blocks must hold
exactly the KV its tokens and positions define, or that KV's FP8 round trip when the block came back from an
FP8 entry. A restore from the wrong slot, a block read before its restore landed or overwritten before its save
read it, shows up as neither.
"""

import random
from contextlib import nullcontext

import pytest
import torch

from kvx import ops
from kvx.engine.cpu_prefix_cache import CPUBlockCache
from kvx.engine.llm_engine import LLMEngine
from kvx.engine.sequence import SamplingParams
from workloads import SyntheticKVRunner, expected_block

pytestmark = pytest.mark.gpu

BS = 256


def holds(pool, block_id, tokens, start, fp8, scale_dtype) -> str | None:
    """'exact' or 'fp8' if the block holds the synthetic KV of `tokens` at `start` (or its FP8 round trip)."""
    expect = expected_block(pool, tokens, start)
    got = pool[:, :, block_id]
    if torch.equal(got.view(torch.int16), expect.view(torch.int16)):
        return "exact"
    if fp8:
        payload = torch.empty(expect.shape, dtype=torch.float8_e4m3fn, device=pool.device)
        scale = torch.empty((*expect.shape[:-1], 1), dtype=scale_dtype, device=pool.device)
        ops.fp8_quantize(expect, payload, scale)
        back = torch.empty_like(expect)
        ops.fp8_dequantize(payload, scale, back)
        if torch.equal(got.view(torch.int16), back.view(torch.int16)):
            return "fp8"
    return None


def run_stream(gpu, seed, fp8, split, batched, options, monkeypatch, heads=2, head_dim=128,
               scale_dtype=torch.float32):
    rng = random.Random(seed)
    num_blocks = rng.randint(8, 14)
    pool = torch.zeros((2, 2, num_blocks, BS, heads, head_dim), dtype=torch.bfloat16, device=gpu)
    engine = LLMEngine(SyntheticKVRunner(pool), max_num_batched_tokens=rng.choice([512, 1024, 4096]),
                       max_num_seqs=rng.randint(1, 4), eos=-1, kvcache_block_size=BS,
                       num_kvcache_blocks=num_blocks, kv_eviction=options.get("eviction", "lru"))
    scale_dtype = scale_dtype if fp8 else None
    if not batched:
        monkeypatch.setattr(CPUBlockCache, "coalesce", lambda self: nullcontext())
    rows = 2 * 2 * BS * heads
    entry = rows * (head_dim + scale_dtype.itemsize if fp8 else 2 * head_dim)  # bytes per CPU entry
    cache = engine.create_cpu_prefix_cache(rng.randint(3, 12) * entry, automatic=True, split_streams=split, fp8=fp8,
                                           scale_dtype=scale_dtype, prefetch=options.get("prefetch", False),
                                           save_on_release=options.get("save_on_release", False),
                                           hybrid=options.get("hybrid"))
    manager = engine.scheduler.block_manager
    documents = []
    for d in range(4):
        shared = documents[rng.randrange(len(documents))][:rng.randint(1, 2)] if documents and rng.random() < 0.6 else []
        documents.append(shared + [10_000 * (seed + 1) + 100 * d + i for i in range(rng.randint(1, 5) - len(shared))])
    prompts, counts = {}, {"exact": 0, "fp8": 0, "requests": 0}
    try:
        for step in range(60):
            for _ in range(rng.choice([0, 0, 1, 1, 2])):
                doc = rng.choice(documents)
                tokens = [v for v in doc[:rng.randint(1, len(doc))] for _ in range(BS)]
                tokens += [20_000 + step] * (rng.randint(0, BS - 1) if rng.random() < 0.7 else 0)
                if len(tokens) // BS + 2 >= num_blocks:
                    continue
                seq_id = engine.add_request(tokens, SamplingParams(temperature=0, max_tokens=rng.randint(1, 3),
                                                                   ignore_eos=True))
                prompts[seq_id] = tokens
                if options.get("prefetch") and rng.random() < 0.3:
                    if options.get("defer_hints"):
                        # A likely later request: the engine starts it after this step's admissions.
                        hint = rng.choice(documents)
                        engine.prefetch_prefix([v for v in hint for _ in range(BS)] + [1], defer=True)
                    else:
                        engine.prefetch_prefix(tokens)
            if engine.is_finished():
                continue
            finished, _ = engine.step()
            for seq_id, completion in finished:
                counts["requests"] += 1
                tokens = prompts.pop(seq_id) + completion
                h = -1
                for i in range(len(tokens) // BS):
                    block = tokens[i * BS:(i + 1) * BS]
                    h = manager.compute_hash(block, h)
                    block_id = manager.hash_to_block_id.get(h)
                    if block_id is None:
                        break
                    cache.before_block_use(block_id)
                    kind = holds(pool, block_id, block, i * BS, fp8, scale_dtype)
                    assert kind, (f"seed {seed} step {step}: block {i} of request {seq_id} (GPU block {block_id}) "
                                  "holds neither its KV nor the FP8 round trip of it")
                    counts[kind] += 1
        stats = dict(cache.stats, prefetched_blocks=cache.prefetched_blocks)
    finally:
        engine.exit()
    return counts, stats


OPTIONS = [pytest.param({}, id="plain"), pytest.param({"prefetch": True, "save_on_release": True}, id="prefetch"),
           pytest.param({"eviction": "mru", "prefetch": True}, id="mru"),
           pytest.param({"prefetch": True, "defer_hints": True, "save_on_release": True}, id="deferred"),
           pytest.param({"hybrid": (2e-4, 1e-6, 0.0), "save_on_release": True}, id="hybrid")]


@pytest.mark.parametrize("options", OPTIONS)
@pytest.mark.parametrize("fp8,split,batched", [(True, True, True), (True, False, False), (False, True, False),
                                               (False, False, True)])
def test_random_request_streams_keep_every_block_intact(gpu, fp8, split, batched, options, monkeypatch):
    totals = {"exact": 0, "fp8": 0, "requests": 0, "restored": 0, "saved": 0, "prefetched": 0}
    for seed in range(8):
        counts, stats = run_stream(gpu, seed, fp8, split, batched, options, monkeypatch)
        for key in ("exact", "fp8", "requests"):
            totals[key] += counts[key]
        totals["restored"] += stats["restored_blocks"]
        totals["saved"] += stats["saved_blocks"]
        totals["prefetched"] += stats["prefetched_blocks"]
    print(totals)
    assert totals["requests"] > 0 and totals["saved"] > 0 and totals["restored"] > 0
    if options.get("defer_hints"):
        assert totals["prefetched"] > 0  # deferred hints started after admissions
    if fp8:
        assert totals["fp8"] > 0  # some verified blocks came back from FP8 entries


@pytest.mark.parametrize("heads,head_dim,scale_dtype", [(4, 64, torch.float32), (1, 96, torch.float32),
                                                        (2, 128, torch.bfloat16), (1, 256, torch.bfloat16),
                                                        (1, 128, torch.float32)])  # last: a TP=8 rank of Qwen3-8B
@pytest.mark.parametrize("fp8", [True, False], ids=["fp8", "bf16"])
def test_random_request_streams_on_other_head_shapes_and_scales(gpu, heads, head_dim, scale_dtype, fp8, monkeypatch):
    # head_dim 96 takes the generic kernels (one thread per row) and staged restores only.
    totals = {"exact": 0, "fp8": 0, "requests": 0}
    for seed in range(4):
        counts, _ = run_stream(gpu, seed, fp8, True, True, {"prefetch": True, "save_on_release": True},
                               monkeypatch, heads, head_dim, scale_dtype)
        for key in totals:
            totals[key] += counts[key]
    print(totals)
    assert totals["requests"] > 0 and (totals["fp8"] > 0 or not fp8)
