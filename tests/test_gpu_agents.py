"""Config 5: agent pressure on the Qwen3-8B pool through the whole engine (store_kvcache, FP8 saves,
restores and prefetches on split streams under slot reuse), verified block by block."""

from contextlib import nullcontext

import pytest
import torch

from kvx.engine.cpu_prefix_cache import CPUBlockCache
from kvx.engine.llm_engine import LLMEngine
from workloads import QWEN3_8B, SyntheticKVRunner, run_agent_pressure

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("copy_calls", ["batched", "per_block"])
def test_config5_agent_pressure_restores_the_right_bytes(gpu, monkeypatch, copy_calls):
    """per_block: one engine call per save and restore, as the reference's BlockManager issues them."""
    if copy_calls == "per_block":
        monkeypatch.setattr(CPUBlockCache, "coalesce", lambda self: nullcontext())
    pool = torch.zeros(QWEN3_8B.shape, dtype=torch.bfloat16, device=gpu)
    engine = LLMEngine(SyntheticKVRunner(pool), max_num_batched_tokens=16384, max_num_seqs=4, eos=-1,
                       kvcache_block_size=256, num_kvcache_blocks=QWEN3_8B.num_blocks)
    cache = engine.create_cpu_prefix_cache(8 << 30, automatic=True, prefetch=True, split_streams=True, fp8=True,
                                           scale_dtype=torch.float32)
    # Batched calls: every full block of every finished request; one call per block: every 8th.
    result = run_agent_pressure(engine, agents=4, context=32768, turns=12, append=2048, verify=True,
                                verify_stride=1 if copy_calls == "batched" else 8)
    print(result, f"{result.link_gbs:.1f} GB/s over the run")
    assert result.saved_blocks > 0 and result.restored_blocks > 0 and result.prefetched_blocks > 0
    # Deferred hints: most restores are prefetches that overlap the previous request's compute.
    assert result.prefetched_blocks > result.restored_blocks // 2
    assert result.blocks_fp8_round_trip > 0 and result.blocks_checked > result.blocks_fp8_round_trip
    engine.exit()
    assert cache.closed
