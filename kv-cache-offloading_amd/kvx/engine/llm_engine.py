"""A model-free serving engine around the copy path: requests, steps, the CPU tier and KV handoff.

The engine owns a Scheduler (and its BlockManager) and delegates model
execution to a runner: `runner.call("run", seqs, is_prefill)` returns one
sampled token per request; the runner also exposes `kv_cache` (the
[2, L, NB, BS, H, hd] pool), `block_size` and `world_size`, as the
reference's ModelRunner does. The CPU-tier and handoff entry points keep
the reference engine's signatures (nanovllm/engine/llm_engine.py:85-173),
so callers switch engines without changes. Tokenising, weights, sampling and
tensor parallelism are the runner's business.
"""

from dataclasses import dataclass, fields

import torch

from kvx.engine import kv_handoff
from kvx.engine.cpu_prefix_cache import CPUBlockCache
from kvx.engine.scheduler import Scheduler
from kvx.engine.sequence import SamplingParams, Sequence


@dataclass
class EngineConfig:
    """The scheduling fields of the reference's Config (nanovllm/config.py:22-66) this engine uses."""

    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    kv_eviction: str = "lru"

    def __post_init__(self):
        for name in ("max_num_batched_tokens", "max_num_seqs", "kvcache_block_size"):
            value = getattr(self, name)
            if type(value) is not int or value < 1:
                raise ValueError(f"{name} must be a positive integer")
        if self.kvcache_block_size % 256:
            raise ValueError("kvcache_block_size must be a multiple of 256")
        if self.kv_eviction not in ("lru", "mru"):
            raise ValueError("kv_eviction must be 'lru' or 'mru'")


class LLMEngine:
    """Engine over `model_runner`; keyword arguments that are EngineConfig fields configure it, others are ignored."""

    def __init__(self, model_runner, **kwargs):
        known = {f.name for f in fields(EngineConfig)}
        config = EngineConfig(**{k: v for k, v in kwargs.items() if k in known})
        if config.num_kvcache_blocks <= 0:
            config.num_kvcache_blocks = model_runner.kv_cache.shape[2]
        Sequence.block_size = config.kvcache_block_size
        self.config = config
        self.model_runner = model_runner
        self.scheduler = Scheduler(config)
        self._cpu_prefix_cache: CPUBlockCache | None = None
        self._detached: dict[int, Sequence] = {}

    # -- requests and steps -------------------------------------------------------

    def add_request(self, prompt, sampling_params: SamplingParams) -> int:
        """Queue a request given as token ids; returns its sequence id."""
        if isinstance(prompt, str):
            raise TypeError("this engine takes token ids; tokenise text before add_request")
        seq = Sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq.seq_id

    def step(self) -> tuple[list[tuple[int, list[int]]], int]:
        """One batch: (finished (seq_id, completion tokens) pairs, prefill tokens > 0 or -decode requests)."""
        seqs, is_prefill = self.scheduler.schedule()
        work = sum(seq.num_scheduled_tokens for seq in seqs) if is_prefill else -len(seqs)
        token_ids = self.model_runner.call("run", seqs, is_prefill)
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        return [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished], work

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def exit(self):
        """Close the CPU tier, release detached requests and stop the runner."""
        if self._cpu_prefix_cache is not None:
            self._cpu_prefix_cache.close()
        for seq_id in list(self._detached):
            self.release_detached_request(seq_id)
        call = getattr(self.model_runner, "call", None)
        if call is not None:
            call("exit")

    # -- CPU tier (llm_engine.py:85-126) -----------------------------------------------

    def create_cpu_prefix_cache(self, max_bytes: int, *, automatic: bool = False, save_on_release: bool = False,
                                preallocate: bool = False, prefetch: bool = False, split_streams: bool = False,
                                fp8: bool = False, hybrid: tuple[float, float, float] | None = None,
                                scale_dtype: torch.dtype | None = None) -> CPUBlockCache:
        """This engine's bounded CPU block cache; the options are CPUBlockCache's. One open cache per engine."""
        if self._cpu_prefix_cache is not None and not self._cpu_prefix_cache.closed:
            raise RuntimeError("this engine already has a CPU prefix cache")
        self._cpu_prefix_cache = CPUBlockCache(
            self.model_runner, self.scheduler.block_manager, max_bytes, automatic=automatic,
            save_on_release=save_on_release, preallocate=preallocate, prefetch=prefetch,
            split_streams=split_streams, fp8=fp8, hybrid=hybrid, scale_dtype=scale_dtype)
        return self._cpu_prefix_cache

    def prefetch_prefix(self, prefix, *, defer: bool = False) -> int:
        """Client hint that a request starting with `prefix` (token ids or a Sequence) arrives soon.

        Restores its CPU hits into free blocks beyond one per running request
        and returns how many it started; nothing while requests wait for
        admission, so a hint never takes blocks they need. Pass the same
        Sequence when repeating a hint (its block hashes are kept on it).

        defer=True keeps a hint given while requests wait (replacing one kept
        before) instead of dropping it. The next step that admits them starts
        it right after their admissions, before the model runs, so the
        hint's restores overlap that step's compute rather than following it.
        The call then returns 0. A hint the engine can start now is started
        now, whatever `defer` says.
        """
        if self.scheduler.waiting and not defer:
            return 0
        seq = prefix if isinstance(prefix, Sequence) else Sequence(prefix)
        if self.scheduler.waiting:
            self.scheduler.prefetch_hint = seq
            return 0
        return self.scheduler.block_manager.prefetch(seq, reserve=len(self.scheduler.running))

    # -- KV handoff (llm_engine.py:128-173) ------------------------------------------------

    def detach_request(self, seq_id: int, *, fp8: bool = False,
                       scale_dtype: torch.dtype = torch.float32) -> kv_handoff.KVSnapshot:
        """Export a running request's KV and stop scheduling it; its blocks stay allocated until released."""
        if seq_id in self._detached:
            raise ValueError(f"request {seq_id} is already detached")
        seq = next((s for s in self.scheduler.running if s.seq_id == seq_id), None)
        if seq is None:
            raise ValueError(f"request {seq_id} is not running at a handoff boundary")
        snapshot = kv_handoff.export_kv(self.model_runner, seq, fp8=fp8, scale_dtype=scale_dtype)
        self.scheduler.running.remove(seq)
        self._detached[seq_id] = seq
        return snapshot

    def release_detached_request(self, seq_id: int):
        """Free a detached request's blocks (its KV now lives elsewhere)."""
        self.scheduler.block_manager.deallocate(self._detached.pop(seq_id))

    def reattach_request(self, seq_id: int) -> int:
        """Resume scheduling a detached request here (the handoff was abandoned)."""
        seq = self._detached.pop(seq_id)
        self.scheduler.running.append(seq)
        return seq.seq_id

    def resume_request(self, snapshot: kv_handoff.KVSnapshot) -> int:
        """Import a snapshot as a running request; it is scheduled only once its KV is in the pool."""
        seq = kv_handoff.import_kv(self.model_runner, self.scheduler.block_manager, snapshot)
        self.scheduler.running.append(seq)
        return seq.seq_id
