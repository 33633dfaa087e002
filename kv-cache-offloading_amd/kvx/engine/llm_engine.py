"""Engine facade over any model runner: request admission, steps, and the CPU-tier API.

Mirrors the public surface of nanovllm/engine/llm_engine.py that the copy path
serves: add_request, step / step_with_events, create_cpu_prefix_cache
(:85-110), prefetch_prefix (:112-126) and exit (:66-75). Model execution is
delegated to `model_runner.call("run", seqs, is_prefill) -> token ids`; the
runner also exposes `kv_cache` ([2, L, NB, BS, H, hd]), `world_size` and
`block_size`, as nanovllm's ModelRunner does. Loading weights, tokenisers and
tensor-parallel workers is the runner's business and outside this package.
"""

from dataclasses import dataclass, fields

import torch

from kvx.engine import kv_handoff
from kvx.engine.handoff_timing import PhaseTimer
from kvx.engine.cpu_prefix_cache import CPUBlockCache
from kvx.engine.scheduler import Scheduler, validate_scheduling_options
from kvx.engine.sequence import SamplingParams, Sequence


@dataclass(frozen=True)
class TokenEvent:
    """One new output token; seq_id is local to this engine."""

    seq_id: int
    output_index: int  # zero-based position within the completion
    token_id: int
    finished: bool


@dataclass(frozen=True)
class StepResult:
    """Finished outputs, signed work count (prefill tokens > 0, decode sequences < 0), new tokens."""

    outputs: list[tuple[int, list[int]]]
    num_tokens: int
    token_events: list[TokenEvent]


@dataclass
class EngineConfig:
    """Scheduling fields of nanovllm/config.py:22-40 the engine uses."""

    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    prefill_policy: str = "legacy"
    prefill_chunk_size: int = 512
    prefill_min_chunk_size: int = 1
    kv_eviction: str = "lru"

    def __post_init__(self):
        validate_scheduling_options(self.prefill_policy, self.prefill_chunk_size, self.prefill_min_chunk_size,
                                    self.max_num_batched_tokens, self.max_num_seqs)
        if self.kvcache_block_size % 256 != 0:
            raise ValueError("kvcache_block_size must be a multiple of 256")
        if self.kv_eviction not in ("lru", "mru"):
            raise ValueError("kv_eviction must be 'lru' or 'mru'")


class LLMEngine:

    def __init__(self, model_runner, tokenizer=None, **kwargs):
        names = {f.name for f in fields(EngineConfig)}
        config = EngineConfig(**{k: v for k, v in kwargs.items() if k in names})
        if config.num_kvcache_blocks <= 0:
            config.num_kvcache_blocks = model_runner.kv_cache.shape[2]
        Sequence.block_size = config.kvcache_block_size
        self.config = config
        self.model_runner = model_runner
        self.tokenizer = tokenizer
        self.scheduler = Scheduler(config)
        self._cpu_prefix_cache: CPUBlockCache | None = None
        self._detached_requests: dict[int, Sequence] = {}

    def exit(self):
        cache = getattr(self, "_cpu_prefix_cache", None)
        if cache is not None:
            cache.close()
        for seq_id in tuple(self._detached_requests):
            self.release_detached_request(seq_id)
        call = getattr(self.model_runner, "call", None)
        if call is not None:
            call("exit")

    def add_request(self, prompt, sampling_params: SamplingParams) -> int:
        """Enqueue a request (token ids, or text with a tokenizer); return its sequence ID."""
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("text prompts need a tokenizer")
            prompt = self.tokenizer.encode(prompt)
        seq = Sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq.seq_id

    def create_cpu_prefix_cache(self, max_bytes: int, *, automatic: bool = False, save_on_release: bool = False,
                                preallocate: bool = False, prefetch: bool = False, split_streams: bool = False,
                                fp8: bool = False, hybrid: tuple[float, float, float] | None = None,
                                scale_dtype=None) -> CPUBlockCache:
        """This engine's bounded CPU block cache (llm_engine.py:85-110); see CPUBlockCache for the options."""
        existing = getattr(self, "_cpu_prefix_cache", None)
        if existing is not None and not existing.closed:
            raise RuntimeError("this engine already has a CPU prefix cache")
        cache = CPUBlockCache(self.model_runner, self.scheduler.block_manager, max_bytes,
                              automatic=automatic, save_on_release=save_on_release, preallocate=preallocate,
                              prefetch=prefetch, split_streams=split_streams, fp8=fp8, hybrid=hybrid,
                              scale_dtype=scale_dtype)
        self._cpu_prefix_cache = cache
        return cache

    def prefetch_prefix(self, prefix) -> int:
        """Hint that a request starting with `prefix` will arrive; restore its CPU hits now (:112-126).

        Never runs while requests wait for admission, so hints never take
        blocks they need. Pass the same Sequence when repeating a hint.
        """
        if self.scheduler.waiting:
            return 0
        if not isinstance(prefix, Sequence):
            prefix = Sequence(prefix)
        return self.scheduler.block_manager.prefetch(prefix, reserve=len(self.scheduler.running))

    # -- KV handoff between engines (llm_engine.py:127-173) -------------------

    def detach_request(self, seq_id: int) -> kv_handoff.KVSnapshot:
        """Export a running request's KV and take it out of scheduling; its blocks stay owned."""
        if seq_id in self._detached_requests:
            raise ValueError(f"request {seq_id} is already detached")
        seq = next((seq for seq in self.scheduler.running if seq.seq_id == seq_id), None)
        if seq is None:
            raise ValueError(f"request {seq_id} is not running at a handoff boundary")
        timer = PhaseTimer("detach_request", seq_id=seq_id)
        with timer.phase("export"):
            snapshot = kv_handoff.export_kv(self.model_runner, seq)
        with timer.phase("unschedule"):
            self._detached_requests[seq_id] = seq
            self.scheduler.running.remove(seq)
        timer.finish()
        return snapshot

    def release_detached_request(self, seq_id: int):
        seq = self._detached_requests[seq_id]
        self.scheduler.block_manager.deallocate(seq)
        del self._detached_requests[seq_id]

    def reattach_request(self, seq_id: int) -> int:
        seq = self._detached_requests[seq_id]
        self.scheduler.running.append(seq)
        del self._detached_requests[seq_id]
        return seq.seq_id

    def resume_request(self, snapshot: kv_handoff.KVSnapshot) -> int:
        """Import a snapshot as a running request; admit it only once its KV is on the device."""
        manager = self.scheduler.block_manager
        timer = PhaseTimer("resume_request")
        seq = None
        try:
            with timer.phase("import"):
                seq = kv_handoff.import_kv(self.model_runner, manager, snapshot)
            with timer.phase("cuda_sync"):
                device = self.model_runner.kv_cache.device
                if device.type == "cuda":
                    torch.cuda.synchronize(device)
            with timer.phase("admit"):
                self.scheduler.running.append(seq)
        except Exception as error:
            timer.abort(error)
            if seq is not None:
                manager.deallocate(seq)
            raise
        timer.finish(seq_id=seq.seq_id)
        return seq.seq_id

    def step(self):
        result = self._step(emit_events=False)
        return result.outputs, result.num_tokens

    def step_with_events(self) -> StepResult:
        """One batch; each new token reported once (the final prefill chunk emits output_index 0)."""
        return self._step(emit_events=True)

    def _step(self, *, emit_events: bool) -> StepResult:
        seqs, is_prefill = self.scheduler.schedule()
        previous = [seq.num_completion_tokens for seq in seqs] if emit_events else []
        num_tokens = sum(seq.num_scheduled_tokens for seq in seqs) if is_prefill else -len(seqs)
        token_ids = self.model_runner.call("run", seqs, is_prefill)
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        outputs = [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished]
        events = [TokenEvent(seq.seq_id, seq.num_completion_tokens - 1, seq.last_token, seq.is_finished)
                  for seq, before in zip(seqs, previous) if seq.num_completion_tokens > before]
        return StepResult(outputs, num_tokens, events)

    def is_finished(self):
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, use_tqdm: bool = True) -> list[dict]:
        """Run prompts to completion; outputs in submission order as {"text", "token_ids"} (llm_engine.py:206-234).

        `sampling_params` is one SamplingParams for every prompt or one per prompt.
        Text needs the engine's tokenizer.
        """
        from time import perf_counter

        from tqdm.auto import tqdm

        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        ids = [self.add_request(prompt, sp) for prompt, sp in zip(prompts, sampling_params)]
        done: dict[int, list[int]] = {}
        bar = tqdm(total=len(ids), desc="Generating", dynamic_ncols=True, disable=not use_tqdm)
        while not self.is_finished():
            started = perf_counter()
            finished, num_tokens = self.step()
            rate = abs(num_tokens) / max(perf_counter() - started, 1e-9)
            bar.set_postfix({"Prefill" if num_tokens > 0 else "Decode": f"{int(rate)}tok/s"})
            for seq_id, token_ids in finished:
                done[seq_id] = token_ids
                bar.update(1)
        bar.close()
        decode = self.tokenizer.decode if self.tokenizer is not None else None
        return [{"text": decode(done[i]) if decode else None, "token_ids": done[i]} for i in ids]


def prefill_slot_mapping(seqs, block_size: int) -> list[int]:
    """Pool slot of every scheduled prefill token (model_runner.py:156-166): block_table[pos // BS] * BS + pos % BS."""
    slots = []
    for seq in seqs:
        if not seq.block_table:  # warm-up batches own no blocks
            continue
        start = seq.num_cached_tokens
        for pos in range(start, start + seq.num_scheduled_tokens):
            slots.append(seq.block_table[pos // block_size] * block_size + pos % block_size)
    return slots


def decode_slot_mapping(seqs, block_size: int, padded_to: int | None = None) -> list[int]:
    """Slot of each sequence's last token (model_runner.py:186); -1 pads a captured graph's batch (:211)."""
    slots = [seq.block_table[-1] * block_size + seq.last_block_num_tokens - 1 for seq in seqs]
    if padded_to is not None:
        slots += [-1] * (padded_to - len(slots))
    return slots
