"""The request record the block manager, scheduler and runners share.

A Sequence holds a request's tokens (prompt, then completion), how many of
them already have KV in the pool (num_cached_tokens), how many the current
step writes (num_scheduled_tokens), the pool blocks that hold them
(block_table) and, for a split admission, the token span being restored by
copy while its head is recomputed (restore_span). Runners compute slot
mappings from these fields and CPUBlockCache reads them, so they keep the
names of the reference's request record (nanovllm/engine/sequence.py:14-73).

The chained prefix hashes of the request's full blocks are cached on the
record (block_hashes) so an admission retried every step does not re-hash a
long waiting prompt; tokens only ever grow, so cached hashes stay valid.
"""

from dataclasses import dataclass
from enum import Enum
from itertools import count


@dataclass(frozen=True, slots=True)
class SamplingParams:
    """Per-request generation limits (nanovllm/sampling_params.py:5-13)."""

    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        if not (self.temperature == 0 or self.temperature > 1e-10):
            raise ValueError("temperature must be 0 (greedy) or greater than 1e-10")
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be at least 1")


class SequenceStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


_DEFAULT_PARAMS = SamplingParams()


class Sequence:
    """One request. `block_size` is the engine's KV block size (set by the engine)."""

    block_size = 256
    _ids = count()

    __slots__ = ("seq_id", "status", "token_ids", "num_prompt_tokens", "num_cached_tokens", "num_scheduled_tokens",
                 "is_prefill", "block_table", "restore_span", "temperature", "max_tokens", "ignore_eos",
                 "block_hashes")

    def __init__(self, token_ids, sampling_params: SamplingParams = _DEFAULT_PARAMS):
        tokens = list(token_ids)
        if not tokens:
            raise ValueError("a request needs at least one token")
        self.seq_id = next(Sequence._ids)
        self.status = SequenceStatus.WAITING
        self.token_ids = tokens
        self.num_prompt_tokens = len(tokens)
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table: list[int] = []
        self.restore_span: tuple[int, int] | None = None
        self.temperature = sampling_params.temperature
        self.max_tokens = sampling_params.max_tokens
        self.ignore_eos = sampling_params.ignore_eos
        # (chained hash, token list, token tuple) of leading full blocks, filled by the block manager.
        self.block_hashes: list[tuple[int, list[int], tuple[int, ...]]] = []

    @classmethod
    def resumed(cls, token_ids, num_prompt_tokens: int, sampling_params: SamplingParams) -> "Sequence":
        """A request rebuilt mid-completion (KV handoff): the first num_prompt_tokens are its prompt."""
        seq = cls(token_ids, sampling_params)
        if not 0 < num_prompt_tokens <= len(seq.token_ids):
            raise ValueError("num_prompt_tokens must be within the token list")
        seq.num_prompt_tokens = num_prompt_tokens
        return seq

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def last_token(self) -> int:
        return self.token_ids[-1]

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_blocks(self) -> int:
        """Blocks the tokens occupy (the last one possibly partial)."""
        return -(-len(self.token_ids) // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        return len(self.token_ids) - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        """Tokens of logical block i."""
        if not 0 <= i < self.num_blocks:
            raise IndexError(f"block {i} outside [0, {self.num_blocks})")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
