"""GPU block accounting for the paged KV pool, and the caller of the CPU tier's hooks.

The pool has `num_blocks` physical blocks of `block_size` tokens. A block is
*published* while its chained prefix hash maps to it in `hash_to_block_id`;
a published block that no request references stays in the free order as a
GPU prefix hit until it is recycled. A CPU tier (CPUBlockCache, or any object
with the same duck-typed hooks) attached as `_cpu_prefix_cache` is told:

  recycling a published block    _preserve_before_recycle(hash), before the
                                 hash is dropped; then before_block_reuse(id)
                                 unless the new contents are copied in by a
                                 prefetch or manual restore
  releasing a published block    _preserve_on_release(hash)
  taking a reference on a hit    before_block_use(id)
  planning an admission          _entry_for(hash, tokens) (a pure lookup)
  admitting or prefetching a     _copy_entry(entry, id, wait): waited on
  CPU hit                        admission, unwaited after a hybrid split and
                                 for prefetches
  prefilling up to a split span  before_block_use(id) for each block of the span

These calls, their order and their arguments are what the reference's
BlockManager issues (nanovllm/engine/block_manager.py:97-183, 202-237,
266-347), so a cache written for one works under the other;
tests/test_hook_contract.py replays scenarios recorded from the reference and
requires identical traces.

How this module is built:
- the free order is an insertion-ordered set (constant-time removal and
  move-to-back);
- which idle block is recycled next is a policy object (_Lru, _Mru); the MRU
  policy keeps its own ledger of when and where each block was released, and
  the idle hits a prefetch keeps for a waiting request;
- an admission is planned first (_Plan: the prefix hits it uses, the split,
  the fresh positions) without touching the pool, then carried out under a
  journal that drops every reference it took if a copy raises;
- the chained hashes of a request's full blocks are computed once and kept
  on the request (Sequence.block_hashes); lookups and publication read them.

When the tier has coalesce() (kvx's CPUBlockCache), the admission, prefetch
and release loops run inside it, so their copies reach the copy engine as
batches; the order of hook calls is unchanged.
"""

from collections.abc import Callable, Iterable, Sequence as TokenSequence
from contextlib import nullcontext
from dataclasses import dataclass
from functools import partial
from struct import Struct
from typing import NamedTuple

import xxhash

from kvx.engine.sequence import Sequence

_HASH_LIMIT = 1 << 64

# Packers of n little-endian int64s, by n: a block's tokens are packed in one
# call (3.7 us for 256 tokens, against 11 us through a numpy array).
_PACKERS: dict[int, Struct] = {}
_MAX_PACKERS = 64


def plan_split(cpu_blocks: int, block_size: int, restore_s_per_block: float,
               recompute_s_per_token: float, recompute_s_per_token2: float) -> int:
    """Leading CPU-hit blocks to recompute while the others restore (block_manager.py:9-23).

    Recomputing the head overlaps restoring the tail, so the admission costs
    the slower of the two: max(recompute(k * block_size), (cpu_blocks - k) *
    restore_s_per_block) with recompute(t) = t * recompute_s_per_token +
    t^2 * recompute_s_per_token2. Returns the smallest minimising k.
    """
    a, b = recompute_s_per_token, recompute_s_per_token2

    def admission_s(k: int) -> float:
        t = k * block_size
        return max(t * a + t * t * b, (cpu_blocks - k) * restore_s_per_block)

    costs = [admission_s(k) for k in range(cpu_blocks + 1)]
    return costs.index(min(costs))


class Block:
    """Metadata of one physical block. `hash` is -1 unless the block was published."""

    __slots__ = ("block_id", "ref_count", "hash", "token_ids")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []

    def update(self, hash: int, token_ids: list[int]):
        self.hash = hash
        self.token_ids = token_ids


class FreeOrder:
    """Idle block ids in recycle order (front first): an insertion-ordered set.

    Membership, removal, append and move-to-back are O(1). It also offers the
    deque operations callers of the reference's free list use (index 0 and
    -1, appendleft, popleft, extend).
    """

    __slots__ = ("_ids",)

    def __init__(self, ids: Iterable[int] = ()):
        self._ids: dict[int, None] = dict.fromkeys(ids)

    def __len__(self):
        return len(self._ids)

    def __bool__(self):
        return bool(self._ids)

    def __iter__(self):
        return iter(self._ids)

    def __contains__(self, block_id):
        return block_id in self._ids

    def __getitem__(self, i: int) -> int:
        if i == 0 and self._ids:
            return next(iter(self._ids))
        if i == -1 and self._ids:
            return next(reversed(self._ids))
        return list(self._ids)[i]

    def __repr__(self):
        return f"FreeOrder({list(self._ids)})"

    def append(self, block_id: int):
        if block_id in self._ids:
            raise ValueError(f"block {block_id} is already free")
        self._ids[block_id] = None

    def appendleft(self, block_id: int):
        if block_id in self._ids:
            raise ValueError(f"block {block_id} is already free")
        self._ids = {block_id: None, **self._ids}

    def extend(self, block_ids: Iterable[int]):
        for block_id in block_ids:
            self.append(block_id)

    def remove(self, block_id: int):
        del self._ids[block_id]

    def move_to_back(self, block_id: int):
        del self._ids[block_id]
        self._ids[block_id] = None

    def popleft(self) -> int:
        block_id = next(iter(self._ids))
        del self._ids[block_id]
        return block_id

    def clear(self):
        self._ids.clear()


class _Lru:
    """Recycles the front of the free order: released blocks queue at the back."""

    def choose(self, manager: "BlockManager") -> int:
        return manager._free[0]

    def released(self, block_ids: list[int]):
        pass

    def keep(self, block_ids: Iterable[int]):
        pass

    def keep_also(self, block_id: int):
        pass

    def unkeep(self, block_id: int | None = None):
        pass


class _Mru(_Lru):
    """Recycles what will likely be needed last.

    First a free block that no prefix can hit again. Otherwise the idle hit
    released most recently, the tail of that release first (highest release
    number, then highest position in the releasing request's block table),
    skipping hits a prefetch keeps for a waiting request: the agent that
    finished last will likely return last, so it loses its context first.
    A block never released ranks lowest; ties go to the front of the order.
    """

    def __init__(self):
        self.release_count = 0
        self.rank: dict[int, tuple[int, int]] = {}
        self.kept: set[int] = set()

    def choose(self, manager: "BlockManager") -> int:
        best, best_rank = None, None
        for block_id in manager._free:
            if not manager._is_hit(block_id):
                return block_id
            if block_id in self.kept:
                continue
            rank = self.rank.get(block_id, (0, 0))
            if best_rank is None or rank > best_rank:
                best, best_rank = block_id, rank
        return manager._free[0] if best is None else best

    def released(self, block_ids: list[int]):
        self.release_count += 1
        for position, block_id in enumerate(block_ids):
            self.rank[block_id] = (self.release_count, position)

    def keep(self, block_ids: Iterable[int]):
        self.kept = set(block_ids)

    def keep_also(self, block_id: int):
        self.kept.add(block_id)

    def unkeep(self, block_id: int | None = None):
        if block_id is None:
            self.kept.clear()
        else:
            self.kept.discard(block_id)


class PrefixHit(NamedTuple):
    """One leading full block of a request found in the pool (block_id) or in the CPU tier (entry)."""

    index: int
    hash: int
    tokens: list[int]
    block_id: int | None
    entry: object | None


@dataclass
class _Plan:
    """What an admission will do, decided before the pool changes.

    `hits` are the leading cached blocks it uses. CPU hits from `split` on
    are restored; the `split` leading ones (all CPU hits) are recomputed with
    fresh blocks, as are the positions after the hits.
    """

    hits: list[PrefixHit]
    split: int
    num_blocks: int

    @property
    def gpu_hits(self) -> list[PrefixHit]:
        return [hit for hit in self.hits if hit.block_id is not None]

    @property
    def restores(self) -> list[PrefixHit]:
        return [hit for hit in self.hits if hit.block_id is None and hit.index >= self.split]

    @property
    def fresh(self) -> list[int]:
        return [*range(self.split), *range(len(self.hits), self.num_blocks)]


class _Journal:
    """The references an admission took, dropped again (newest first) if it raises.

    `as_release`: the rollback counts as a release of the blocks taken, in
    the order taken, for the MRU policy (as deallocating a partial table
    does).
    """

    def __init__(self, manager: "BlockManager", as_release: bool = False):
        self.manager = manager
        self.as_release = as_release
        self.taken: list[int] = []

    def __enter__(self):
        return self

    def __exit__(self, kind, error, trace):
        if kind is not None:
            if self.as_release:
                self.manager._policy.released(self.taken)
            for block_id in reversed(self.taken):
                self.manager._release_block(block_id)
        return False

    def share(self, hit: PrefixHit) -> int:
        self.manager._acquire_block(hit.block_id)
        self.taken.append(hit.block_id)
        return hit.block_id

    def restore(self, hit: PrefixHit, wait: bool) -> int:
        manager = self.manager
        block_id = manager._allocate_block()
        self.taken.append(block_id)
        if wait:
            manager._cpu_prefix_cache._copy_entry(hit.entry, block_id)
        else:
            manager._cpu_prefix_cache._copy_entry(hit.entry, block_id, wait=False)
        manager._publish(block_id, hit.hash, hit.tokens)
        return block_id

    def fresh(self) -> int:
        block_id = self.manager._allocate_block()
        self.taken.append(block_id)
        return block_id


class BlockManager:
    """Allocation, prefix caching and CPU-tier hooks for one pool. `eviction`: "lru" or "mru"."""

    def __init__(self, num_blocks: int, block_size: int, eviction: str = "lru"):
        if eviction not in ("lru", "mru"):
            raise ValueError("eviction must be 'lru' or 'mru'")
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.block_size = block_size
        self.eviction = eviction
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self._free = FreeOrder(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self._cpu_prefix_cache = None
        # Set by the scheduler while the head of the waiting queue cannot be admitted.
        self.admission_blocked = False
        self._policy = _Mru() if eviction == "mru" else _Lru()
        self._last_prefetch = None  # (request, free blocks) of the last prefetch attempt

    @property
    def free_block_ids(self) -> FreeOrder:
        return self._free

    @free_block_ids.setter
    def free_block_ids(self, ids: Iterable[int]):
        self._free = FreeOrder(ids)

    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1) -> int:
        """Chained block hash: xxh64 of the previous block's hash (8 bytes, little-endian; omitted for the
        first block) followed by the int64 token ids (block_manager.py:67-73). CPU entries are keyed by it."""
        n = len(token_ids)
        packer = _PACKERS.get(n)
        if packer is None:
            packer = Struct(f"<{n}q")
            if len(_PACKERS) < _MAX_PACKERS:
                _PACKERS[n] = packer
        head = b"" if prefix == -1 else prefix.to_bytes(8, "little")
        return xxhash.xxh64_intdigest(head + packer.pack(*token_ids))

    # -- one block at a time ------------------------------------------------------

    def _is_hit(self, block_id: int) -> bool:
        """Whether the block is published: the index maps its hash back to it."""
        h = self.blocks[block_id].hash
        return h != -1 and self.hash_to_block_id.get(h) == block_id

    def _publish(self, block_id: int, h: int, tokens: list[int]):
        self.blocks[block_id].update(h, tokens)
        self.hash_to_block_id[h] = block_id

    def _allocate_block(self, order_writes: bool = True) -> int:
        """Take the policy's victim for a new owner (one reference, no contents) and return its id.

        A published victim is offered to the CPU tier first; if that raises,
        nothing has changed. With order_writes, later writes on the caller's
        stream wait for copies still reading or writing the block; a restore
        into the block orders itself instead.
        """
        block_id = self._policy.choose(self)
        block = self.blocks[block_id]
        assert block.ref_count == 0, f"free block {block_id} is referenced"
        tier = self._cpu_prefix_cache
        if self._is_hit(block_id):
            if tier is not None:
                tier._preserve_before_recycle(block.hash)
            del self.hash_to_block_id[block.hash]
        if order_writes and tier is not None:
            tier.before_block_reuse(block_id)
        self._free.remove(block_id)
        self._policy.unkeep(block_id)
        block.ref_count, block.hash, block.token_ids = 1, -1, []
        self.used_block_ids.add(block_id)
        return block_id

    def _free_block(self, block_id: int):
        """The last reference is gone: the block joins the back of the free order (a hit may be saved now)."""
        self.used_block_ids.remove(block_id)
        self._free.append(block_id)
        tier = self._cpu_prefix_cache
        if tier is not None and self._is_hit(block_id):
            tier._preserve_on_release(self.blocks[block_id].hash)

    def _acquire_block(self, block_id: int):
        """A reference on a GPU hit. Readers wait for any restore still copying into it (also when shared:
        another request's split span may be copying it)."""
        block = self.blocks[block_id]
        if not block.ref_count:
            self._free.remove(block_id)
            self.used_block_ids.add(block_id)
        if self._cpu_prefix_cache is not None:
            self._cpu_prefix_cache.before_block_use(block_id)
        block.ref_count += 1

    def _release_block(self, block_id: int):
        block = self.blocks[block_id]
        block.ref_count -= 1
        if not block.ref_count:
            self._free_block(block_id)

    def _batched(self):
        """The tier's coalesce() context, if it has one (copies are then issued as batches)."""
        coalesce = getattr(self._cpu_prefix_cache, "coalesce", None)
        return coalesce() if coalesce is not None else nullcontext()

    # -- prefix lookup ----------------------------------------------------------

    def _block_hashes(self, seq: Sequence, count: int):
        """(hash, token list, token tuple) of the request's first `count` full blocks, cached on the request.

        Tokens only ever grow, so the cached entries stay valid; an admission
        retried every step does not hash a long waiting prompt again.
        """
        known = seq.block_hashes
        prev = known[-1][0] if known else -1
        while len(known) < count:
            tokens = seq.block(len(known))
            prev = self.compute_hash(tokens, prev)
            known.append((prev, tokens, tuple(tokens)))
        return known

    def _lookup(self, seq: Sequence) -> list[PrefixHit]:
        """The request's leading full blocks found on the GPU or in the CPU tier, up to the first miss.

        The last block is never a hit (its last token must be computed), so
        at most num_blocks - 1. Nothing is copied or changed.
        """
        hits = []
        tier = self._cpu_prefix_cache
        for i, (h, tokens, key) in enumerate(self._block_hashes(seq, seq.num_blocks - 1)):
            block_id = self.hash_to_block_id.get(h)
            if block_id is not None:
                block = self.blocks[block_id]
                if block.hash != h or block.token_ids != tokens:
                    break  # a hash collision: treat as a miss
                hits.append(PrefixHit(i, h, tokens, block_id, None))
                continue
            entry = tier._entry_for(h, key) if tier is not None else None
            if entry is None:
                break
            hits.append(PrefixHit(i, h, tokens, None, entry))
        return hits

    def _blocks_to_take(self, seq: Sequence, hits: list[PrefixHit]) -> int:
        """Free blocks an admission consumes: every position except hits that other requests already hold."""
        held = sum(1 for hit in hits if hit.block_id is not None and hit.block_id in self.used_block_ids)
        return seq.num_blocks - held

    def _plan(self, seq: Sequence, num_cached_blocks: int) -> _Plan:
        hits = self._lookup(seq)
        if not 0 <= num_cached_blocks <= len(hits):
            raise ValueError("requested prefix is no longer available")
        hits = hits[:num_cached_blocks]
        if len(self._free) < self._blocks_to_take(seq, hits):
            raise MemoryError("not enough free KV blocks to admit the request")
        tier = self._cpu_prefix_cache
        split = 0
        if tier is not None and tier.hybrid is not None:
            # Only the CPU-only run before the first GPU hit can be split, and
            # a split reaching that GPU hit would restore nothing.
            lead = next((hit.index for hit in hits if hit.block_id is not None), len(hits))
            split = plan_split(lead, self.block_size, *tier.hybrid)
            if split == lead < len(hits):
                split = 0
        if split == len(hits):  # recomputing the whole prefix is cheapest
            return _Plan([], 0, seq.num_blocks)
        return _Plan(hits, split, seq.num_blocks)

    # -- admission ----------------------------------------------------------------

    def can_allocate(self, seq: Sequence) -> int:
        """Leading cached blocks the request can reuse, or -1 if it cannot be admitted now."""
        hits = self._lookup(seq)
        return -1 if len(self._free) < self._blocks_to_take(seq, hits) else len(hits)

    def allocate(self, seq: Sequence, num_cached_blocks: int):
        """Give the request its block table, reusing its first `num_cached_blocks` cached blocks.

        GPU hits are referenced first, so nothing taken afterwards can recycle
        them. CPU hits are restored into recycled blocks and published, waited
        for on the caller's stream unless a hybrid split recomputes the head
        (the restored span is then pending until finish_restore_span). The
        other positions get fresh blocks. On any failure every reference
        taken is dropped and the error propagates.
        """
        assert not seq.block_table, "request already has blocks"
        plan = self._plan(seq, num_cached_blocks)
        self._policy.unkeep()
        table = [-1] * seq.num_blocks
        with _Journal(self) as journal:
            for hit in plan.gpu_hits:
                table[hit.index] = journal.share(hit)
            with self._batched():
                for hit in plan.restores:
                    table[hit.index] = journal.restore(hit, wait=not plan.split)
                for index in plan.fresh:
                    table[index] = journal.fresh()
        seq.block_table = table
        cached = len(plan.hits) * self.block_size
        if plan.split:
            seq.num_cached_tokens = 0
            seq.restore_span = (plan.split * self.block_size, cached)
        else:
            seq.num_cached_tokens = cached

    def finish_restore_span(self, seq: Sequence):
        """The head of a split admission is prefilled: skip the restored span; its first reads wait for it."""
        start, end = seq.restore_span
        assert seq.num_cached_tokens == start, "the head is not prefilled yet"
        seq.num_cached_tokens, seq.restore_span = end, None
        for block_id in seq.block_table[start // self.block_size:end // self.block_size]:
            self._cpu_prefix_cache.before_block_use(block_id)

    def deallocate(self, seq: Sequence):
        """Release the request's blocks, last block first (the MRU policy notes where each one sat)."""
        self._policy.released(seq.block_table)
        with self._batched():
            for block_id in reversed(seq.block_table):
                self._release_block(block_id)
        seq.block_table.clear()
        seq.num_cached_tokens = 0
        seq.restore_span = None

    def allocate_for_resume(self, seq: Sequence, num_cached_tokens: int):
        """Fresh blocks for a request whose KV is copied in (KV handoff); the one uncached token decodes next.

        A pending token at a block boundary gets its block from may_append on
        that decode step, not here. Blocks are published after their copy.
        """
        if seq.block_table or not 0 < num_cached_tokens == len(seq) - 1:
            raise ValueError("resume needs an empty block table and one uncached token")
        needed = -(-num_cached_tokens // self.block_size)
        if len(self._free) < needed:
            raise MemoryError("not enough free KV blocks to resume")
        with _Journal(self, as_release=True) as journal:
            table = [journal.fresh() for _ in range(needed)]
        seq.block_table = table
        seq.num_cached_tokens = num_cached_tokens

    # -- decode growth and publication -------------------------------------------

    def _opens_block(self, seq: Sequence) -> bool:
        """Whether the request's newest token is the first of a block (it needs one more block)."""
        return len(seq) % self.block_size == 1

    def can_append(self, seq: Sequence) -> bool:
        """Whether the next decode step's token has a block."""
        return bool(self._free) or not self._opens_block(seq)

    def may_append(self, seq: Sequence):
        if self._opens_block(seq):
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq: Sequence):
        """Publish the blocks this step fills (tokens [num_cached, num_cached + num_scheduled)), under the
        request's chained block hashes."""
        first = seq.num_cached_tokens // self.block_size
        stop = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        if first == stop:
            return
        for i, (h, tokens, _) in enumerate(self._block_hashes(seq, stop)[first:stop], first):
            self._publish(seq.block_table[i], h, tokens)

    # -- restores outside admission --------------------------------------------------

    def restore_cached_block(self, prefix_hash: int, token_ids: TokenSequence[int],
                             copy_to_block: Callable[[int], None]) -> int:
        """Copy one full prefix block into an idle GPU block and publish it; returns its id.

        An existing GPU hit is returned without a copy. The destination is
        recycled without write ordering: `copy_to_block` must order its copy
        after pending work itself and make later readers wait (the CPU
        tier's restore stream does both). Either way the block ends idle (a
        published hit, or, if the copy raised, unpublished and free) and the
        error propagates; an idle victim it recycled stays evicted. Call
        between steps.
        """
        tokens = list(token_ids)
        if type(prefix_hash) is not int or not 0 <= prefix_hash < _HASH_LIMIT or len(tokens) != self.block_size:
            raise ValueError("restore requires a valid prefix hash and one full block")
        known = self.hash_to_block_id.get(prefix_hash)
        if known is not None:
            if self.blocks[known].hash != prefix_hash or self.blocks[known].token_ids != tokens:
                raise ValueError("prefix hash has conflicting token metadata")
            return known
        if not self._free:
            raise MemoryError("not enough free KV blocks to restore a prefix")
        block_id = self._allocate_block(order_writes=False)
        try:
            copy_to_block(block_id)
        except BaseException:
            self._release_block(block_id)
            raise
        self._publish(block_id, prefix_hash, tokens)
        self._release_block(block_id)
        return block_id

    def prefetch(self, seq: Sequence, reserve: int = 0) -> int:
        """Start background restores of a waiting request's CPU hits; returns how many were started.

        Restored blocks become idle GPU hits, so the admission skips their
        copies. Uses only free blocks beyond `reserve` (kept for running
        requests' growth) and never recycles the request's own idle GPU hits,
        which move to the back of the free order and are kept from MRU
        recycling. Needs a tier with prefetch_enabled; does nothing when
        called again with the same request and free-block count. Call
        between steps.
        """
        tier = self._cpu_prefix_cache
        if tier is None or not tier.prefetch_enabled:
            return 0
        attempt = (seq.seq_id, len(self._free))
        if attempt == self._last_prefetch:
            return 0
        self._last_prefetch = attempt
        hits = self._lookup(seq)
        own_idle = [hit.block_id for hit in hits
                    if hit.block_id is not None and self.blocks[hit.block_id].ref_count == 0]
        room = len(self._free) - reserve - len(own_idle)
        wanted = [hit for hit in hits if hit.entry is not None][:max(room, 0)]
        if not wanted:
            return 0
        for block_id in own_idle:
            self._free.move_to_back(block_id)
        self._policy.keep(own_idle)
        with self._batched():
            for hit in wanted:
                copy = partial(tier._copy_entry, hit.entry, wait=False)
                self._policy.keep_also(self.restore_cached_block(hit.hash, hit.tokens, copy))
        tier._prefetched_blocks += len(wanted)
        return len(wanted)
