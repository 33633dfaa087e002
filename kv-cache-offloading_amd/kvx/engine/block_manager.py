"""Paged KV block allocator with chained prefix hashes and CPU-tier hooks.

This is the caller surface of the copy path: it decides which GPU blocks are
saved before recycling, which CPU hits are restored on admission or
prefetched, and when compute must wait for a copy. It follows
nanovllm/engine/block_manager.py (line citations below) hook for hook, so a
CPUBlockCache from kvx.engine.cpu_prefix_cache (or any object with the same
duck-typed hooks) plugs in unchanged.
"""

from collections import deque
from contextlib import nullcontext
from collections.abc import Callable, Sequence as TokenSequence

import numpy as np
import xxhash

from kvx.engine.sequence import Sequence


def plan_split(cpu_blocks: int, block_size: int, restore_s_per_block: float,
               recompute_s_per_token: float, recompute_s_per_token2: float) -> int:
    """Leading CPU-hit blocks to recompute while the rest restore (block_manager.py:9-23).

    Returns the smallest k in [0, cpu_blocks] minimising
    max(recompute(k * block_size), (cpu_blocks - k) * restore_s_per_block) with
    recompute(t) = t * recompute_s_per_token + t^2 * recompute_s_per_token2.
    """
    best_k, best_cost = 0, None
    for k in range(cpu_blocks + 1):
        tokens = k * block_size
        recompute = tokens * recompute_s_per_token + tokens * tokens * recompute_s_per_token2
        cost = max(recompute, (cpu_blocks - k) * restore_s_per_block)
        if best_cost is None or cost < best_cost:
            best_k, best_cost = k, cost
    return best_k


class Block:
    """One physical GPU block (block_manager.py:26-44)."""

    __slots__ = ("block_id", "ref_count", "hash", "token_ids", "release_gen", "seq_index")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []
        # Generation of the last owner release and the block's index there (MRU order).
        self.release_gen = 0
        self.seq_index = 0

    def update(self, hash: int, token_ids: list[int]):
        self.hash = hash
        self.token_ids = token_ids

    def reset(self):
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int, eviction: str = "lru"):
        if eviction not in ("lru", "mru"):
            raise ValueError("eviction must be 'lru' or 'mru'")
        self.block_size = block_size
        self.eviction = eviction
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self._cpu_prefix_cache = None
        self._last_prefetch = None
        self._release_gen = 0
        # Idle blocks a blocked request's prefetch keeps (consulted by MRU eviction).
        self._protected: set[int] = set()
        # Set by the scheduler while the head waiting request cannot be admitted.
        self.admission_blocked = False

    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1) -> int:
        """xxh64 of the previous block's hash (8 bytes LE) then the int64 token ids (:67-73)."""
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.array(token_ids).tobytes())
        return h.intdigest()

    def _is_published(self, block: Block) -> bool:
        return block.hash != -1 and self.hash_to_block_id.get(block.hash) == block.block_id

    def _victim(self) -> int:
        """Next free block to recycle (:78-95): the oldest for LRU; for MRU
        unpublished blocks first, then the latest release's blocks, tail first."""
        if self.eviction == "lru":
            return self.free_block_ids[0]
        best_key, best_id = None, None
        for block_id in self.free_block_ids:
            block = self.blocks[block_id]
            if not self._is_published(block):
                return block_id
            if block_id in self._protected:
                continue
            key = (block.release_gen, block.seq_index)
            if best_key is None or key > best_key:
                best_key, best_id = key, block_id
        return best_id if best_id is not None else self.free_block_ids[0]

    def _allocate_block(self, order_writes: bool = True) -> int:
        """Recycle a free block (:97-116). A published victim is saved to the
        CPU tier before its hash is dropped; a save failure leaves it free and
        indexed. order_writes makes the caller's stream wait for pending copies."""
        block_id = self._victim()
        block = self.blocks[block_id]
        assert block.ref_count == 0
        if self._is_published(block):
            if self._cpu_prefix_cache is not None:
                self._cpu_prefix_cache._preserve_before_recycle(block.hash)
            del self.hash_to_block_id[block.hash]
        if order_writes and self._cpu_prefix_cache is not None:
            self._cpu_prefix_cache.before_block_reuse(block_id)
        if self.free_block_ids[0] == block_id:
            self.free_block_ids.popleft()
        else:
            self.free_block_ids.remove(block_id)
        self._protected.discard(block_id)
        block.reset()
        self.used_block_ids.add(block_id)
        return block_id

    def _deallocate_block(self, block_id: int):
        """Return a block to the free list; an idle published block may be saved now (:118-127)."""
        block = self.blocks[block_id]
        assert block.ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)
        if self._cpu_prefix_cache is not None and self._is_published(block):
            self._cpu_prefix_cache._preserve_on_release(block.hash)

    def _acquire_block(self, block_id: int):
        """Take a reference on a GPU hit; readers wait for a pending restore into it (:129-137)."""
        block = self.blocks[block_id]
        if block.ref_count == 0:
            self.free_block_ids.remove(block_id)
            self.used_block_ids.add(block_id)
        if self._cpu_prefix_cache is not None:
            self._cpu_prefix_cache.before_block_use(block_id)
        block.ref_count += 1

    def _release_block(self, block_id: int):
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:
            self._deallocate_block(block_id)

    def restore_cached_block(self, prefix_hash: int, token_ids: TokenSequence[int],
                             copy_to_block: Callable[[int], None]) -> int:
        """Reserve, populate, then publish one full idle prefix block (:145-183).

        An existing GPU hit is returned without copying. On copy failure the
        destination returns to the free list unpublished and the error
        propagates; an idle victim it recycled stays evicted.
        """
        tokens = list(token_ids)
        if (type(prefix_hash) is not int or not 0 <= prefix_hash < 2**64
                or len(tokens) != self.block_size):
            raise ValueError("restore requires a valid prefix hash and one full block")
        existing = self.hash_to_block_id.get(prefix_hash)
        if existing is not None:
            block = self.blocks[existing]
            if block.hash != prefix_hash or block.token_ids != tokens:
                raise ValueError("prefix hash has conflicting token metadata")
            return existing
        if not self.free_block_ids:
            raise MemoryError("not enough free KV blocks to restore a prefix")
        block_id = self._allocate_block(order_writes=False)
        block = self.blocks[block_id]
        try:
            copy_to_block(block_id)
            block.update(prefix_hash, tokens)
            self.hash_to_block_id[prefix_hash] = block_id
        except BaseException:
            if self.hash_to_block_id.get(prefix_hash) == block_id:
                del self.hash_to_block_id[prefix_hash]
            block.hash, block.token_ids = -1, []
            raise
        finally:
            block.ref_count = 0
            self._deallocate_block(block_id)
        return block_id

    def _full_block_hashes(self, seq: Sequence, count: int):
        """Memoised (chained hash, token list, token tuple) of a sequence's leading blocks (:185-200)."""
        memo = getattr(seq, "_block_hash_memo", None)
        if memo is None:
            memo = seq._block_hash_memo = []
        h = memo[-1][0] if memo else -1
        for i in range(len(memo), count):
            token_ids = seq.block(i)
            h = self.compute_hash(token_ids, h)
            memo.append((h, token_ids, tuple(token_ids)))
        return memo

    def _batched_copies(self):
        """The cache's coalesce() context (restores handed over as batches), if it has one."""
        coalesce = getattr(self._cpu_prefix_cache, "coalesce", None)
        return coalesce() if coalesce is not None else nullcontext()

    def prefetch(self, seq: Sequence, reserve: int = 0) -> int:
        """Start background restores of a waiting request's CPU hits (:202-237); returns how many.

        Uses only free blocks beyond `reserve` and this request's own idle
        hits, never recycling the latter. Throttled while nothing changed.
        """
        cache = self._cpu_prefix_cache
        if cache is None or not cache.prefetch_enabled:
            return 0
        key = (seq.seq_id, len(self.free_block_ids))
        if key == self._last_prefetch:
            return 0
        self._last_prefetch = key
        prefix = self._prefix_blocks(seq)
        own_idle = [block_id for _, _, block_id, _ in prefix
                    if block_id is not None and self.blocks[block_id].ref_count == 0]
        budget = len(self.free_block_ids) - reserve - len(own_idle)
        if budget <= 0 or all(entry is None for *_, entry in prefix):
            return 0
        # Recycle other idle blocks first: this request's hits go to the back.
        for block_id in own_idle:
            self.free_block_ids.remove(block_id)
            self.free_block_ids.append(block_id)
        self._protected = set(own_idle)
        started = 0
        with self._batched_copies():
            for h, token_ids, block_id, entry in prefix:
                if started == budget:
                    break
                if entry is None:
                    continue
                target = self.restore_cached_block(
                    h, token_ids, lambda target, e=entry: cache._copy_entry(e, target, wait=False))
                self._protected.add(target)
                started += 1
        cache._prefetched_blocks += started
        return started

    def _prefix_blocks(self, seq: Sequence):
        """Leading contiguous GPU hits (block id) and CPU hits (entry); pure lookup (:239-256)."""
        prefix = []
        memo = self._full_block_hashes(seq, seq.num_blocks - 1)
        for i in range(seq.num_blocks - 1):
            h, token_ids, token_tuple = memo[i]
            block_id = self.hash_to_block_id.get(h)
            if block_id is not None:
                block = self.blocks[block_id]
                if block.hash != h or block.token_ids != token_ids:
                    break
                prefix.append((h, token_ids, block_id, None))
                continue
            cache = self._cpu_prefix_cache
            entry = cache._entry_for(h, token_tuple) if cache is not None else None
            if entry is None:
                break
            prefix.append((h, token_ids, None, entry))
        return prefix

    def _blocks_needed(self, seq: Sequence, prefix) -> int:
        return seq.num_blocks - sum(block_id in self.used_block_ids for _, _, block_id, _ in prefix)

    def can_allocate(self, seq: Sequence) -> int:
        """Number of leading cached blocks, or -1 if the request cannot fit now (:258-264)."""
        prefix = self._prefix_blocks(seq)
        if len(self.free_block_ids) < self._blocks_needed(seq, prefix):
            return -1
        return len(prefix)

    def allocate(self, seq: Sequence, num_cached_blocks: int):
        """Admit a request with its first num_cached_blocks cached (:266-316).

        GPU hits are referenced first so no restore or allocation can recycle
        them; CPU hits are restored (all of them, or only the tail after a
        hybrid split whose head is recomputed); the rest are fresh blocks.
        Any failure releases everything this call took.
        """
        assert not seq.block_table
        prefix = self._prefix_blocks(seq)
        if not 0 <= num_cached_blocks <= len(prefix):
            raise ValueError("requested prefix is no longer available")
        prefix = prefix[:num_cached_blocks]
        if len(self.free_block_ids) < self._blocks_needed(seq, prefix):
            raise MemoryError("not enough free KV blocks to admit the request")
        split = self._plan_split(prefix)
        if split == len(prefix):
            prefix, num_cached_blocks, split = [], 0, 0  # Recomputing everything is fastest.
        self._protected.clear()
        table = [-1] * seq.num_blocks
        owned = []
        try:
            for i, (_, _, block_id, _) in enumerate(prefix):
                if block_id is not None:
                    self._acquire_block(block_id)
                    owned.append(block_id)
                    table[i] = block_id
            with self._batched_copies():
                for i, (h, token_ids, block_id, entry) in enumerate(prefix):
                    if block_id is not None or i < split:
                        continue
                    block_id = self._allocate_block()
                    owned.append(block_id)
                    table[i] = block_id
                    # After a split, the head's prefill overlaps these copies and
                    # finish_restore_span orders the first read after them.
                    if split:
                        self._cpu_prefix_cache._copy_entry(entry, block_id, wait=False)
                    else:
                        self._cpu_prefix_cache._copy_entry(entry, block_id)
                    self.blocks[block_id].update(h, token_ids)
                    self.hash_to_block_id[h] = block_id
                for i in [*range(split), *range(num_cached_blocks, seq.num_blocks)]:
                    block_id = self._allocate_block()
                    owned.append(block_id)
                    table[i] = block_id
        except BaseException:
            for block_id in reversed(owned):
                self._release_block(block_id)
            raise
        seq.block_table = table
        if split:
            seq.num_cached_tokens = 0
            seq.restore_span = (split * self.block_size, num_cached_blocks * self.block_size)
        else:
            seq.num_cached_tokens = num_cached_blocks * self.block_size

    def _plan_split(self, prefix) -> int:
        """Leading CPU-only blocks to recompute (0: restore every hit) (:318-327)."""
        cache = self._cpu_prefix_cache
        if cache is None or cache.hybrid is None:
            return 0
        lead = next((i for i, (_, _, block_id, _) in enumerate(prefix) if block_id is not None), len(prefix))
        split = plan_split(lead, self.block_size, *cache.hybrid)
        # Splitting before a GPU hit only helps if something still restores.
        return split if split < lead or lead == len(prefix) else 0

    def finish_restore_span(self, seq: Sequence):
        """Skip a split admission's restored span once its head is prefilled (:329-336)."""
        start, end = seq.restore_span
        assert seq.num_cached_tokens == start
        seq.restore_span = None
        seq.num_cached_tokens = end
        for block_id in seq.block_table[start // self.block_size:end // self.block_size]:
            self._cpu_prefix_cache.before_block_use(block_id)

    def deallocate(self, seq: Sequence):
        """Release a request's blocks tail first, stamping MRU order (:338-347)."""
        self._release_gen += 1
        for i, block_id in enumerate(seq.block_table):
            self.blocks[block_id].release_gen = self._release_gen
            self.blocks[block_id].seq_index = i
        with self._batched_copies():
            for block_id in reversed(seq.block_table):
                self._release_block(block_id)
        seq.num_cached_tokens = 0
        seq.restore_span = None
        seq.block_table.clear()

    def allocate_for_resume(self, seq: Sequence, num_cached_tokens: int):
        """Fresh blocks for imported KV, leaving the pending token to decode (:349-367)."""
        if seq.block_table or not 0 < num_cached_tokens == len(seq) - 1:
            raise ValueError("resume needs an empty block table and one uncached token")
        num_blocks = -(-num_cached_tokens // self.block_size)
        if len(self.free_block_ids) < num_blocks:
            raise MemoryError("not enough free KV blocks to resume")
        try:
            for _ in range(num_blocks):
                seq.block_table.append(self._allocate_block())
        except BaseException:
            self.deallocate(seq)
            raise
        seq.num_cached_tokens = num_cached_tokens

    def can_append(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq: Sequence):
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq: Sequence):
        """Publish the chained hashes of blocks this step completed (:376-386)."""
        start = seq.num_cached_tokens // self.block_size
        end = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        if start == end:
            return
        h = self.blocks[seq.block_table[start - 1]].hash if start > 0 else -1
        for i in range(start, end):
            block = self.blocks[seq.block_table[i]]
            token_ids = seq.block(i)
            h = self.compute_hash(token_ids, h)
            block.update(h, token_ids)
            self.hash_to_block_id[h] = block.block_id
