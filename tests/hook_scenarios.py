"""Scripted block-manager and scheduler scenarios with a recording CPU tier.

Each scenario drives a block manager (and, in the scheduler scenarios, a
scheduler) through admissions, prefetches, releases, manual restores and
injected failures, and returns a trace: every side-effecting hook the CPU
tier receives, in order, interleaved with snapshots of the pool's
bookkeeping and the outcome of each step. Pure lookups (`_entry_for`) are
not recorded: how often an implementation looks an entry up is not part of
the contract, only what it then copies, saves and orders.

tests/golden/make_hook_traces.py runs these scenarios on the reference's
BlockManager and Scheduler (nanovllm/engine/block_manager.py,
nanovllm/engine/scheduler.py) and commits the traces as
tests/golden/hook_traces.json; tests/test_hook_contract.py runs them on
kvx's engine and requires the same traces. A scenario only uses what both
expose: the constructors, the reference's public methods and attributes,
and the duck-typed tier hooks (block_manager.py:97-137, 145-183, 202-237,
266-336).

`api` is any object with attributes BlockManager, Sequence, SamplingParams
and Scheduler.
"""

from dataclasses import dataclass
from types import SimpleNamespace

BS = 256


@dataclass(frozen=True)
class Entry:
    """A CPU entry as the block manager sees it: opaque, handed back to _copy_entry."""

    key: int
    token_ids: tuple


class RecordingTier:
    """Duck-typed CPU tier: records every side-effecting hook and emulates saves.

    A "save" (from _preserve_before_recycle, or from _preserve_on_release
    while admission is blocked and save_on_release is set) stores the
    published block's tokens under its hash, up to `budget` entries.
    """

    def __init__(self, trace, manager, *, prefetch=False, hybrid=None, save_on_release=False, budget=None):
        self.trace = trace
        self.manager = manager
        self.prefetch_enabled = prefetch
        self.hybrid = hybrid
        self._prefetched_blocks = 0
        self.save_on_release = save_on_release
        self.budget = budget
        self.cpu: dict[int, tuple] = {}
        self.copies = 0
        self.fail_copy_at = None  # the n-th _copy_entry (0-based) raises
        self.fail_preserve = False

    def _save(self, h):
        block_id = self.manager.hash_to_block_id[h]
        tokens = tuple(self.manager.blocks[block_id].token_ids)
        if h in self.cpu:
            return
        if self.budget is not None and len(self.cpu) >= self.budget:
            self.trace.append(["budget_skip", h])
            return
        self.cpu[h] = tokens

    def _preserve_before_recycle(self, h):
        self.trace.append(["preserve_before_recycle", h, self.manager.hash_to_block_id.get(h)])
        if self.fail_preserve:
            raise RuntimeError("injected preservation failure")
        self._save(h)

    def _preserve_on_release(self, h):
        blocked = bool(self.manager.admission_blocked)
        self.trace.append(["preserve_on_release", h, blocked])
        if self.save_on_release and blocked:
            self._save(h)

    def before_block_reuse(self, block_id):
        self.trace.append(["before_block_reuse", block_id])

    def before_block_use(self, block_id):
        self.trace.append(["before_block_use", block_id])

    def _entry_for(self, h, token_ids):
        tokens = self.cpu.get(h)
        return Entry(h, tokens) if tokens is not None and tokens == tuple(token_ids) else None

    def _copy_entry(self, entry, block_id, wait=True):
        n = self.copies
        self.copies += 1
        self.trace.append(["copy_entry", entry.key, block_id, bool(wait)])
        if self.fail_copy_at == n:
            raise RuntimeError("injected copy failure")


class Run:
    """One scenario's trace and the sequences it names (by creation order, not seq_id)."""

    def __init__(self, api):
        self.api = api
        self.trace: list = []
        self.seqs: list = []
        self.manager = None
        self.tier = None

    def seq(self, tokens, max_tokens=1, ignore_eos=False):
        s = self.api.Sequence(list(tokens), self.api.SamplingParams(temperature=0, max_tokens=max_tokens,
                                                                     ignore_eos=ignore_eos))
        self.seqs.append(s)
        return s

    def name(self, seq):
        return next(i for i, s in enumerate(self.seqs) if s is seq)

    def attach(self, **kwargs):
        self.tier = RecordingTier(self.trace, self.manager, **kwargs)
        self.manager._cpu_prefix_cache = self.tier
        return self.tier

    def snap(self, label):
        m = self.manager
        self.trace.append(["state", label, {
            "free": list(m.free_block_ids),
            "used": sorted(m.used_block_ids),
            "published": sorted([h, b] for h, b in m.hash_to_block_id.items()),
            "refs": [b.ref_count for b in m.blocks],
            "seqs": [[list(s.block_table), s.num_cached_tokens, list(s.restore_span) if s.restore_span else None]
                     for s in self.seqs],
            "cpu": sorted(self.tier.cpu) if self.tier is not None else [],
            "prefetched": self.tier._prefetched_blocks if self.tier is not None else 0,
        }])

    def step(self, label, fn, *args, **kwargs):
        """Runs fn, recording its result or the type of the exception it raised."""
        try:
            result = fn(*args, **kwargs)
        except Exception as error:  # the trace records which error, the test compares it
            self.trace.append(["raised", label, type(error).__name__])
            return None
        self.trace.append(["returned", label, result if isinstance(result, (int, bool, type(None))) else None])
        return result


def tokens_of(*values, tail=0, tail_value=None):
    """Full blocks of the given token values, then `tail` extra tokens."""
    out = []
    for v in values:
        out += [v] * BS
    out += [tail_value if tail_value is not None else values[-1] + 1000] * tail
    return out


def chain(api, blocks, prefix=-1):
    """Chained hashes of full token blocks."""
    hashes, h = [], prefix
    for block in blocks:
        h = api.BlockManager.compute_hash(list(block), h)
        hashes.append(h)
    return hashes


def finish(run, seq):
    """Admit a request, write all of its tokens and release it (its full blocks stay published GPU hits)."""
    m = run.manager
    n = m.can_allocate(seq)
    assert n >= 0
    m.allocate(seq, n)
    seq.num_scheduled_tokens = len(seq) - seq.num_cached_tokens
    m.hash_blocks(seq)
    seq.num_cached_tokens, seq.num_scheduled_tokens = len(seq), 0
    m.deallocate(seq)


def hold(run, seq):
    """Admit and write a request without releasing it."""
    m = run.manager
    n = m.can_allocate(seq)
    assert n >= 0
    m.allocate(seq, n)
    seq.num_scheduled_tokens = len(seq) - seq.num_cached_tokens
    m.hash_blocks(seq)
    seq.num_cached_tokens, seq.num_scheduled_tokens = len(seq), 0


def seed_cpu(run, token_blocks, prefix=-1):
    """Put entries for these chained full blocks into the tier (as if saved earlier)."""
    hashes = chain(run.api, token_blocks, prefix)
    for h, block in zip(hashes, token_blocks):
        run.tier.cpu[h] = tuple(block)
    return hashes


# ---------------------------------------------------------------------------
# Block-manager scenarios

def admission_with_gpu_and_cpu_hits(api, eviction="lru"):
    """GPU hits on both sides of a CPU hit, victims saved on recycling, a waited restore, a fresh suffix."""
    run = Run(api)
    run.manager = api.BlockManager(12, BS, eviction)
    tier = run.attach()
    a = run.seq(tokens_of(1, 2, 3, 4, tail=1))
    finish(run, a)
    run.snap("after A")
    # A long request recycles the tail of A's prefix (its last two full blocks are saved on the way).
    z = run.seq(tokens_of(*range(301, 310), tail=1))
    hold(run, z)
    run.snap("after Z admitted")
    run.step("deallocate Z", run.manager.deallocate, z)
    h = chain(api, [[1] * BS, [2] * BS, [3] * BS, [4] * BS])
    # Publish A's fourth block on a free unpublished block: a GPU hit after the CPU hit of the third.
    spare = next(b for b in run.manager.free_block_ids if run.manager.blocks[b].hash == -1)
    run.manager.blocks[spare].update(h[3], [4] * BS)
    run.manager.hash_to_block_id[h[3]] = spare
    run.snap("before B")
    b = run.seq(tokens_of(1, 2, 3, 4, 5, tail=7))
    run.step("can_allocate B", run.manager.can_allocate, b)
    run.step("allocate B", run.manager.allocate, b, run.manager.can_allocate(b))
    run.snap("after B admitted")
    run.step("deallocate B", run.manager.deallocate, b)
    run.snap("after B released")
    del tier
    return run.trace


def admission_mru(api):
    return admission_with_gpu_and_cpu_hits(api, "mru")


def split_admission_and_restore_span(api):
    """Hybrid planning recomputes the head of a CPU-only prefix; the tail restores without waiting."""
    run = Run(api)
    run.manager = api.BlockManager(12, BS)
    tier = run.attach(hybrid=(1.0, 1.0 / BS, 0.0))
    blocks = [[v] * BS for v in (11, 12, 13, 14, 15, 16, 17, 18)]
    seed_cpu(run, blocks)
    s = run.seq([t for b in blocks for t in b] + [99] * 5)
    run.step("can_allocate", run.manager.can_allocate, s)
    run.step("allocate", run.manager.allocate, s, run.manager.can_allocate(s))
    run.snap("after split admission")
    # Prefill the head, then the span is skipped and its blocks ordered before their first read.
    s.num_scheduled_tokens = s.restore_span[0] - s.num_cached_tokens
    run.manager.hash_blocks(s)
    s.num_cached_tokens += s.num_scheduled_tokens
    s.num_scheduled_tokens = 0
    run.step("finish_restore_span", run.manager.finish_restore_span, s)
    run.snap("after restore span")
    # A GPU hit inside the prefix: splitting before it only pays if something still restores.
    run.step("deallocate", run.manager.deallocate, s)
    tier.hybrid = (1e-9, 1.0, 0.0)  # restores nearly free: restore everything
    t = run.seq([t for b in blocks for t in b] + [98] * 3)
    run.step("allocate restore-all", run.manager.allocate, t, run.manager.can_allocate(t))
    run.snap("after restore-all")
    run.step("deallocate", run.manager.deallocate, t)
    tier.hybrid = (1.0, 0.0, 0.0)  # recompute free: a CPU-only prefix is recomputed whole
    fresh = [[v] * BS for v in (19, 20, 21)]
    seed_cpu(run, fresh)
    u = run.seq([t for b in fresh for t in b] + [97] * 3)
    run.step("allocate recompute-all", run.manager.allocate, u, run.manager.can_allocate(u))
    run.step("deallocate", run.manager.deallocate, u)
    # The GPU hits of t's prefix lead: nothing to split before them.
    v = run.seq([t for b in blocks[:3] for t in b] + [96] * 3)
    run.step("allocate gpu-led", run.manager.allocate, v, run.manager.can_allocate(v))
    run.snap("after recompute-all")
    return run.trace


def split_before_a_gpu_hit(api):
    """CPU hits ahead of a GPU hit: a split that would reach the GPU hit restores everything instead."""
    run = Run(api)
    run.manager = api.BlockManager(10, BS)
    tier = run.attach(hybrid=(1.0, 0.0, 0.0))  # recomputing costs nothing: the plan recomputes the whole run
    blocks = [[31] * BS, [32] * BS, [33] * BS]
    h = seed_cpu(run, blocks[:2])
    (h3,) = chain(api, blocks[2:], h[-1])
    run.manager.blocks[9].update(h3, blocks[2])
    run.manager.hash_to_block_id[h3] = 9
    s = run.seq([t for b in blocks for t in b] + [5] * 4)
    run.step("allocate (plan reaches the GPU hit)", run.manager.allocate, s, run.manager.can_allocate(s))
    run.snap("after restore-all")
    run.step("deallocate", run.manager.deallocate, s)
    for key in h:
        block_id = run.manager.hash_to_block_id.pop(key, None)  # evict the two restored blocks again
        if block_id is not None:
            run.manager.blocks[block_id].update(-1, [])
    tier.hybrid = (1.0, 1.0 / BS, 0.0)  # one block costs one restore: recompute one, restore one
    t = run.seq([t for b in blocks for t in b] + [6] * 4)
    run.step("allocate (split before the GPU hit)", run.manager.allocate, t, run.manager.can_allocate(t))
    run.snap("after split")
    return run.trace


def prefetch_of_a_blocked_request(api, eviction="lru"):
    """A blocked request's CPU hits restore into spare blocks without write ordering, then admission reuses them."""
    run = Run(api)
    run.manager = api.BlockManager(8, BS, eviction)
    tier = run.attach(prefetch=True)
    blocks = [[v] * BS for v in (21, 22, 23, 24)]
    seed_cpu(run, blocks)
    own = run.seq(tokens_of(21, tail=3))
    finish(run, own)  # its first block is an idle GPU hit of the blocked request
    other = run.seq(tokens_of(31, 32, tail=1))
    finish(run, other)  # idle published blocks prefetch may recycle
    runner = run.seq(tokens_of(41, 42, tail=9))
    hold(run, runner)
    run.snap("before prefetch")
    blocked = run.seq([t for b in blocks for t in b] + [77] * 6)
    run.step("can_allocate blocked", run.manager.can_allocate, blocked)
    run.step("prefetch", run.manager.prefetch, blocked, 1)
    run.snap("after prefetch")
    run.step("prefetch again (throttled)", run.manager.prefetch, blocked, 1)
    run.step("deallocate runner", run.manager.deallocate, runner)
    run.step("prefetch after release", run.manager.prefetch, blocked, 1)
    run.snap("after second prefetch")
    run.step("allocate blocked", run.manager.allocate, blocked, run.manager.can_allocate(blocked))
    run.snap("after admission")
    return run.trace


def prefetch_mru(api):
    return prefetch_of_a_blocked_request(api, "mru")


def copy_failure_rolls_back(api):
    """A restore failing mid-admission releases everything the admission took; a retry succeeds."""
    run = Run(api)
    run.manager = api.BlockManager(9, BS)
    tier = run.attach()
    a = run.seq(tokens_of(51, 52, tail=2))
    finish(run, a)
    blocks = [[51] * BS, [52] * BS, [53] * BS, [54] * BS]
    seed_cpu(run, blocks)
    b = run.seq([t for blk in blocks for t in blk] + [5] * 4)
    tier.fail_copy_at = 1
    run.step("allocate (second copy fails)", run.manager.allocate, b, run.manager.can_allocate(b))
    run.snap("after failed admission")
    tier.fail_copy_at = None
    run.step("allocate retry", run.manager.allocate, b, run.manager.can_allocate(b))
    run.snap("after retry")
    return run.trace


def preservation_failure_keeps_the_victim(api):
    """A victim whose save raises stays free and published; nothing is recycled."""
    run = Run(api)
    run.manager = api.BlockManager(3, BS)
    tier = run.attach()
    a = run.seq(tokens_of(61, 62, tail=1))
    finish(run, a)
    run.snap("before")
    tier.fail_preserve = True
    run.step("allocate_block", run.manager._allocate_block)
    run.snap("after failed preserve")
    tier.fail_preserve = False
    run.step("allocate_block", run.manager._allocate_block)
    run.step("allocate_block", run.manager._allocate_block)
    run.snap("after two recycles")
    return run.trace


def manual_restores(api):
    """restore_cached_block: GPU hit without a copy, bad arguments, a full pool, and a failing copy."""
    run = Run(api)
    run.manager = api.BlockManager(4, BS)
    run.attach()
    a = run.seq(tokens_of(71, 72, tail=1))
    finish(run, a)
    h71, h72 = chain(api, [[71] * BS, [72] * BS])
    copies = []

    def copy_ok(block_id):
        copies.append(block_id)

    def copy_fail(block_id):
        copies.append(block_id)
        raise RuntimeError("injected copy failure")

    run.step("restore existing", run.manager.restore_cached_block, h71, [71] * BS, copy_ok)
    run.step("restore conflicting tokens", run.manager.restore_cached_block, h71, [70] * BS, copy_ok)
    run.step("restore short block", run.manager.restore_cached_block, 12345, [1] * 10, copy_ok)
    run.step("restore bad hash", run.manager.restore_cached_block, -5, [1] * BS, copy_ok)
    (h80,) = chain(api, [[80] * BS])
    run.step("restore new", run.manager.restore_cached_block, h80, [80] * BS, copy_ok)
    run.snap("after restore new")
    (h81,) = chain(api, [[81] * BS])
    run.step("restore failing", run.manager.restore_cached_block, h81, [81] * BS, copy_fail)
    run.snap("after failing restore")
    held = run.seq(tokens_of(91, 92, 93, tail=5))
    hold(run, held)
    (h82,) = chain(api, [[82] * BS])
    run.step("restore into a full pool", run.manager.restore_cached_block, h82, [82] * BS, copy_ok)
    run.trace.append(["copies", copies])
    run.snap("end")
    return run.trace


def resume_and_growth(api):
    """allocate_for_resume, decode growth at block boundaries, can_append with an empty free list."""
    run = Run(api)
    run.manager = api.BlockManager(5, BS)
    tier = run.attach()
    a = run.seq(tokens_of(101, tail=1))
    finish(run, a)
    s = run.seq(tokens_of(102, 103, tail=0) + [7], max_tokens=8)
    run.step("resume bad count", run.manager.allocate_for_resume, s, 10)
    run.step("resume", run.manager.allocate_for_resume, s, len(s) - 1)
    run.snap("after resume")
    s.num_scheduled_tokens = len(s) - s.num_cached_tokens
    run.manager.hash_blocks(s)
    s.num_cached_tokens += s.num_scheduled_tokens
    s.num_scheduled_tokens = 0
    for token in (8, 9):
        run.step("can_append", run.manager.can_append, s)
        run.step("may_append", run.manager.may_append, s)
        s.append_token(token)
    run.snap("after growth")
    big = run.seq(tokens_of(111, tail=1))
    run.step("can_allocate big", run.manager.can_allocate, big)
    hold(run, big)
    run.step("can_append when full", run.manager.can_append, s)
    run.snap("end")
    del tier
    return run.trace


def save_on_release_while_blocked(api):
    """Release saves published blocks only while admission is blocked (tail first)."""
    run = Run(api)
    run.manager = api.BlockManager(8, BS)
    run.attach(save_on_release=True, budget=2)
    a = run.seq(tokens_of(121, 122, 123, tail=2))
    hold(run, a)
    run.manager.admission_blocked = False
    run.step("deallocate (not blocked)", run.manager.deallocate, a)
    b = run.seq(tokens_of(131, 132, 133, tail=2))
    hold(run, b)
    run.manager.admission_blocked = True
    run.step("deallocate (blocked)", run.manager.deallocate, b)
    run.snap("end")
    return run.trace


# ---------------------------------------------------------------------------
# Scheduler scenarios: schedule() / postprocess() with scripted model outputs.

def scheduler_config(num_blocks, budget=4096, max_seqs=4, eos=99, kv_eviction="lru"):
    return SimpleNamespace(max_num_seqs=max_seqs, max_num_batched_tokens=budget, eos=eos, kvcache_block_size=BS,
                           num_kvcache_blocks=num_blocks, kv_eviction=kv_eviction)


class SchedulerRun(Run):
    def __init__(self, api, num_blocks, **config):
        super().__init__(api)
        api.Sequence.block_size = BS
        self.scheduler = api.Scheduler(scheduler_config(num_blocks, **config))
        self.manager = self.scheduler.block_manager

    def add(self, tokens, max_tokens=1, ignore_eos=False):
        s = self.seq(tokens, max_tokens, ignore_eos)
        self.scheduler.add(s)
        return s

    def tick(self, label, token=7):
        """One engine step: schedule, then postprocess with `token` for every scheduled request."""
        try:
            seqs, is_prefill = self.scheduler.schedule()
        except Exception as error:
            self.trace.append(["raised", label, type(error).__name__])
            return None
        self.trace.append(["scheduled", label, bool(is_prefill),
                           [[self.name(s), s.num_cached_tokens, s.num_scheduled_tokens] for s in seqs],
                           bool(self.manager.admission_blocked)])
        self.scheduler.postprocess(seqs, [token] * len(seqs), is_prefill)
        self.trace.append(["queues", label, [self.name(s) for s in self.scheduler.waiting],
                           [self.name(s) for s in self.scheduler.running]])
        return seqs


def scheduler_blocked_admission(api):
    """A waiting request that does not fit arms save-on-release and prefetches into spare blocks."""
    run = SchedulerRun(api, 6)
    tier = run.attach(prefetch=True, save_on_release=True)
    a = run.add(tokens_of(201, 202, tail=3), max_tokens=2)
    run.tick("prefill A")
    run.tick("decode A")
    blocks = [[v] * BS for v in (211, 212, 213)]
    seed_cpu(run, blocks)
    b = run.add(tokens_of(221, 222, 223, tail=1), max_tokens=3)
    run.tick("prefill B")
    c = run.add([t for blk in blocks for t in blk] + [5] * 2, max_tokens=1)
    for i in range(6):
        if run.scheduler.is_finished():
            break
        run.tick(f"step {i}")
    run.snap("end")
    del a, b, c, tier
    return run.trace


def scheduler_chunked_restore(api):
    """A CPU restore and a small token budget compose: the restored block is skipped, the rest is chunked."""
    run = SchedulerRun(api, 2, budget=512)
    run.add(tokens_of(1, tail=1), max_tokens=1)
    run.tick("prefill warm")
    tier = run.attach()
    for value, length in ((3, 257), (4, 1)):
        run.add([value] * length, max_tokens=1)
        run.tick(f"prefill {value}")
    run.scheduler.max_num_batched_tokens = 8
    run.add([1] * 269, max_tokens=1)
    run.tick("chunk 1")
    run.tick("chunk 2")
    run.snap("end")
    del tier
    return run.trace


def scheduler_copy_failure_rollback(api):
    """A restore failing inside schedule() leaves every queue and request as it was; the retry admits both."""
    run = SchedulerRun(api, 8, budget=4096)
    tier = run.attach()
    blocks = [[v] * BS for v in (231, 232)]
    seed_cpu(run, blocks)
    run.add(tokens_of(241, tail=2), max_tokens=1)
    run.add([t for blk in blocks for t in blk] + [3] * 3, max_tokens=1)
    tier.fail_copy_at = 1
    run.tick("failing prefill")
    run.snap("after failure")
    tier.fail_copy_at = None
    run.tick("retry")
    run.snap("end")
    return run.trace


def scheduler_decode_growth_and_preemption(api):
    """Decode growth recycles a published block (saving it) and preempts the newest request when full."""
    run = SchedulerRun(api, 5)
    run.attach(budget=8)
    old = run.seq(tokens_of(251, tail=1))
    finish(run, old)
    a = run.add([5] * 510, max_tokens=6, ignore_eos=True)
    b = run.add([6] * 510, max_tokens=6, ignore_eos=True)
    run.tick("prefill")
    for i in range(12):
        if run.scheduler.is_finished():
            break
        run.tick(f"step {i}")
    run.snap("end")
    del a, b
    return run.trace


def random_workload(api, seed, eviction="lru", prefetch=False, save_on_release=False, budget=None, hybrid=None):
    """A seeded stream of requests over shared documents, scheduled and decoded for 40 steps.

    Documents of 1-5 full blocks share leading blocks with each other, so
    requests hit GPU blocks, CPU entries or nothing; requests arrive at random
    steps with a random tail and 1-3 output tokens. Pool size, token budget and
    batch size vary with the seed.
    """
    import random

    rng = random.Random(seed)
    num_blocks = rng.randint(6, 14)
    run = SchedulerRun(api, num_blocks, budget=rng.choice([512, 1024, 4096]), max_seqs=rng.randint(1, 4),
                       kv_eviction=eviction)
    run.attach(prefetch=prefetch, save_on_release=save_on_release, budget=budget, hybrid=hybrid)
    base = 1000 + 100 * seed
    documents = []
    for d in range(4):
        shared = documents[rng.randrange(len(documents))][:rng.randint(1, 2)] if documents and rng.random() < 0.6 else []
        own = [base + 10 * d + i for i in range(rng.randint(1, 5) - len(shared))]
        documents.append(shared + own)
    for step in range(40):
        for _ in range(rng.choice([0, 0, 1, 1, 2])):
            doc = rng.choice(documents)
            blocks = doc[:rng.randint(1, len(doc))]
            tail = rng.randint(0, BS - 1) if rng.random() < 0.7 else 0
            tokens = tokens_of(*blocks, tail=tail, tail_value=base + 90 + step)
            if len(tokens) // BS + 2 < num_blocks:
                run.add(tokens, max_tokens=rng.randint(1, 3), ignore_eos=True)
        if not run.scheduler.is_finished():
            run.tick(f"step {step}")
        if step % 10 == 9:
            run.snap(f"after step {step}")
    return run.trace


def _random_scenarios():
    out = {}
    for seed, options in enumerate([{}, {"eviction": "mru"}, {"prefetch": True, "save_on_release": True},
                                    {"prefetch": True, "eviction": "mru"}, {"budget": 3},
                                    {"save_on_release": True, "budget": 5, "eviction": "mru"},
                                    {"prefetch": True, "hybrid": (1e-3, 1e-6, 0.0)},
                                    {"hybrid": (1e-4, 1e-5, 1e-9), "save_on_release": True},
                                    {"prefetch": True, "save_on_release": True, "budget": 4},
                                    {}, {"eviction": "mru", "prefetch": True, "save_on_release": True},
                                    {"prefetch": True, "hybrid": (5e-4, 2e-6, 0.0), "eviction": "mru"}]):
        out[f"random_workload_{seed}"] = (lambda api, seed=seed, options=options:
                                          random_workload(api, seed, **options))
    return out


SCENARIOS = {
    "admission_with_gpu_and_cpu_hits": admission_with_gpu_and_cpu_hits,
    "admission_mru": admission_mru,
    "split_admission_and_restore_span": split_admission_and_restore_span,
    "split_before_a_gpu_hit": split_before_a_gpu_hit,
    "prefetch_of_a_blocked_request": prefetch_of_a_blocked_request,
    "prefetch_mru": prefetch_mru,
    "copy_failure_rolls_back": copy_failure_rolls_back,
    "preservation_failure_keeps_the_victim": preservation_failure_keeps_the_victim,
    "manual_restores": manual_restores,
    "resume_and_growth": resume_and_growth,
    "save_on_release_while_blocked": save_on_release_while_blocked,
    "scheduler_blocked_admission": scheduler_blocked_admission,
    "scheduler_chunked_restore": scheduler_chunked_restore,
    "scheduler_copy_failure_rollback": scheduler_copy_failure_rollback,
    "scheduler_decode_growth_and_preemption": scheduler_decode_growth_and_preemption,
    **_random_scenarios(),
}


def run_all(api) -> dict:
    return {name: fn(api) for name, fn in SCENARIOS.items()}
