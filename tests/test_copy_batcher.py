"""The cache's batching rules, driven with a recording copy engine (CPU only).

The GPU tests show that batched copies land in order on the device; these pin
which engine calls the batcher makes and when: outside coalesce() every call
goes straight through, inside it saves, before_block_reuse waits and restores
are held back and flushed as saves (restore targets first) -> restores (one
call per run of equal wait flags) -> reuse waits (none for blocks restored
into), and a copy that must follow a held-back one flushes first. A batcher
that reordered the flush (restores before saves, reuse waits before the
restores they would hold back) fails here.
"""

import pytest

from kvx.engine.cpu_prefix_cache import _CopyBatcher

STREAM = 7


class RecordingEngine:
    def __init__(self):
        self.calls = []

    def save(self, blocks, slots, stream):
        assert stream == STREAM
        self.calls.append(("save", list(blocks), list(slots)))

    def restore(self, slots, blocks, wait, stream):
        assert stream == STREAM
        self.calls.append(("restore", list(slots), list(blocks), wait))

    def before_block_reuse(self, block, stream):
        assert stream == STREAM
        self.calls.append(("reuse", block))

    def before_block_use(self, block, stream):
        assert stream == STREAM
        self.calls.append(("use", block))


def make():
    engine = RecordingEngine()
    return engine, _CopyBatcher(engine, lambda: STREAM)


def test_calls_go_straight_through_outside_coalesce():
    engine, batcher = make()
    batcher.save(3, 0)
    batcher.before_block_reuse(3)
    batcher.restore(0, 5, True)
    batcher.before_block_use(5)
    assert engine.calls == [("save", [3], [0]), ("reuse", 3), ("restore", [0], [5], True), ("use", 5)]


def test_flush_order_is_saves_then_restore_runs_then_reuse_waits():
    engine, batcher = make()
    with batcher.coalesce():
        batcher.restore(10, 1, True)
        batcher.save(2, 20)
        batcher.before_block_reuse(2)
        batcher.restore(11, 3, True)
        batcher.restore(12, 4, False)
        batcher.save(5, 21)
        batcher.before_block_reuse(5)
        batcher.restore(13, 6, True)
        assert engine.calls == []
    assert engine.calls == [
        ("save", [2, 5], [20, 21]),
        ("restore", [10, 11], [1, 3], True),
        ("restore", [12], [4], False),
        ("restore", [13], [6], True),
        ("reuse", 2),
        ("reuse", 5),
    ]
    assert not (batcher.saves or batcher.reuse or batcher.restores)


def test_recycled_victims_restored_into_are_saved_first_and_get_no_reuse_wait():
    # The block manager's admission: each victim is saved and ordered for reuse, then some are restored into.
    engine, batcher = make()
    with batcher.coalesce():
        for block, slot in ((3, 20), (7, 21), (9, 22)):
            batcher.save(block, slot)
            batcher.before_block_reuse(block)
        batcher.restore(30, 9, False)
        batcher.restore(31, 7, False)
    assert engine.calls == [
        ("save", [7, 9, 3], [21, 22, 20]),
        ("restore", [30, 31], [9, 7], False),
        ("reuse", 3),
    ]


def test_reuse_wait_without_held_back_saves_is_immediate():
    engine, batcher = make()
    with batcher.coalesce():
        batcher.restore(10, 1, False)
        batcher.before_block_reuse(2)  # nothing held back that block 2's save could be
        assert engine.calls == [("reuse", 2)]
    assert engine.calls[-1] == ("restore", [10], [1], False)


@pytest.mark.parametrize("conflict, call, after", [
    ("save of a block a held-back restore writes", lambda b: b.save(2, 21), ("save", [2], [21])),
    ("save into a slot a held-back restore reads", lambda b: b.save(3, 10), ("save", [3], [10])),
    ("save into a slot a held-back save writes", lambda b: b.save(3, 20), ("save", [3], [20])),
    ("use of a block a held-back restore writes", lambda b: b.before_block_use(2), ("use", 2)),
    ("restore into a block a held-back restore writes", lambda b: b.restore(11, 2, False),
     ("restore", [11], [2], False)),
    ("reuse of a block a held-back restore writes", lambda b: b.before_block_reuse(2), ("reuse", 2)),
])
def test_conflicts_flush_first(conflict, call, after):
    engine, batcher = make()
    flushed = [("save", [1], [20]), ("restore", [10], [2], True)]
    with batcher.coalesce():
        batcher.save(1, 20)
        batcher.restore(10, 2, True)
        call(batcher)
        # The conflicting call comes after the flush; a copy is held back again until the block ends.
        assert engine.calls == flushed + ([] if after[0] in ("save", "restore") else [after]), conflict
    assert engine.calls == flushed + [after], conflict


def test_use_of_an_unqueued_block_does_not_flush():
    engine, batcher = make()
    with batcher.coalesce():
        batcher.restore(10, 2, True)
        batcher.before_block_use(7)
        assert engine.calls == [("use", 7)]
    assert engine.calls[-1] == ("restore", [10], [2], True)


def test_nested_blocks_flush_once_at_the_outer_end():
    engine, batcher = make()
    with batcher.coalesce():
        batcher.save(1, 20)
        with batcher.coalesce():
            batcher.restore(10, 2, False)
        assert engine.calls == []
        batcher.restore(11, 3, False)
    assert engine.calls == [("save", [1], [20]), ("restore", [10, 11], [2, 3], False)]


def test_exception_inside_the_block_still_issues_queued_copies():
    engine, batcher = make()
    with pytest.raises(KeyError):
        with batcher.coalesce():
            batcher.save(1, 20)
            batcher.restore(10, 2, True)
            raise KeyError("admission failed")
    assert engine.calls == [("save", [1], [20]), ("restore", [10], [2], True)]
    assert batcher.depth == 0
    batcher.save(4, 21)  # back to immediate calls
    assert engine.calls[-1] == ("save", [4], [21])


class FailingEngine(RecordingEngine):
    def restore(self, slots, blocks, wait, stream):
        raise RuntimeError("hipErrorLaunchFailure")


def test_a_failed_flush_reports_every_copy_of_it_and_raises():
    engine = FailingEngine()
    failed = []
    batcher = _CopyBatcher(engine, lambda: STREAM, lambda saves, restores: failed.append((saves, restores)))
    with pytest.raises(RuntimeError, match="LaunchFailure"):
        with batcher.coalesce():
            batcher.save(1, 20)
            batcher.restore(10, 2, True)
            batcher.restore(11, 3, False)
    # The save was issued before the restore failed; it is reported too (the caller cannot tell).
    assert engine.calls == [("save", [1], [20])]
    assert failed == [([(1, 20)], [(10, 2, True), (11, 3, False)])]
    assert batcher.depth == 0 and not (batcher.saves or batcher.restores or batcher.restore_blocks)
    batcher.save(4, 21)  # the batcher is usable again
    assert engine.calls[-1] == ("save", [4], [21])
