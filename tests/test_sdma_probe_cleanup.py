"""bench.py's SDMA probe leaves no HSA state of its own behind, on the CPU with a recording HSA double.

Every signal the copier creates is destroyed on every path that can destroy
it safely (success, a copy that fails to queue); a wait that times out keeps
its signals and buffers (copies may still write them) and the copier takes no
more work; close() balances the copier's hsa_init once; and the probe refuses
to run when a profiler tool is mapped into the process.
"""

import ctypes

import pytest

import bench


class FakeHSA:
    def __init__(self, fail_at=None, complete=True):
        self.values, self.destroyed, self.queued = {}, [], 0
        self.shut_downs, self.next_signal = 0, 100
        self.fail_at, self.complete = fail_at, complete

    def hsa_signal_create(self, initial, consumers, agents, out):
        self.next_signal += 1
        out._obj.value = self.next_signal
        self.values[self.next_signal] = initial
        return 0

    def hsa_amd_memory_async_copy_on_engine(self, dst, dst_agent, src, src_agent, size, deps, dep_list, signal,
                                            engine, force):
        if self.fail_at is not None and self.queued == self.fail_at:
            return 4096  # HSA_STATUS_ERROR
        self.queued += 1
        if self.complete:
            self.values[signal] -= 1
        return 0

    def hsa_signal_subtract_screlease(self, signal, amount):
        self.values[signal] -= amount

    def hsa_signal_load_scacquire(self, signal):
        return self.values[signal]

    def hsa_signal_destroy(self, signal):
        assert signal in self.values and signal not in self.destroyed
        self.destroyed.append(signal)

    def hsa_shut_down(self):
        self.shut_downs += 1
        return 0


class Buffer:
    def data_ptr(self):
        return 0x1000


def copier(hsa, pieces=4):
    c = object.__new__(bench.SdmaCopier)
    c.unavailable, c.abandoned, c._live = None, False, []
    c.hsa, c.cpu, c.gpu = hsa, 1, 2
    c.nbytes, c.piece = pieces * 64, 64
    c.pieces = [(i * 64, 64) for i in range(pieces)]
    c.engines = {"d2h": [1], "h2d": [4]}
    c.dev_src = c.dev_dst = c.host_dst = c.host_src = Buffer()
    return c


def test_a_run_destroys_its_signals_and_close_balances_hsa_init():
    hsa = FakeHSA()
    c = copier(hsa)
    assert c.run(["d2h", "h2d"]) >= 0
    assert sorted(hsa.destroyed) == sorted(hsa.values) and not c._live
    c.close()
    c.close()
    assert hsa.shut_downs == 1 and c.hsa is None


def test_a_copy_that_fails_to_queue_leaves_no_signal_behind():
    hsa = FakeHSA(fail_at=6)  # the third piece of the second direction
    c = copier(hsa)
    with pytest.raises(RuntimeError, match="h2d"):
        c.start(["d2h", "h2d"])
    # The un-queued pieces were taken off the count, the queued ones waited for, and both signals destroyed.
    assert all(v == 0 for v in hsa.values.values())
    assert sorted(hsa.destroyed) == sorted(hsa.values) and not c._live
    c.close()
    assert hsa.shut_downs == 1


def test_a_timed_out_wait_keeps_signals_and_buffers_and_skips_shutdown():
    hsa = FakeHSA(complete=False)
    c = copier(hsa)
    signals = c.start(["d2h"])
    with pytest.raises(RuntimeError, match="did not finish"):
        c.wait(signals, limit_s=0.01)
    assert c.abandoned and not hsa.destroyed
    with pytest.raises(RuntimeError, match="cannot queue"):
        c.start(["d2h"])
    c.close()
    assert hsa.shut_downs == 0 and c in bench._ABANDONED_COPIERS and c.host_dst is not None
    bench._ABANDONED_COPIERS.remove(c)


def test_the_probe_refuses_to_run_under_a_profiler_tool(tmp_path, monkeypatch):
    maps = tmp_path / "maps"
    maps.write_text("7f00-7f10 r-xp 0 08:01 1 /usr/lib/libc.so.6\n"
                    "7f20-7f30 r-xp 0 08:01 2 /opt/rocm/lib/librocprofiler-sdk-tool.so.1\n")
    assert bench.profiler_tool_loaded(str(maps)).endswith("librocprofiler-sdk-tool.so.1")
    maps.write_text("7f00-7f10 r-xp 0 08:01 1 /usr/lib/libc.so.6\n")
    assert bench.profiler_tool_loaded(str(maps)) is None
    assert bench.profiler_tool_loaded(str(tmp_path / "missing")) is None

    loaded = []
    monkeypatch.setattr(bench, "profiler_tool_loaded", lambda: "/opt/rocm/lib/librocprofiler-sdk.so.1")
    monkeypatch.setattr(ctypes, "CDLL", lambda *a, **k: loaded.append(a) or pytest.fail("HSA was loaded"))
    c = bench.SdmaCopier(None, 1 << 20)
    assert "profiler tool" in c.unavailable and not loaded
    assert bench.sdma_probe(None, 1 << 20) == {"skipped": c.unavailable}
