"""bench.py's NUMA placement helpers on fake sysfs and procfs files (no GPU)."""

import os

import bench


def test_cpu_lists_expand_ranges_and_singles():
    assert bench._cpu_list("0-3,8,10-11\n") == {0, 1, 2, 3, 8, 10, 11}
    assert bench._cpu_list("") == set()


def test_pages_by_node_reads_the_mapping_that_holds_the_address(tmp_path):
    maps = tmp_path / "maps"
    numa = tmp_path / "numa_maps"
    maps.write_text("7f0000000000-7f0000400000 rw-p 00000000 00:00 0\n"
                    "7f0000400000-7f0004400000 rw-s 00000000 00:05 123 /dev/kfd\n")
    numa.write_text("7f0000000000 default anon=12 dirty=12 N0=12 kernelpagesize_kB=4\n"
                    "7f0000400000 default file=/dev/kfd mapped=16384 N0=4096 N1=12288 kernelpagesize_kB=4\n")
    assert bench.pages_by_node(0x7F0000500000, str(maps), str(numa)) == {"0": 4096, "1": 12288}
    assert bench.pages_by_node(0x7F0000000010, str(maps), str(numa)) == {"0": 12}
    assert bench.pages_by_node(0x10, str(maps), str(numa)) is None


def test_numa_placement_from_a_fake_sysfs(tmp_path):
    affinity = sorted(os.sched_getaffinity(0))
    node_cpus = {"0": affinity[: max(1, len(affinity) // 2)], "1": affinity[max(1, len(affinity) // 2):] + [4096]}
    for node, cpus in node_cpus.items():
        d = tmp_path / "devices" / "system" / "node" / f"node{node}"
        d.mkdir(parents=True)
        (d / "cpulist").write_text(",".join(map(str, cpus)) + "\n")
    gpu = tmp_path / "bus" / "pci" / "devices" / "0000:5a:00.0"
    gpu.mkdir(parents=True)
    (gpu / "numa_node").write_text("1\n")
    out = bench.numa_placement(None, "0000:5a:00.0", sysfs=str(tmp_path))
    assert out["gpu_numa_node"] == 1
    assert out["nodes"] == {node: len(cpus) for node, cpus in node_cpus.items()}
    mine = {node: len([c for c in cpus if c in affinity]) for node, cpus in node_cpus.items()}
    assert out["affinity_cpus_by_node"] == {node: n for node, n in mine.items() if n}
    assert out["pinned_pages_by_node"] is None
