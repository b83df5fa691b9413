"""CPU tests of the pinned-host placement rule (gpu_offloading_amd.hostmem):
the reference's alloc_pinned_numa (system_profiling/profile_interconnect.py:
80-89) runs the allocation on the GPU node's CPUs and restores the affinity."""
import os

import pytest
import torch

from gpu_offloading_amd import hostmem


def test_cpulist_parsing():
    assert hostmem._parse_cpulist("0-3,8,10-11\n") == {0, 1, 2, 3, 8, 10, 11}
    assert hostmem._parse_cpulist("5") == {5}
    assert hostmem._parse_cpulist("") == set()


def _fake_alloc(monkeypatch, seen):
    def empty(n, dtype=None, pin_memory=False):
        seen.append((n, pin_memory, frozenset(os.sched_getaffinity(0))))
        return torch.zeros(n, dtype=dtype)
    monkeypatch.setattr(hostmem.torch, "empty", empty)


def test_allocation_runs_on_the_gpu_nodes_cpus(monkeypatch):
    allowed = os.sched_getaffinity(0)
    if len(allowed) < 2:
        pytest.skip("needs two allowed CPUs")
    first = min(allowed)
    monkeypatch.setattr(hostmem, "gpu_numa_node", lambda device: 1)
    monkeypatch.setattr(hostmem, "node_cpus", lambda node: {first} if node == 1 else set())
    seen = []
    _fake_alloc(monkeypatch, seen)
    t = hostmem.pinned_empty(64, "cuda", torch.int32)
    assert t.numel() == 16
    assert seen == [(16, True, frozenset({first}))]       # allocated on the node's CPUs
    assert os.sched_getaffinity(0) == allowed              # and the affinity is restored


@pytest.mark.parametrize("node,cpus", [(-1, set()), (0, {10 ** 6})])
def test_unknown_or_unusable_node_keeps_the_process_placement(monkeypatch, node, cpus):
    allowed = os.sched_getaffinity(0)
    monkeypatch.setattr(hostmem, "gpu_numa_node", lambda device: node)
    monkeypatch.setattr(hostmem, "node_cpus", lambda n: cpus)
    seen = []
    _fake_alloc(monkeypatch, seen)
    hostmem.pinned_empty(8, "cuda")
    assert seen == [(8, True, frozenset(allowed))]
    p = hostmem.placement("cuda")
    assert p["policy"] == "process" and p["host_buffer_node"] is None
