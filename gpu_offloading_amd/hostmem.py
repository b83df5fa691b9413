"""Pinned host memory for the swap and offload paths, placed on the GPU's
NUMA node, and a calibration of the host link those paths run over.

The reference allocates every pinned buffer of its host-link measurements on
the GPU's NUMA node: it reads the node from
``/sys/bus/pci/devices/<bdf>/numa_node``, runs the allocation with the
thread pinned to that node's CPUs, first-touches the pages and pins them
(system_profiling/profile_interconnect.py:38-50 (GPU -> node), :53-77 (node
-> CPUs), :80-89 (alloc_pinned_numa)).  ``pinned_empty`` follows the same
rule for this path's host images.  On ROCm a pinned allocation
(``hipHostMalloc``, which ``torch.empty(pin_memory=True)`` calls) gets its
pages when it is made, not at first touch, so the thread affinity during the
call is what places them; there is no separate first-touch pass.

When sysfs reports no node for the GPU (-1, as in a guest that exposes one
node) or the node's CPUs are not among the process's allowed CPUs, the
buffer is allocated with the process's own placement, and ``placement``
says so.
"""
from __future__ import annotations

import os
from typing import Optional

import torch

__all__ = ["gpu_numa_node", "node_cpus", "placement", "pinned_empty", "calibrate_link"]


def _parse_cpulist(text: str) -> set:
    cpus = set()
    for part in text.strip().split(","):
        if not part:
            continue
        if "-" in part:
            lo, hi = part.split("-")
            cpus.update(range(int(lo), int(hi) + 1))
        else:
            cpus.add(int(part))
    return cpus


def _pci_bdf(device) -> Optional[str]:
    p = torch.cuda.get_device_properties(torch.device(device))
    dom = getattr(p, "pci_domain_id", None)
    bus = getattr(p, "pci_bus_id", None)
    dev = getattr(p, "pci_device_id", None)
    if bus is None or dev is None:
        return None
    return "%04x:%02x:%02x.0" % (dom or 0, bus, dev)


def gpu_numa_node(device="cuda") -> int:
    """NUMA node of the GPU's PCI device from sysfs; -1 when unknown."""
    bdf = _pci_bdf(device)
    if bdf is None:
        return -1
    try:
        with open(f"/sys/bus/pci/devices/{bdf}/numa_node") as f:
            return int(f.read().strip())
    except (OSError, ValueError):
        return -1


def node_cpus(node: int) -> set:
    """CPUs of a NUMA node (empty if the node or sysfs is absent)."""
    try:
        with open(f"/sys/devices/system/node/node{node}/cpulist") as f:
            return _parse_cpulist(f.read())
    except OSError:
        return set()


def _status_field(name: str) -> str:
    try:
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith(name + ":"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def placement(device="cuda") -> dict:
    """Where ``pinned_empty`` puts a buffer for ``device``: the GPU's node,
    the nodes and CPUs the process may use, and the rule applied
    ("gpu-local": the allocation runs on the GPU node's CPUs; "process":
    the GPU's node is unknown or not usable, the process's own placement)."""
    node = gpu_numa_node(device)
    allowed = os.sched_getaffinity(0)
    local = node_cpus(node) & allowed if node >= 0 else set()
    return {"gpu_numa_node": node,
            "mems_allowed": _status_field("Mems_allowed_list"),
            "cpus_allowed": _status_field("Cpus_allowed_list"),
            "host_buffer_node": node if local else None,
            "policy": "gpu-local" if local else "process"}


def pinned_empty(nbytes: int, device="cuda", dtype: torch.dtype = torch.uint8) -> torch.Tensor:
    """A pinned host tensor of ``nbytes`` bytes (as ``dtype`` elements),
    allocated with this thread pinned to the CPUs of the GPU's NUMA node when
    that node is known and usable (the reference's alloc_pinned_numa)."""
    n = nbytes // dtype.itemsize
    node = gpu_numa_node(device)
    old = os.sched_getaffinity(0)
    local = node_cpus(node) & old if node >= 0 else set()
    if not local or local == old:
        return torch.empty(n, dtype=dtype, pin_memory=True)
    os.sched_setaffinity(0, local)
    try:
        return torch.empty(n, dtype=dtype, pin_memory=True)
    finally:
        os.sched_setaffinity(0, old)


def calibrate_link(device="cuda", nbytes: int = 1 << 30, reps: int = 5) -> dict:
    """Host-link rate of plain copies between a pinned ``pinned_empty``
    buffer and device memory, one direction at a time, on a side stream
    (the reference's pcie_h2d_sequential method,
    system_profiling/profile_interconnect.py:96-126: warm-up copies, then
    ``reps`` timed copies of ``nbytes``).  Returns GB/s each way."""
    dev = torch.device(device)
    host = pinned_empty(nbytes, dev)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    res = {}
    for name, dst, src in (("h2d_GBps", buf, host), ("d2h_GBps", host, buf)):
        with torch.cuda.stream(s):
            for _ in range(2):
                dst.copy_(src, non_blocking=True)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                dst.copy_(src, non_blocking=True)
            e1.record(s)
        e1.synchronize()
        res[name] = nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    s.synchronize()
    res["bytes_per_copy"] = nbytes
    res.update(placement(dev))
    del host, buf
    return res
