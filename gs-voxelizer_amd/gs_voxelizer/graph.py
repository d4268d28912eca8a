"""Whole training steps captured in one HIP graph.

The reference reads the intersection count back to the host inside every
forward (voxelize.py:87-88), so its training step cannot be captured.  Here a
captured forward keeps the capacity recorded by an earlier eager step: binning
and the kernels run at that capacity and read the live count from device
memory, and the prefix-sum kernel writes the count into pinned host memory at
every replay.  `CapturedStep.replay()` checks that count against the capacity
the graph was captured with; when the scene has outgrown it, the step is
captured again at a larger capacity and replayed, so a returned result always
covers every intersection.

A step function suitable for capture runs on tensors whose addresses stay fixed
(the leaves and any targets), sets the leaves' ``.grad`` to None before its
backward (so the gradients are allocated inside the graph), and performs no
host synchronisation of its own.  Its outputs, and the leaves' ``.grad``, are
the graph's static outputs: read them after ``replay()``.
"""
from typing import Callable

import torch

from . import voxelize as _vox


class CapturedStep:
    """Captures `step()` (eager warm-up first) and replays it.

    Args:
        step: the training step (forward, loss, backward) to capture.
        warmup: eager runs on a side stream before capture; the first records
            the intersection capacity.
    """

    def __init__(self, step: Callable[[], object], warmup: int = 2):
        self.step = step
        self.device = torch.device("cuda", torch.cuda.current_device())
        self.recaptures = 0
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(int(warmup), 1)):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._capture()

    def _capture(self) -> None:
        self.capacity = _vox.capacity(self.device)
        if self.capacity is None:
            raise RuntimeError("gs_voxelizer: the step ran no voxelization before capture")
        self.graph = torch.cuda.CUDAGraph()
        _vox.begin_capture()
        try:
            with torch.cuda.graph(self.graph):
                self.outputs = self.step()
        finally:
            # (pinned count, capacity) of every voxelization in the step
            self.counts = _vox.end_capture()
        torch.cuda.synchronize()

    def replay(self):
        """Runs the captured step; returns its (static) outputs.  Waits only for
        the prefix sums of the replay, not for the whole step."""
        for host, _ in self.counts:
            host.fill_(-1)
        self.graph.replay()
        grown = 0
        for host, cap in self.counts:
            count = _vox._await_count(host, self.device)
            if count > cap:
                grown = max(grown, count)
        if grown:
            # the replay sorted only a prefix of some forward's intersections:
            # grow the capacity, capture again and rerun
            torch.cuda.synchronize()
            key = self.device.index
            _vox._capacity[key] = max(_vox._capacity.get(key) or 0, _vox._grow(grown))
            self.recaptures += 1
            self._capture()
            return self.replay()
        return self.outputs
