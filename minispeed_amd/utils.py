"""``engine.timers`` and ``set_seed`` (the surface of minispeed/utils.py:14-66).

Wall-clock sections on the host; they are what minispeed reports
(``Timers.log()``: ``"name: 0.123s | ..."``).  Device time of the boundary
kernels is measured with HIP events (``boundary.LaunchTimer``) and
``rocprofv3``, not here: a host timer around an asynchronous launch sees
only the launch, plus whatever host synchronisation the section contains.
"""

from __future__ import annotations

import time
from typing import Dict, List

import torch

from . import comm


class Timer:
    """Accumulated seconds of one named section; ``with timer.section():``
    (or ``with timer:``) adds the wall time of the block.  ``started_at``
    (minispeed/utils.py:18) is the ``time.perf_counter()`` value at which
    the outermost open section began, None while none is open."""

    __slots__ = ("name", "elapsed", "started_at", "_open")

    def __init__(self, name: str):
        self.name = name
        self.elapsed = 0.0
        self.started_at = None
        self._open: List[float] = []    # start times of the sections entered, innermost last

    def __enter__(self) -> "Timer":
        now = time.perf_counter()
        if not self._open:
            self.started_at = now
        self._open.append(now)
        return self

    def __exit__(self, *exc) -> bool:
        self.elapsed += time.perf_counter() - self._open.pop()
        if not self._open:
            self.started_at = None
        return False

    def section(self) -> "Timer":
        return self

    def reset(self) -> None:
        self.elapsed = 0.0


class Timers(Dict[str, Timer]):
    """Registry of named :class:`Timer`s, created on first use."""

    def __missing__(self, name: str) -> Timer:
        timer = self[name] = Timer(name)
        return timer

    def __call__(self, name: str) -> Timer:
        return self[name]

    def timer(self, name: str) -> Timer:
        return self[name]

    def names(self) -> List[str]:
        return list(self.keys())

    def reset(self) -> None:
        for t in self.values():
            t.elapsed = 0.0

    def log(self, rank0_only: bool = True) -> str:
        """``"name: 0.123s | ..."`` in creation order; empty off rank 0."""
        if rank0_only and comm.get_rank() != 0:
            return ""
        return " | ".join("%s: %.3fs" % (t.name, t.elapsed) for t in self.values())


def set_seed(seed: int) -> None:
    """Seed torch's generators on the CPU and on every GPU."""
    torch.manual_seed(int(seed))
