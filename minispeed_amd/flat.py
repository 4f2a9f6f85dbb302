"""Flat fp32 parameter groups (the layout of minispeed/flat.py).

A parameter group is laid out as one flat index space: parameter ``i`` owns
``[offset_i, offset_i + numel_i)`` with ``offset_i`` the prefix sum of the
numels in group order, and the space is zero-padded to
``numel_padded = round_up(numel, world_size)`` (flat.py:16-17, 50-52).  Rank
``r`` owns ``[r*S, (r+1)*S)`` with ``S = numel_padded / world_size`` for
ZeRO stage >= 1 and the whole space at stage 0 (flat.py:54-59).

Device buffers, all fp32 and resident in HBM (flat.py:61-73):
  ``data``        masters, ``numel_padded`` (the owned shard only after a
                  ZeRO-3 ``partition_params``)
  ``grad``        flat gradient, ``numel_padded`` (stage 3: ``None`` outside
                  the boundary)
  ``grad_shard``  owned gradient slice, stage >= 2
and the AdamW moments of the owned range, allocated with the masters so the
three can be placed apart in HBM (``state_buffers``) and handed to the
optimizer (``take_moment_buffers``).

The boundary kernels address ragged per-parameter storage (``param.grad``,
``param.data``) through segment tables built by :class:`FlatLayout`; a table
is a sorted list of ``(begin, numel, grad_ptr, model_ptr)`` rows that tiles a
flat range exactly, gaps and padding being rows with NULL pointers.
"""

from __future__ import annotations

import logging
import os
from typing import Iterable, List, Optional, Sequence, Tuple

import numpy as np
import torch
from torch import nn

from . import _native

Range = Tuple[int, int]


def _round_up(x: int, multiple: int) -> int:
    return -(-x // multiple) * multiple


def _overlap(a: Range, b: Range) -> Range:
    lo, hi = max(a[0], b[0]), min(a[1], b[1])
    return (lo, hi) if lo < hi else (lo, lo)


def _walk():
    """The C++ pointer walk (``_walk.so``, built next to this file)."""
    try:
        from . import _walk as mod
    except ImportError as exc:
        raise _native.NativeLibraryError(
            "minispeed_amd/_walk.so is missing or does not load; build it with "
            "`python -m minispeed_amd.build`") from exc
    return mod


def record_streams(tensors: Sequence[Optional[torch.Tensor]], stream: torch.cuda.Stream) -> None:
    """``t.record_stream(stream)`` for every device tensor of ``tensors``
    (``None`` entries skipped), in one call into the C++ walk."""
    items = tensors if isinstance(tensors, list) else list(tensors)
    _walk().record_streams(items, int(stream.device_type), int(stream.device_index),
                           int(stream.stream_id))


def _with_pad_slot(ptrs, n_params: int) -> np.ndarray:
    """Addresses as int64 with a trailing 0 for the padding row."""
    if isinstance(ptrs, np.ndarray) and ptrs.shape == (n_params + 1,):
        return ptrs
    return np.asarray(list(ptrs) + [0], dtype=np.uint64).astype(np.int64)


# --------------------------------------------------------------------------
class FlatLayout:
    """Index math of one flat group; no device memory, CPU-testable."""

    def __init__(self, numels: Sequence[int], *, rank: int, world_size: int, zero_stage: int):
        if len(numels) == 0:
            raise ValueError("FlatParamGroup requires at least one parameter")
        if world_size < 1 or not (0 <= rank < world_size):
            raise ValueError(f"bad rank/world_size {rank}/{world_size}")
        self.numels: List[int] = [int(n) for n in numels]
        self.offsets: List[int] = []
        acc = 0
        for n in self.numels:
            self.offsets.append(acc)
            acc += n
        self.numel = acc
        self.numel_padded = _round_up(acc, world_size)
        self.shard_size = self.numel_padded // world_size
        if zero_stage >= 1:
            self.shard_start = rank * self.shard_size
            self.shard_end = self.shard_start + self.shard_size
        else:
            self.shard_start, self.shard_end = 0, self.numel_padded

    def param_range(self, i: int) -> Range:
        return self.offsets[i], self.offsets[i] + self.numels[i]

    def segments(
        self,
        lo: int,
        hi: int,
        grads: Sequence[Optional[Tuple[int, Range, int]]],
        models: Sequence[Optional[Tuple[int, Range, int]]],
    ) -> np.ndarray:
        """Segment table tiling ``[lo, hi)``.

        ``grads[i]`` / ``models[i]`` describe parameter ``i``'s gradient and
        model storage as ``(base_ptr, (flat_begin, flat_end), elem_bytes)``:
        element ``j`` of the flat range lives at
        ``base_ptr + (j - flat_begin) * elem_bytes``; ``None`` means no such
        storage.  Rows are cut wherever either storage starts or ends, so
        every row has one grad pointer and one model pointer (or NULL).
        """
        fast = self._segments_whole(lo, hi, grads, models)
        if fast is not None:
            return fast
        rows: List[Tuple[int, int, int, int]] = []

        def emit(b: int, e: int, g: int, m: int) -> None:
            if e <= b:
                return
            if rows and rows[-1][0] + rows[-1][1] == b and rows[-1][2] == 0 and rows[-1][3] == 0 \
                    and g == 0 and m == 0:
                prev = rows[-1]
                rows[-1] = (prev[0], prev[1] + (e - b), 0, 0)
                return
            rows.append((b, e - b, g, m))

        cursor = lo
        for i in range(len(self.numels)):
            pb, pe = _overlap(self.param_range(i), (lo, hi))
            if pb >= pe:
                continue
            cuts = {pb, pe}
            for store in (grads[i], models[i]):
                if store is not None:
                    sb, se = _overlap(store[1], (pb, pe))
                    if sb < se:
                        cuts.update((sb, se))
            pts = sorted(cuts)
            for b, e in zip(pts[:-1], pts[1:]):
                gp = mp = 0
                g = grads[i]
                if g is not None and g[1][0] <= b and e <= g[1][1]:
                    gp = g[0] + (b - g[1][0]) * g[2]
                m = models[i]
                if m is not None and m[1][0] <= b and e <= m[1][1]:
                    mp = m[0] + (b - m[1][0]) * m[2]
                if b > cursor:
                    emit(cursor, b, 0, 0)
                emit(b, e, gp, mp)
                cursor = e
        if cursor < hi:
            emit(cursor, hi, 0, 0)
        table = np.zeros((len(rows), 4), dtype=np.int64)
        if rows:
            table[:] = np.asarray(rows, dtype=np.uint64).astype(np.int64)
        return table

    def _segments_whole(self, lo, hi, grads, models) -> Optional[np.ndarray]:
        """Table for the common case: the range is the whole padded space and
        every storage covers exactly its parameter (one row per non-empty
        parameter plus one padding row).  ``None`` when that does not hold."""
        if lo != 0 or hi != self.numel_padded:
            return None
        rows = []
        for i, (off, n) in enumerate(zip(self.offsets, self.numels)):
            g, m = grads[i], models[i]
            if (g is not None and g[1] != (off, off + n)) or (m is not None and m[1] != (off, off + n)):
                return None
            if n:
                rows.append((off, n, g[0] if g is not None else 0, m[0] if m is not None else 0))
        if self.numel_padded > self.numel:
            rows.append((self.numel, self.numel_padded - self.numel, 0, 0))
        table = np.zeros((len(rows), 4), dtype=np.int64)
        if rows:
            table[:] = np.asarray(rows, dtype=np.uint64).astype(np.int64)
        return table


def check_table(table: np.ndarray, lo: int, hi: int) -> None:
    """Assert that a segment table tiles ``[lo, hi)`` (host-side guard run
    before every upload, so the kernels' segment walks stay in bounds)."""
    if hi <= lo:
        return
    if table.shape[0] == 0:
        raise RuntimeError("empty segment table for a non-empty range")
    begins, numels = table[:, 0], table[:, 1]
    if begins[0] != lo or begins[-1] + numels[-1] != hi:
        raise RuntimeError("segment table does not cover its range")
    if np.any(numels <= 0) or np.any(begins[1:] != begins[:-1] + numels[:-1]):
        raise RuntimeError("segment table rows are not contiguous")


class SegmentTable:
    """Device copies of the last few segment tables of one purpose.

    A table equal to a cached one is reused without any copy (the gradient
    addresses of consecutive windows often repeat).  A new table goes
    through a fresh pinned host tensor with a non-blocking copy on the
    current stream, replacing the least recently used entry; torch's host
    allocator keeps the staging memory until the copy has run, and the copy
    is stream-ordered before the kernels that read the table.  A replaced
    entry's device memory is overwritten in place only when every kernel
    that read it ran on the uploading stream (the copy queues behind them);
    otherwise the entry is dropped and a new one allocated.  Every use
    records the current stream on the device table, so that when an entry
    is dropped torch's caching allocator does not hand its memory to
    another stream before the kernels that read it have run.
    """

    SLOTS = 4

    def __init__(self, device: torch.device):
        self.device = device
        # (host table, device table, streams recorded on it); most recent last
        self._entries: List[Tuple[np.ndarray, torch.Tensor, set]] = []

    def upload(self, table: np.ndarray, stream: Optional[torch.cuda.Stream] = None) -> Tuple[int, int]:
        """Return (device pointer, row count) of ``table`` for kernels
        queued on ``stream`` (default: the current stream)."""
        n = int(table.shape[0])
        if n == 0:
            return 0, 0
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        for k, entry in enumerate(self._entries):
            host, dev, seen = entry
            if host.shape == table.shape and np.array_equal(host, table):
                self._entries.append(self._entries.pop(k))
                if stream.cuda_stream not in seen:
                    dev.record_stream(stream)
                    seen.add(stream.cuda_stream)
                return dev.data_ptr(), n
        staging = torch.empty((n, 4), dtype=torch.int64, pin_memory=True)
        staging.numpy()[:] = table
        dev = None
        seen = set()
        if len(self._entries) >= self.SLOTS:
            _, old, old_seen = self._entries.pop(0)
            # overwrite the evicted table in place only if every kernel that
            # read it was queued on this stream (the copy is then ordered
            # after them); a table another stream read is dropped instead,
            # and record_stream keeps its memory until that stream is done
            if old.shape[0] == n and old_seen <= {stream.cuda_stream}:
                dev, seen = old, old_seen
        with torch.cuda.stream(stream):
            if dev is None:
                dev = torch.empty((n, 4), dtype=torch.int64, device=self.device)
            dev.copy_(staging, non_blocking=True)
        if stream.cuda_stream not in seen:
            dev.record_stream(stream)
            seen.add(stream.cuda_stream)
        self._entries.append((table.copy(), dev, seen))
        return dev.data_ptr(), n


_ELEM_BYTES = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}


# State placement (``hip_boundary.state_spacing_gib``): AUTO_SPACING picks
# the window from the state's size (``auto_window``), 0 means separate
# allocations, a positive value is the window in bytes.
AUTO_SPACING = -1
_AUTO_WINDOW = 36 << 30
_AUTO_MIN_COLUMN = 256 << 20   # the Infinity Cache: smaller states stay cache resident
_AUTO_MAX_SHARE = 0.5      # of the free device memory
_ARENA_SLACK_BYTES = 1 << 30
_ARENA_ALIGN = 1 << 21

_log = logging.getLogger("minispeed_amd")


def state_sizes(layout: "FlatLayout", zero_stage: int) -> Tuple[int, int, int]:
    """Element counts of a group's (masters, exp_avg, exp_avg_sq): the
    masters cover the whole padded space, or only the owned shard when a
    ZeRO-3 partition will shrink them to it; the moments cover the owned
    range (optim/adam.py:38-56)."""
    n_own = layout.shard_end - layout.shard_start
    if zero_stage >= 3 and n_own != layout.numel_padded:
        return n_own, n_own, n_own
    return layout.numel_padded, n_own, n_own


def _column_bytes(sizes: Sequence[Sequence[int]]) -> List[int]:
    """Bytes of each state column (array j of every group, 2 MiB slots)."""
    k = len(sizes[0])
    if any(len(row) != k for row in sizes):
        raise ValueError("every group needs the same number of state arrays")
    return [sum(_round_up(4 * int(row[j]), _ARENA_ALIGN) for row in sizes) for j in range(k)]


def auto_window(sizes: Sequence[Sequence[int]], free_bytes: Optional[int] = None) -> int:
    """The window ``state_buffers`` uses by default: 36 GiB when the largest
    column holds between 256 MiB and 36 GiB and the arena (three windows,
    108 GiB) takes at most half of ``free_bytes`` (when given), else 0,
    separate allocations.  Smaller states largely stay in the 256 MB
    Infinity Cache between steps, where placement does not show (3.3M
    params: the same step time either way); at 124M params (0.5 GB arrays)
    the arena takes K3 from 0.61-0.63 to 0.53 ms; states over a window lie
    far apart anyway.  Window sizes over 1.3B-param steps, each size in
    every position of a sequence of processes on a box (the driver places
    an allocation according to what earlier processes left), mean step:
    32 GiB 6.16 ms, 34 GiB 6.19, 35 GiB 6.08, 36 GiB 6.10 (18 processes,
    6.07-6.16), 37 GiB 6.08, 38 GiB 6.17, 40 GiB 6.14, 42 GiB 6.11, 44 GiB
    6.09 (a 132 GiB arena, over half of the free memory beside a 1.3B
    model), 48 GiB 6.15 (6.06-6.26).  36 GiB sits inside the good 35-37
    GiB band."""
    if not sizes:
        return 0
    cols = _column_bytes(sizes)
    if not _AUTO_MIN_COLUMN <= max(cols) <= _AUTO_WINDOW:
        return 0
    if free_bytes is not None and len(cols) * _AUTO_WINDOW > _AUTO_MAX_SHARE * free_bytes:
        return 0
    return _AUTO_WINDOW


class StatePlacement:
    """Where :func:`place_state` put the masters and moments.

    ``window``: the arena's window in bytes, 0 for separate allocations.
    ``arena_bytes``: size of the arena's allocation (0 without one).
    ``held_bytes``: device memory the state buffers hold (their 2 MiB slots).
    ``returned_bytes``: the arena's part that is not state, handed back to
    torch's caching allocator as free blocks (0 when the arena could not be
    carved and stays one tensor).
    """

    __slots__ = ("window", "arena_bytes", "held_bytes", "returned_bytes")

    def __init__(self, window: int = 0, arena_bytes: int = 0, held_bytes: int = 0,
                 returned_bytes: int = 0):
        self.window = window
        self.arena_bytes = arena_bytes
        self.held_bytes = held_bytes
        self.returned_bytes = returned_bytes

    def __repr__(self) -> str:
        return (f"StatePlacement(window={self.window}, arena_bytes={self.arena_bytes}, "
                f"held_bytes={self.held_bytes}, returned_bytes={self.returned_bytes})")


_CARVE_TRIES = 64


def _expandable_segments() -> bool:
    conf = ",".join(os.environ.get(k, "") for k in ("PYTORCH_HIP_ALLOC_CONF", "PYTORCH_CUDA_ALLOC_CONF",
                                                   "PYTORCH_ALLOC_CONF"))
    return "expandable_segments:true" in conf.replace(" ", "").lower()


def _take_at(addr: int, nbytes: int, device: torch.device,
             spare: List[torch.Tensor]) -> Optional[torch.Tensor]:
    """A uint8 tensor of ``nbytes`` from torch's caching allocator that starts
    at ``addr``, or None.  The allocator serves a request from the smallest
    free block that fits, splitting it from its start; blocks it picks
    elsewhere are held in ``spare`` (released by the caller) so that the
    next request moves on to a larger one."""
    for _ in range(_CARVE_TRIES):
        reserved = torch.cuda.memory_reserved(device)
        t = torch.empty(nbytes, dtype=torch.uint8, device=device)
        if t.data_ptr() == addr:
            return t
        if torch.cuda.memory_reserved(device) > reserved:
            # a new segment: no free block of the pool serves the request
            # (e.g. max_split_size_mb keeps the arena's block from being
            # split); asking again would only allocate more
            del t
            return None
        spare.append(t)
    return None


def _carve(total: int, slots: Sequence[Tuple[int, int]],
           device: torch.device) -> Optional[List[torch.Tensor]]:
    """Tensors for ``slots`` ((byte offset, bytes), sorted, disjoint, 2 MiB
    multiples) at those offsets of one fresh allocation of ``total`` bytes,
    with every byte between and after them handed back to torch's caching
    allocator as free blocks of that allocation; None (nothing kept) when
    the allocator does not serve the requests from that allocation.

    The allocation is made whole, then freed into the allocator's pool (the
    allocator keeps it: its memory stays where the driver put it), and the
    slots and the gaps between them are requested in address order: each
    request splits the remaining free block from its start.  Then the gap
    tensors are dropped, so later tensors of the process (activations,
    gradients) can be served from the gaps."""
    arena = torch.empty(total, dtype=torch.uint8, device=device)
    base = arena.data_ptr()
    del arena
    spare: List[torch.Tensor] = []
    gaps: List[torch.Tensor] = []
    out: List[torch.Tensor] = []
    cursor = 0
    try:
        for off, nbytes in slots:
            if off > cursor:
                gap = _take_at(base + cursor, off - cursor, device, spare)
                if gap is None:
                    return None
                gaps.append(gap)
            t = _take_at(base + off, nbytes, device, spare)
            if t is None:
                return None
            out.append(t)
            cursor = off + nbytes
        return out
    finally:
        del spare, gaps


def state_buffers(sizes: Sequence[Sequence[int]], device: torch.device,
                  window: int) -> List[List[torch.Tensor]]:
    """The buffers of :func:`place_state` without the placement record."""
    return place_state(sizes, device, window)[0]


def place_state(sizes: Sequence[Sequence[int]], device: torch.device,
                window: int) -> Tuple[List[List[torch.Tensor]], StatePlacement]:
    """Zeroed fp32 buffers, ``sizes[g][j]`` elements for array j of group g,
    and where they were put.

    With ``window`` 0 they are separate allocations; ``AUTO_SPACING`` picks
    the window with :func:`auto_window`.  With a window they lie in one
    allocation of three windows, the state arena (:func:`arena_layout`):
    array j of every group starts at ``j * window``, the groups back to back
    at the same offsets in every window.  The fused AdamW kernel reads and
    writes the masters, exp_avg and exp_avg_sq at the same flat index in
    lockstep, and on MI355X that streams fastest when the three lie far
    apart in *physical* HBM (the same requests wait longer at the memory
    side when they collide on channels and banks).  Measured on the
    1.3B-param state (three 4.9 GiB arrays): K3 in the arena 5.64-5.74 ms
    with 36 GiB windows, 5.72-5.76 with 32 GiB ones; three separate
    allocations 6.1-6.9 ms; one allocation holding the three back to back
    6.0-6.3 ms, with staggers of 4 KiB to 1.5 GiB between them 6.2-6.3 ms;
    windows of 6 to 28 GiB inside one 64 GiB block 6.0-6.3 ms on one box.

    The arena is carved through torch's caching allocator (:func:`_carve`):
    the state keeps only its slots, and the rest of the arena -- the
    windows' unused part -- goes back to the allocator as free blocks that
    any later tensor allocated on the same stream can use.  If the
    allocator does not serve the slots from the arena (another free block
    of the pool fits better each time, or a request would need a new
    segment, as when ``max_split_size_mb`` keeps the arena's block whole),
    the arena stays one tensor; with expandable segments the state is
    allocated separately.  Columns larger than the window are allocated
    separately, and so is everything when the device lacks the free memory
    (with a log line).  The placement changes no result.
    """
    def plain() -> List[List[torch.Tensor]]:
        return [[torch.zeros(int(n), dtype=torch.float32, device=device) for n in row] for row in sizes]

    def held(rows) -> int:
        return sum(_round_up(4 * int(n), _ARENA_ALIGN) for row in rows for n in row)

    if window == AUTO_SPACING:
        window = auto_window(sizes, torch.cuda.mem_get_info(device)[0])
    layout = arena_layout(sizes, window)
    if layout is None:
        return plain(), StatePlacement(held_bytes=held(sizes))
    if _expandable_segments():
        _log.warning("state arena skipped: torch's expandable segments map memory page by page, "
                     "so the arena's windows would not be apart in physical memory; allocating the "
                     "masters and moments separately")
        return plain(), StatePlacement(held_bytes=held(sizes))
    starts, total = layout
    window = total // len(sizes[0])          # rounded up to 2 MiB by arena_layout
    free, _ = torch.cuda.mem_get_info(device)
    if free < total + _ARENA_SLACK_BYTES:
        _log.warning("state arena of %.1f GiB does not fit in %.1f GiB free device memory; "
                     "allocating the masters and moments separately", total / 2**30, free / 2**30)
        return plain(), StatePlacement(held_bytes=held(sizes))
    slots = sorted((a, _round_up(4 * int(n), _ARENA_ALIGN))
                   for row, row_starts in zip(sizes, starts) for n, a in zip(row, row_starts))
    carved = _carve(total, slots, device)
    if carved is not None:
        by_start = {a: t for (a, _), t in zip(slots, carved)}
        bufs = [[by_start[a][:4 * int(n)].view(torch.float32).zero_() for n, a in zip(row, row_starts)]
                for row, row_starts in zip(sizes, starts)]
        kept = sum(b for _, b in slots)
        placement = StatePlacement(window, total, kept, total - kept)
        _log.info("state arena: masters and moments in %d windows of %.0f GiB; %.2f GiB held by "
                  "the state, %.2f GiB returned to torch's allocator", len(sizes[0]),
                  window / 2**30, kept / 2**30, (total - kept) / 2**30)
        return bufs, placement
    _log.warning("state arena: torch's allocator did not serve the state slots from the arena; "
                 "keeping the whole %.0f GiB arena as one tensor", total / 2**30)
    arena = torch.empty(total, dtype=torch.uint8, device=device)
    bufs = [[arena[a:a + 4 * int(n)].view(torch.float32).zero_() for n, a in zip(row, row_starts)]
            for row, row_starts in zip(sizes, starts)]
    return bufs, StatePlacement(window, total, total, 0)


def arena_layout(sizes: Sequence[Sequence[int]],
                 window: int) -> Optional[Tuple[List[List[int]], int]]:
    """Byte offsets of ``state_buffers``' arena: ``(starts, total)`` with
    ``starts[g][j]`` the start of array j of group g (fp32 elements
    ``sizes[g][j]``) and ``total`` the arena size, ``k`` whole windows.  None
    for separate allocations (no window, nothing to place, or a column that
    does not fit in one window).  Windows and slots are rounded up to 2 MiB."""
    if window <= 0 or not sizes:
        return None
    cols = _column_bytes(sizes)
    k = len(cols)
    window = _round_up(int(window), _ARENA_ALIGN)
    if max(cols) > window:
        return None
    fill = [0] * k
    starts = []
    for row in sizes:
        starts.append([j * window + fill[j] for j in range(k)])
        for j, n in enumerate(row):
            fill[j] += _round_up(4 * int(n), _ARENA_ALIGN)
    return starts, k * window


# --------------------------------------------------------------------------
class FlatParamGroup:
    """One parameter group flattened into contiguous fp32 HBM buffers.

    Attributes and methods follow minispeed/flat.py:20-260; the data
    movement (ragged flatten, master->model casts) runs as HIP kernels of the
    boundary library.
    """

    def __init__(
        self,
        params: Sequence[nn.Parameter],
        *,
        rank: int,
        world_size: int,
        zero_stage: int,
        device: torch.device,
        state: Optional[Sequence[torch.Tensor]] = None,
    ):
        device = torch.device(device)
        if len(params) == 0:
            raise ValueError("FlatParamGroup requires at least one parameter")
        if device.type != "cuda":
            raise RuntimeError(
                f"FlatParamGroup on {device}: the flat buffers live in HBM and are "
                "updated by HIP kernels; use a ROCm GPU device"
            )
        self.params: List[nn.Parameter] = list(params)
        self.zero_stage = zero_stage
        self.device = device
        self.layout = FlatLayout(
            [p.numel() for p in self.params], rank=rank, world_size=world_size, zero_stage=zero_stage
        )
        lay = self.layout
        self.numel = lay.numel
        self.numel_padded = lay.numel_padded
        self.shard_size = lay.shard_size
        self.shard_start, self.shard_end = lay.shard_start, lay.shard_end

        # the masters and the AdamW moments of the owned range, which the
        # fused AdamW kernel streams together: given (placed by
        # state_buffers) or allocated here; the optimizer takes the moments
        sizes = state_sizes(lay, zero_stage)
        if state is None:
            state = state_buffers([sizes], device, 0)[0]
        index = device.index if device.index is not None else torch.cuda.current_device()
        if tuple(int(t.numel()) for t in state) != sizes or any(
                t.dtype != torch.float32 or t.device.type != "cuda" or t.device.index != index
                for t in state):
            raise ValueError(f"state buffers must be fp32 on cuda:{index} with {sizes} elements")
        self.state_placement = StatePlacement(held_bytes=sum(_round_up(4 * n, _ARENA_ALIGN) for n in sizes))
        self._master_shard: Optional[torch.Tensor] = None
        if sizes[0] != self.numel_padded:
            # the masters shrink to the owned range in partition_params
            self._master_shard, exp_avg, exp_avg_sq = state
            self.data = torch.zeros(self.numel_padded, dtype=torch.float32, device=device)
        else:
            self.data, exp_avg, exp_avg_sq = state
        self._moments: Optional[Tuple[torch.Tensor, torch.Tensor]] = (exp_avg, exp_avg_sq)
        # True while `grad` is logically zero but its memory still holds the
        # last boundary's values (see the `grad` property)
        self._grad_stale = False
        self._grad: Optional[torch.Tensor] = (
            None if zero_stage >= 3 else torch.zeros(self.numel_padded, dtype=torch.float32, device=device)
        )
        self.grad_shard: Optional[torch.Tensor] = (
            torch.zeros(self.shard_size, dtype=torch.float32, device=device) if zero_stage >= 2 else None
        )
        self._offsets: List[Tuple[int, nn.Parameter]] = list(zip(lay.offsets, self.params))
        self._numels: List[int] = list(lay.numels)
        self._numels_np = np.asarray(self._numels, dtype=np.int64)
        self._shapes: List[Tuple[int, ...]] = [tuple(p.shape) for p in self.params]
        self._partitioned = False
        # ZeRO-3: the model-dtype copy of the owned shard.  Freed parameters
        # are flat views into it; at world size 1 the gathered parameters are
        # shaped views into it as well, so gather and free move no data.
        self.model_shard: Optional[torch.Tensor] = None
        self._full_model: Optional[torch.Tensor] = None   # gathered buffer, world size > 1
        self._materialized = False
        self._shard_views: Optional[List[torch.Tensor]] = None   # placeholders, built once
        self._full_views: Optional[List[torch.Tensor]] = None    # gathered, world size 1
        # (address and version of `data`, summed parameter versions) when
        # model_shard last received the cast of `data`; None once the masters
        # changed without that cast
        self._model_token: Optional[Tuple[int, int, int]] = None
        # True while `grad` / `grad_shard` may hold non-zero values; lets
        # zero_grad skip clearing buffers nothing wrote.
        self._grad_dirty = False
        self._shard_dirty = False
        self._tables = {}
        self._rows = None   # static (begin, numel) rows of the whole-range table
        self._device_index = device.index if device.index is not None else torch.cuda.current_device()

    # ------------------------------------------------------------- ranges
    @property
    def master_range(self) -> Range:
        if self._partitioned:
            return self.shard_start, self.shard_end
        return 0, self.numel_padded

    @property
    def own_range(self) -> Range:
        return self.shard_start, self.shard_end

    def _pdata_range(self, offset: int, n: int, p: nn.Parameter) -> Range:
        """Flat range covered by ``p.data``: the whole parameter, or the
        owned slice of a ZeRO-3 placeholder (flat.py:103-113)."""
        k = p.numel()
        if k == n:
            return offset, offset + n
        start = max(offset, self.shard_start)
        return start, start + k

    def model_dtype(self) -> torch.dtype:
        d = self.params[0].dtype
        if any(p.dtype != d for p in self.params):
            dtypes = sorted({str(p.dtype) for p in self.params})
            raise TypeError(f"parameters of one group must share a dtype, got {dtypes}")
        return d

    def table(self, key: str) -> SegmentTable:
        t = self._tables.get(key)
        if t is None:
            t = self._tables[key] = SegmentTable(self.device)
        return t

    def model_storages(self) -> List[Optional[tuple]]:
        out = []
        for (offset, p), n in zip(self._offsets, self._numels):
            if p.device.type != "cuda":
                raise RuntimeError(f"parameter on {p.device}; the flat group lives on a HIP device")
            if not p.is_contiguous():
                raise RuntimeError("parameter data must be contiguous")
            out.append((p.data_ptr(), self._pdata_range(offset, n, p), p.element_size()))
        return out

    # -------------------------------------------------------- conversions
    def _model_table(self, lo: int, hi: int, as_source: bool) -> np.ndarray:
        """Segment table of ``[lo, hi)`` over the parameters' storage, in
        the gradient column (the source K1 widens) or in the model column
        (the target K4 narrows into).  The whole padded range of full-size
        parameters takes the cached rows and the C++ pointer walk; anything
        else (a shard, ZeRO-3 placeholders) the general table."""
        if (lo, hi) == (0, self.numel_padded) and not self._partitioned:
            ptrs = self.model_pointers()
            if as_source:
                return self.boundary_table(lo, hi, ptrs, None, _ELEM_BYTES[self.model_dtype()])
            return self.boundary_table(lo, hi, None, ptrs)
        stores = self.model_storages()
        none = [None] * len(stores)
        table = (self.layout.segments(lo, hi, stores, none) if as_source
                 else self.layout.segments(lo, hi, none, stores))
        check_table(table, lo, hi)
        return table

    @torch.no_grad()
    def copy_model_to_flat(self) -> None:
        """Snapshot the parameters covered by ``master_range`` into ``data``
        (flat.py:115-131): a ragged widening copy on the GPU."""
        ms, me = self.master_range
        dtype = self.model_dtype()
        table = self._model_table(ms, me, as_source=True)
        ptr, n = self.table("to_flat").upload(table)
        lib = _native.load()
        rc = lib.ms_grad_stats(
            ptr, n, _native.ms_dtype(dtype), ms, me, ms, me, 0, 1.0,
            self.data.data_ptr(), None, None, 0, None, None, 0, _native.stream_handle(self.device),
        )
        _native.check(rc, "ms_grad_stats(flatten)")
        self.masters_written()

    @torch.no_grad()
    def copy_flat_to_model(self, full_flat: Optional[torch.Tensor] = None) -> None:
        """Cast fp32 masters into the covered parameter elements
        (flat.py:133-154): ``full_flat`` covers ``[0, numel_padded)``; by
        default ``data`` over ``master_range`` is used."""
        if full_flat is not None:
            buf, base = full_flat, 0
        else:
            buf, base = self.data, self.master_range[0]
        _native.require_hip_tensor(buf, "flat master buffer")
        end = base + buf.numel()
        dtype = self.model_dtype()
        into_shard = self._params_view_model_shard()
        if into_shard and (base, end) == (self.shard_start, self.shard_end):
            # the parameters tile model_shard: one contiguous segment
            table = np.array([[base, end - base, 0, self.model_shard.data_ptr()]], dtype=np.int64)
            check_table(table, base, end)
        else:
            table = self._model_table(base, end, as_source=False)
        ptr, n = self.table("to_model").upload(table)
        rc = _native.load().ms_cast_to_model(
            buf.data_ptr(), base, end, ptr, n, _native.ms_dtype(dtype),
            _native.stream_handle(self.device),
        )
        _native.check(rc, "ms_cast_to_model")
        if into_shard:
            if full_flat is None or full_flat is self.data:
                self.model_written()
            else:
                self.masters_written()   # model_shard now holds the cast of another buffer

    # ---------------------------------------------------- stage-3 params
    @torch.no_grad()
    def partition_params(self) -> None:
        """Keep only the owned master shard; parameters become flat
        placeholders of their owned slices (flat.py:157-172).  The
        placeholders are views into one model-dtype buffer of the shard,
        ``model_shard``."""
        if self._partitioned:
            return
        if self._master_shard is not None:
            self.data = self._master_shard.copy_(self.data[self.shard_start:self.shard_end])
            self._master_shard = None
        # (otherwise the shard is the whole buffer, kept where it was allocated)
        self.model_shard = torch.empty(self.numel_shard(), dtype=self.model_dtype(), device=self.device)
        self._partitioned = True
        self._materialized = True      # full-shaped until dematerialized
        self.dematerialize_params()
        self.copy_flat_to_model()

    @torch.no_grad()
    def materialize_params(self) -> None:
        """Give the parameters their full shapes (flat.py:174-182).  At world
        size 1 they become views into ``model_shard``, which already holds the
        cast of the masters whenever :meth:`model_is_fresh`; with more ranks
        they are views into one full model-dtype buffer that the caller
        fills (the all-gather target)."""
        if not self._partitioned or self._materialized:
            return
        if self.whole_range:
            if self._full_views is None:
                self._full_views = [self.model_shard[off:off + n].view(shape) for off, n, shape
                                    in zip(self.layout.offsets, self._numels, self._shapes)]
            views = self._full_views
        else:
            base = self._full_model = torch.empty(self.numel_padded, dtype=self.model_shard.dtype,
                                                  device=self.device)
            views = [base[off:off + n].view(shape) for off, n, shape
                     in zip(self.layout.offsets, self._numels, self._shapes)]
        for p, view in zip(self.params, views):
            p.data = view
        self._materialized = True

    @torch.no_grad()
    def dematerialize_params(self) -> None:
        """Parameters drop back to flat views of their owned slices in
        ``model_shard`` (flat.py:184-193); nothing is allocated or copied."""
        if not self._partitioned or not self._materialized:
            return
        if self._shard_views is None:
            ms, me = self.shard_start, self.shard_end
            self._shard_views = []
            for off, n in zip(self.layout.offsets, self._numels):
                lo, hi = _overlap((off, off + n), (ms, me))
                self._shard_views.append(self.model_shard[lo - ms:hi - ms])
        for p, view in zip(self.params, self._shard_views):
            p.data = view
        self._full_model = None
        self._materialized = False

    def _params_view_model_shard(self) -> bool:
        """The parameters' storage is exactly ``model_shard`` (freed, or
        gathered at world size 1)."""
        return self._partitioned and (not self._materialized or self.whole_range)

    def _token(self) -> Tuple[int, int, int]:
        # in-place writes to `data` or to any parameter (placeholder or
        # gathered view) advance these torch version counters
        return (self.data.data_ptr(), self.data._version,
                sum(p._version for p in self.params))

    def model_is_fresh(self) -> bool:
        """``model_shard`` holds the model-dtype cast of the current masters
        and nothing has been written into the parameters since."""
        return self._model_token is not None and self._model_token == self._token()

    def model_written(self) -> None:
        """Record that ``model_shard`` was just given the cast of ``data``."""
        if self._partitioned:
            self._model_token = self._token()

    def masters_written(self) -> None:
        """Record that ``data`` changed without the cast into ``model_shard``
        (kernels write through raw addresses, which torch's version counter
        does not see)."""
        self._model_token = None

    # ------------------------------------------------ boundary pointers
    @property
    def whole_range(self) -> bool:
        """The owned range is the whole padded space (world size 1)."""
        return self.shard_start == 0 and self.shard_end == self.numel_padded

    def _check_grad(self, g: torch.Tensor, n: int) -> torch.Tensor:
        if g.numel() != n:
            raise RuntimeError(f"gradient of a parameter has {g.numel()} elements, expected {n}")
        if g.dtype not in _ELEM_BYTES:
            raise TypeError(f"gradient dtype {g.dtype} is not float32, float16 or bfloat16")
        if g.device != self.device:
            raise RuntimeError(f"gradient on {g.device}, expected {self.device}")
        return g.contiguous()

    def grad_pointers(self) -> Tuple[np.ndarray, List[Optional[torch.Tensor]], Optional[int]]:
        """Device address of every parameter's gradient (0: no gradient),
        the tensors behind them, which the caller keeps alive until the
        kernels reading them are queued, and the ``MS_DTYPE_*`` the
        addresses hold (``None``: the parameters' dtype).

        The addresses are an int64 array with one extra trailing 0 (the
        padding row's).  Every gradient is checked for its size, device and
        layout; the C++ walk covers the common case (every gradient in the
        parameters' dtype) and this loop takes over at the first gradient it
        does not accept, to raise, or to make a contiguous copy.  A gradient
        in another floating dtype is widened like minispeed's flatten
        (flat.py:209-212): then every gradient of the group is widened into
        one fp32 buffer and the addresses point into it.
        """
        n_params = len(self.params)
        ptrs = np.zeros(n_params + 1, dtype=np.int64)
        bad, keep = _walk().grad_pointers(self.params, self._numels_np, self._device_index, ptrs)
        if bad < 0:
            return ptrs, keep, None
        dtype = self.params[0].dtype
        index = self._device_index
        mixed = False
        for k in range(bad, n_params):
            g, n = self.params[k].grad, self._numels[k]
            if g is not None:
                # dtypes are singletons; get_device() is -1 for host tensors
                if g.dtype is not dtype or g.numel() != n or g.get_device() != index \
                        or not g.is_contiguous():
                    g = self._check_grad(g, n)
                    mixed |= g.dtype is not dtype
                ptrs[k] = g.data_ptr()
            keep.append(g)
        if not mixed:
            return ptrs, keep, None
        return self._widen_grads(keep)

    def _widen_grads(self, grads: List[Optional[torch.Tensor]]):
        """Every gradient widened exactly into its parameter's slice of one
        fp32 buffer (the opt-in accumulation kernel with ``first`` set):
        addresses into it, the tensors to keep, and ``MS_DTYPE_F32``."""
        from .contiguous import ACCUM_ROW, accumulate_rows
        buf = torch.empty(self.numel, dtype=torch.float32, device=self.device)
        base = buf.data_ptr()
        ptrs = np.zeros(len(self.params) + 1, dtype=np.int64)
        by_dtype = {}
        for k, (g, off, n) in enumerate(zip(grads, self.layout.offsets, self._numels)):
            if g is None or n == 0:
                continue
            by_dtype.setdefault(g.dtype, []).append((base + 4 * off, g.data_ptr(), n))
            ptrs[k] = base + 4 * off
        for dtype, items in by_dtype.items():
            rows = np.zeros(len(items), dtype=ACCUM_ROW)
            rows["dst"], rows["src"], rows["numel"] = zip(*items)
            rows["first"] = 1
            accumulate_rows(rows, _native.ms_dtype(dtype), self.device)
        return ptrs, [*grads, buf], _native.DTYPE_F32

    def model_pointers(self) -> np.ndarray:
        """Device address of every parameter's storage (the cast target),
        with a trailing 0 like :meth:`grad_pointers`; every parameter must
        have the group's dtype, be contiguous and live on its device."""
        ptrs = np.zeros(len(self.params) + 1, dtype=np.int64)
        bad = _walk().model_pointers(self.params, self._device_index, ptrs)
        if bad >= 0:
            p = self.params[bad]
            self.model_dtype()   # raises for mixed dtypes
            raise RuntimeError(
                f"parameter storage must be contiguous on {self.device}, got {p.device}"
                + ("" if p.is_contiguous() else " (non-contiguous)"))
        return ptrs

    def boundary_table(self, lo: int, hi: int, gptrs: Optional[List[int]],
                       mptrs: Optional[List[int]], grad_elem_bytes: Optional[int] = None) -> np.ndarray:
        """Segment table of ``[lo, hi)`` with the given grad / model
        addresses (``None``: no such storage); the gradient storage holds
        ``grad_elem_bytes``-byte elements (default: the parameters' size;
        4 for the fp32 sums of contiguous gradients).  For the whole padded
        range with full-size parameters the rows are static and only the two
        pointer columns are filled in."""
        n_params = len(self.params)
        full = True
        if mptrs is not None and self._partitioned:   # ZeRO-3 placeholders may be slices
            full = all(p.numel() == n for p, n in zip(self.params, self._numels))
        if lo == 0 and hi == self.numel_padded and full:
            if self._rows is None:
                rows, idx = [], []
                for i, (off, n) in enumerate(zip(self.layout.offsets, self._numels)):
                    if n:
                        rows.append((off, n))
                        idx.append(i)
                if self.numel_padded > self.numel:
                    rows.append((self.numel, self.numel_padded - self.numel))
                    idx.append(n_params)
                base = np.zeros((len(rows), 4), dtype=np.int64)
                base[:, :2] = np.asarray(rows, dtype=np.int64).reshape(-1, 2)
                check_table(base, 0, self.numel_padded)
                self._rows = (base, np.asarray(idx, dtype=np.int64))
            base, idx = self._rows
            table = base.copy()
            if gptrs is not None:
                table[:, 2] = _with_pad_slot(gptrs, n_params)[idx]
            if mptrs is not None:
                table[:, 3] = _with_pad_slot(mptrs, n_params)[idx]
            return table
        esz_g = grad_elem_bytes or _ELEM_BYTES[self.model_dtype()]
        grads = [None] * n_params
        models = [None] * n_params
        for i, ((off, p), n) in enumerate(zip(self._offsets, self._numels)):
            if gptrs is not None and gptrs[i]:
                grads[i] = (gptrs[i], (off, off + n), esz_g)
            if mptrs is not None and mptrs[i]:
                models[i] = (mptrs[i], self._pdata_range(off, n, p), p.element_size())
        table = self.layout.segments(lo, hi, grads, models)
        check_table(table, lo, hi)
        return table

    # ----------------------------------------------------------- grads
    @property
    def grad(self) -> Optional[torch.Tensor]:
        """The fp32 flat gradient (flat.py:61-73).  After ``zero_grad`` it
        reads as zeros, as in the reference; the clearing itself waits until
        something reads the buffer, because the boundary that writes it
        next (the flattening scan) overwrites every element anyway.  A
        training loop that never looks at ``grad`` therefore pays no
        clearing pass (4 B/param per step)."""
        if self._grad_stale:
            self._grad.zero_()
            self._grad_stale = False
        return self._grad

    @grad.setter
    def grad(self, value: Optional[torch.Tensor]) -> None:
        self._grad = value
        self._grad_stale = False

    def flat_grad_for_overwrite(self) -> torch.Tensor:
        """The flat gradient buffer (allocated if absent) for a kernel that
        writes every element of it: a pending clear is dropped, not done."""
        if self._grad is None:
            self._grad = torch.empty(self.numel_padded, dtype=torch.float32, device=self.device)
        self._grad_stale = False
        self._grad_dirty = True
        return self._grad

    def release_grads(self) -> None:
        for p in self.params:
            p.grad = None

    @torch.no_grad()
    def flatten_grads(self) -> None:
        """``param.grad`` -> fp32 flat ``grad`` (flat.py:196-213); params
        without a gradient contribute zeros, every floating dtype is widened
        exactly, ``param.grad`` is released."""
        flat = self.flat_grad_for_overwrite()
        # the C++ walk of the gradients; a gradient in another floating dtype
        # makes every address point into one exactly widened fp32 buffer
        ptrs, keep, gdtype = self.grad_pointers()
        if gdtype is None:
            gdtype = _native.ms_dtype(self.model_dtype())
        gbytes = 4 if gdtype == _native.DTYPE_F32 else 2
        table = self.boundary_table(0, self.numel_padded, ptrs, None, gbytes)
        ptr, n = self.table("flatten").upload(table)
        rc = _native.load().ms_grad_stats(
            ptr, n, gdtype, 0, self.numel_padded, 0, 0, 0, 1.0, flat.data_ptr(),
            None, None, 0, None, None, 0, _native.stream_handle(self.device),
        )
        _native.check(rc, "ms_grad_stats(flatten)")
        self.release_grads()
        # the gradients may have been allocated on another stream: their
        # memory must not be reused there before the kernel above has read it
        record_streams(keep, torch.cuda.current_stream(self.device))
        del keep

    @torch.no_grad()
    def zero_grad(self) -> None:
        """flat.py:215-223.  Buffers nothing wrote are already zero and are
        not cleared again; a written ``grad`` is cleared when it is next
        read (the ``grad`` property), ``grad_shard`` at once."""
        if self._grad is not None:
            if self.zero_stage >= 3:
                self.grad = None
            elif self._grad_dirty:
                self._grad_stale = True
        if self.grad_shard is not None and self._shard_dirty:
            self.grad_shard.zero_()
        self._grad_dirty = False
        self._shard_dirty = False

    def grad_for_shard(self) -> torch.Tensor:
        if self.grad_shard is not None:
            return self.grad_shard
        return self.grad[self.shard_start:self.shard_end]

    # The unfused step pieces of the reference (flat.py:232-257).  The fused
    # boundary does all three inside K1-K3 without a flat gradient; these
    # work on the materialized ``grad`` / ``grad_shard`` (after
    # ``flatten_grads``) for callers that drive the steps one by one.
    def local_grad_sumsq(self) -> torch.Tensor:
        """Sum of squares of the owned gradient slice, a 0-dim fp32 device
        tensor (flat.py:232-234)."""
        from .boundary import sumsq_device
        return sumsq_device(self.grad_for_shard())

    @torch.no_grad()
    def unscale_grads(self, scale: float) -> None:
        """``grad /= scale`` over the whole flat gradient (flat.py:243-247)."""
        if scale == 1.0 or self._grad is None or self._grad_stale:
            return      # nothing, or zeros: dividing them changes nothing
        from .boundary import scale_in_place
        scale_in_place(self._grad, _native.SCALE_DIVIDE, scale)

    @torch.no_grad()
    def scale_grads(self, factor: float) -> None:
        """Multiply the owned gradients by a clip coefficient
        (flat.py:249-257): ``grad_shard`` if it exists, else ``grad``."""
        if factor == 1.0:
            return
        target = self.grad_shard if self.grad_shard is not None else self.grad
        if target is None:
            return
        from .boundary import scale_in_place
        scale_in_place(target, _native.SCALE_MULTIPLY, factor)
        if target is self.grad_shard:
            self._shard_dirty = True
        else:
            self._grad_dirty = True

    @property
    def shard(self) -> torch.Tensor:
        if self._partitioned:
            return self.data
        return self.data[self.shard_start:self.shard_end]

    def numel_shard(self) -> int:
        return self.shard_end - self.shard_start

    def take_moment_buffers(self) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """The zeroed fp32 (exp_avg, exp_avg_sq) buffers of the owned range
        allocated next to the masters; handed out once, then None."""
        moments, self._moments = self._moments, None
        return moments


def build_flat_groups(
    param_groups: Iterable[dict],
    *,
    rank: int,
    world_size: int,
    zero_stage: int,
    device: torch.device,
    state_spacing: int = 0,
) -> Tuple[List[FlatParamGroup], List[dict]]:
    """torch-style group dicts -> FlatParamGroups + option dicts
    (flat.py:263-291).  The groups' masters and moments are placed together
    by ``place_state`` (one arena of ``state_spacing``-byte windows, or
    separate allocations when it is 0); every group records the result in
    ``state_placement``."""
    device = torch.device(device)
    kept: List[Tuple[List[nn.Parameter], dict]] = []
    for group in param_groups:
        params = [p for p in group["params"] if p.requires_grad]
        if not params:
            continue
        kept.append((params, {k: v for k, v in group.items() if k != "params"}))
    if not kept:
        raise ValueError("No trainable parameters found")
    sizes = [state_sizes(FlatLayout([p.numel() for p in params], rank=rank, world_size=world_size,
                                    zero_stage=zero_stage), zero_stage)
             for params, _ in kept]
    states, placement = place_state(sizes, device, state_spacing)
    flat_groups = [
        FlatParamGroup(params, rank=rank, world_size=world_size, zero_stage=zero_stage, device=device,
                       state=state)
        for (params, _), state in zip(kept, states)
    ]
    for g in flat_groups:
        g.state_placement = placement
    return flat_groups, [opts for _, opts in kept]
