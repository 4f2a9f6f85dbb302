"""Flat-group index math and segment tables on the CPU (no device memory).

Closed forms: offsets are prefix sums, the padded size is the next multiple
of world_size, rank r owns [r*S, (r+1)*S) for stage >= 1 and everything at
stage 0 (minispeed/flat.py:16-17, 50-59); a segment table tiles its range
exactly and maps every element to the right address.  Shard-size checks
follow minispeed's tests/test_distributed.py:179-193 and
tests/test_zero3.py:94-147.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from minispeed_amd.flat import FlatLayout, check_table


def _brute_map(lay: FlatLayout, lo, hi, grads, models):
    """element -> (grad address, model address) by direct search."""
    out = {}
    for i in range(lo, hi):
        g = m = 0
        for k, (off, n) in enumerate(zip(lay.offsets, lay.numels)):
            if off <= i < off + n:
                if grads[k] is not None and grads[k][1][0] <= i < grads[k][1][1]:
                    g = grads[k][0] + (i - grads[k][1][0]) * grads[k][2]
                if models[k] is not None and models[k][1][0] <= i < models[k][1][1]:
                    m = models[k][0] + (i - models[k][1][0]) * models[k][2]
        out[i] = (g, m)
    return out


def _table_map(table):
    out = {}
    for b, n, g, m in table.tolist():
        for j in range(n):
            out[b + j] = (g + j * _table_map.esize_g if g else 0, m + j * _table_map.esize_m if m else 0)
    return out


@pytest.mark.parametrize("numels,world,rank,stage", [
    ([35, 3], 2, 1, 3),
    ([17 * 9] * 3, 2, 1, 2),
    ([17 * 9] * 3, 1, 0, 0),
    ([5, 0, 7, 1, 11], 3, 2, 1),
    ([4096, 8, 10240], 8, 5, 3),
])
def test_layout_closed_forms(numels, world, rank, stage):
    lay = FlatLayout(numels, rank=rank, world_size=world, zero_stage=stage)
    total = sum(numels)
    assert lay.offsets == [sum(numels[:i]) for i in range(len(numels))]
    assert lay.numel == total
    assert lay.numel_padded % world == 0 and 0 <= lay.numel_padded - total < world
    assert lay.shard_size * world == lay.numel_padded
    if stage >= 1:
        assert (lay.shard_start, lay.shard_end) == (rank * lay.shard_size, (rank + 1) * lay.shard_size)
    else:
        assert (lay.shard_start, lay.shard_end) == (0, lay.numel_padded)


def test_layout_rejects_bad_arguments():
    with pytest.raises(ValueError):
        FlatLayout([], rank=0, world_size=1, zero_stage=0)
    with pytest.raises(ValueError):
        FlatLayout([3], rank=2, world_size=2, zero_stage=1)


def test_llama_one_eighth_shard_size():
    from minispeed_amd.workloads import numel, shapes_of

    shapes = shapes_of("llama3-8b")
    n = [int(np.prod(s)) for s in shapes]
    lay = FlatLayout(n, rank=3, world_size=8, zero_stage=3)
    assert numel(shapes) == 8_030_261_248 and len(shapes) == 291
    assert lay.shard_size == 1_003_782_656
    assert lay.shard_start == 3 * 1_003_782_656


@pytest.mark.parametrize("case", range(6))
def test_segment_table_maps_every_element(case):
    rng = np.random.default_rng(case)
    numels = [int(x) for x in rng.integers(0, 40, size=int(rng.integers(1, 7)))]
    if sum(numels) == 0:
        numels[0] = 5
    world = int(rng.integers(1, 4))
    rank = int(rng.integers(0, world))
    lay = FlatLayout(numels, rank=rank, world_size=world, zero_stage=3)
    esize_g, esize_m = 2, 4
    grads, models = [], []
    for k, (off, n) in enumerate(zip(lay.offsets, lay.numels)):
        grads.append(None if rng.random() < 0.3 else (10_000 * (k + 1), (off, off + n), esize_g))
        if rng.random() < 0.5:   # a placeholder of the owned slice, as at ZeRO-3
            a, b = max(off, lay.shard_start), min(off + n, lay.shard_end)
            models.append((1_000_000 * (k + 1), (a, max(a, b)), esize_m) if b > a else None)
        else:
            models.append((2_000_000 * (k + 1), (off, off + n), esize_m))
    _table_map.esize_g, _table_map.esize_m = esize_g, esize_m
    for lo, hi in [(0, lay.numel_padded), (lay.shard_start, lay.shard_end)]:
        table = lay.segments(lo, hi, grads, models)
        check_table(table, lo, hi)
        assert _table_map(table) == _brute_map(lay, lo, hi, grads, models)


def test_whole_range_fast_table_equals_general_table():
    numels = [35, 3, 2112, 0, 1, 129]
    lay = FlatLayout(numels, rank=0, world_size=1, zero_stage=0)
    grads = [(1000 * (k + 1), (o, o + n), 2) if k != 1 else None
             for k, (o, n) in enumerate(zip(lay.offsets, lay.numels))]
    models = [(5000 * (k + 1), (o, o + n), 2) for k, (o, n) in enumerate(zip(lay.offsets, lay.numels))]
    fast = lay.segments(0, lay.numel_padded, grads, models)
    _table_map.esize_g = _table_map.esize_m = 2
    assert _table_map(fast) == _brute_map(lay, 0, lay.numel_padded, grads, models)
    assert fast.shape[0] == sum(1 for n in numels if n)


def test_check_table_rejects_gaps_and_overlaps():
    good = np.array([[0, 4, 0, 0], [4, 6, 0, 0]], dtype=np.int64)
    check_table(good, 0, 10)
    for bad in ([[0, 4, 0, 0], [5, 5, 0, 0]], [[0, 4, 0, 0], [3, 7, 0, 0]],
                [[0, 4, 0, 0], [4, 0, 0, 0], [4, 6, 0, 0]], [[1, 9, 0, 0]]):
        with pytest.raises(RuntimeError):
            check_table(np.array(bad, dtype=np.int64), 0, 10)
    with pytest.raises(RuntimeError):
        check_table(np.zeros((0, 4), dtype=np.int64), 0, 1)
    check_table(np.zeros((0, 4), dtype=np.int64), 3, 3)


def test_gpt_workload_shapes_match_reference_counts():
    from minispeed_amd.workloads import numel, shapes_of

    expect = {"tiny-lm-3.3m": (52, 3_323_392), "gpt2-124m": (148, 124_439_808),
              "gpt-350m": (292, 354_823_168), "gpt-1.3b": (292, 1_315_723_264)}
    for name, (ntens, n) in expect.items():
        s = shapes_of(name)
        assert (len(s), numel(s)) == (ntens, n)
        d = s[2][0]
        for block in itertools.islice(zip(*[iter(s[2:-2])] * 12), 2):
            assert block[2] == (3 * d, d) and block[8] == (4 * d, d) and block[10] == (d, 4 * d)


def test_state_arena_layout():
    """Array j of every group at window j, groups back to back at equal
    offsets, 2 MiB slots, k whole windows; None when a column overflows its
    window."""
    from minispeed_amd.flat import arena_layout

    mib = 1 << 20
    starts, total = arena_layout([[1000, 700, 700], [mib // 4 + 3, mib // 4 + 3, 5]], 8 * mib)
    assert total == 3 * 8 * mib
    assert starts == [[0, 8 * mib, 16 * mib], [2 * mib, 10 * mib, 18 * mib]]
    # an 11 MiB window is rounded up to 12 MiB
    assert arena_layout([[1, 1, 1]], 11 * mib) == ([[0, 12 * mib, 24 * mib]], 36 * mib)
    # one column just fits, then overflows
    assert arena_layout([[2 * mib, 1, 1], [2 * mib, 1, 1]], 4 * mib * 4) is not None
    assert arena_layout([[3 * mib, 1, 1]], 8 * mib) is None          # 12 MiB > 8 MiB
    assert arena_layout([[1, 1, 1]], 0) is None
    assert arena_layout([], 8 * mib) is None
    import pytest
    with pytest.raises(ValueError):
        arena_layout([[1, 1, 1], [1, 1]], 8 * mib)
    # the 1.3B GPT state at 32 GiB: three windows, 96 GiB
    n = 1_315_723_264
    starts, total = arena_layout([[n, n, n]], 32 << 30)
    assert starts == [[0, 32 << 30, 64 << 30]] and total == 96 << 30


def test_auto_window_is_36_gib_for_states_of_256_mib_to_36_gib_per_array():
    from minispeed_amd.flat import auto_window

    gib = 1 << 30
    n13 = 1_315_723_264                                       # 1.3B GPT: 4.9 GiB arrays
    assert auto_window([[n13, n13, n13]]) == 36 * gib
    n8 = 8_030_261_248                                        # Llama-3-8B whole: 29.9 GiB
    assert auto_window([[n8, n8, n8]]) == 36 * gib
    assert auto_window([[3_323_392] * 3]) == 0                # tiny LM: 13 MB arrays
    assert auto_window([[124_439_808] * 3]) == 36 * gib       # GPT-2 small: 0.46 GiB arrays
    assert auto_window([[(256 << 20) // 4] * 3]) == 36 * gib  # exactly 256 MiB
    assert auto_window([[(256 << 20) // 4 - (1 << 20)] * 3]) == 0    # 252 MiB
    assert auto_window([[n8 + n13] * 3]) == 36 * gib          # 34.8 GiB: fits a window
    assert auto_window([[(36 * gib) // 4] * 3]) == 36 * gib   # exactly 36 GiB
    assert auto_window([[(36 * gib) // 4 + 1] * 3]) == 0      # 36 GiB + one element (a 2 MiB slot)
    assert auto_window([[n8 + 2 * n13] * 3]) == 0             # 39.7 GiB: separate
    assert auto_window([[n13, n13, n13], [n13, n13, n13]]) == 36 * gib     # 9.8 GiB columns
    assert auto_window([]) == 0
    # the 108 GiB arena only when it takes at most half of the free memory
    assert auto_window([[n13, n13, n13]], free_bytes=216 * gib) == 36 * gib
    assert auto_window([[n13, n13, n13]], free_bytes=215 * gib) == 0
