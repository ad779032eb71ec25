"""The host's prefill work-unit plan (fa_prefill_plan_units, csrc/prefill.hip),
checked on the CPU: no GPU is needed to plan.

When a prefill call brings its workspace, the library may split the heaviest
(query tile, head) items into two key chunks and give each CU up to two
units. A wrong plan would leave output rows unwritten or merge a chunk
twice, so every plan is checked for: each item covered exactly once, whole
or as both of its chunks with one partial slot; at most two units per block;
blocks on the XCD of their heavier unit where the plan allows; a busiest-CU
cost no worse than running every item whole. The unit costs restate the
planner's model (tiles over the two key halves, plus 3 steps per unit and 1
more per chunk) and the expected split counts are that model's own choice.
"""

import ctypes
import os
from collections import defaultdict

import pytest

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), os.pardir,
                   "flash-attention-cuda_amd", "flashattn_cuda", "libflashattn_hip.so")
NO_UNIT = 0xFFFFFFFF
ROWS = 128  # query rows per item


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run flash-attention-cuda_amd/build.py")
    return ctypes.CDLL(LIB)


def plan(lib, bh, seq, causal, d, group=1, cu=256):
    cap = 2 * 384
    units = (ctypes.c_uint * cap)()
    nb, ns = ctypes.c_int(), ctypes.c_int()
    rc = lib.fa_prefill_plan_units(bh, seq, int(causal), d, group, cu, units, cap,
                                   ctypes.byref(nb), ctypes.byref(ns))
    assert rc == 0
    return [units[i] for i in range(2 * nb.value)], nb.value, ns.value


def item_tiles(bh, seq, causal, d, pos):
    kbc = 64 if d == 64 else 32
    n_qtiles = -(-seq // ROWS)
    qtile = n_qtiles - 1 - pos // bh
    key_end = min(seq, qtile * ROWS + ROWS) if causal else seq
    return -(-key_end // kbc)


def unit_cost(bh, seq, causal, d, code):
    pos, part = code & 0xFFFFF, (code >> 20) & 3
    nt = item_tiles(bh, seq, causal, d, pos)
    mid = (nt // 2) & ~1
    if part == 0:
        return (nt + 1) // 2 + 3
    n = mid if part == 1 else nt - mid
    return (n + 1) // 2 + 4


def whole_items_makespan(bh, seq, causal, d, cu):
    costs = sorted((unit_cost(bh, seq, causal, d, pos) for pos in range(bh * -(-seq // ROWS))),
                   reverse=True)
    n = len(costs)
    singles = max(0, 2 * cu - n)
    span = max(costs[:singles], default=0)
    i, j = singles, n - 1
    while i < j:
        span = max(span, costs[i] + costs[j])
        i, j = i + 1, j - 1
    if i == j:
        span = max(span, costs[i])
    return span


SHAPES = [  # (B * H, S, causal, head_dim, group, expected split items or None)
    (48, 1024, False, 64, 1, 128),   # config 2 full
    (48, 1024, True, 64, 1, 0),      # config 2 causal: no split pays
    (14, 4096, True, 64, 1, 0),      # config 3: already balanced
    (14, 4096, True, 64, 7, 0),      # config 3 with grouped K/V
    (48, 1024, False, 128, 1, 128),
    (16, 2048, True, 64, 1, 64),
    (2, 1280, True, 64, 1, 8),
    (14, 1024, True, 64, 7, None),   # grouped K/V: splits as many as ungrouped
    (12, 128, True, 64, 1, 0),       # config 1: nothing to split
    (3, 333, True, 64, 1, 0),
    (6, 300, True, 128, 1, None),
]


@pytest.mark.parametrize("bh,seq,causal,d,group,expect", SHAPES)
def test_plan_covers_every_item_once(lib, bh, seq, causal, d, group, expect):
    units, n_blocks, n_splits = plan(lib, bh, seq, causal, d, group)
    n_items = bh * -(-seq // ROWS)
    if expect is not None:
        assert n_splits == expect
    if n_blocks == 0:
        assert n_splits == 0
        return
    assert n_blocks == 256
    whole, chunks = defaultdict(int), defaultdict(list)
    for b in range(n_blocks):
        first, second = units[2 * b], units[2 * b + 1]
        assert not (first == NO_UNIT and second != NO_UNIT), "second unit without a first"
        for u in (first, second):
            if u == NO_UNIT:
                continue
            pos, part, split = u & 0xFFFFF, (u >> 20) & 3, u >> 22
            assert 0 <= pos < n_items and part in (0, 1, 2)
            if part == 0:
                whole[pos] += 1
            else:
                assert 0 <= split < n_splits
                chunks[pos].append((part, split))
    for pos in range(n_items):
        if pos in chunks:
            assert pos not in whole, f"item {pos} both whole and split"
            parts = sorted(chunks[pos])
            assert [p for p, _ in parts] == [1, 2], f"item {pos}: chunks {parts}"
            assert parts[0][1] == parts[1][1], f"item {pos}: two partial slots"
            assert item_tiles(bh, seq, causal, d, pos) >= 8
        else:
            assert whole[pos] == 1, f"item {pos} runs {whole[pos]} times"
    slots = [chunks[p][0][1] for p in chunks]
    assert len(set(slots)) == len(slots) == n_splits


@pytest.mark.parametrize("bh,seq,causal,d,group,expect", SHAPES)
def test_plan_is_no_slower_and_keeps_heads_on_their_xcd(lib, bh, seq, causal, d, group, expect):
    cu = 256
    units, n_blocks, _ = plan(lib, bh, seq, causal, d, group, cu)
    if n_blocks == 0:
        return
    span = max(sum(unit_cost(bh, seq, causal, d, u) for u in units[2 * b:2 * b + 2]
                   if u != NO_UNIT) for b in range(n_blocks))
    assert span < whole_items_makespan(bh, seq, causal, d, cu)
    heavy = [units[2 * b] for b in range(n_blocks) if units[2 * b] != NO_UNIT]
    on_home = sum((units[2 * b] & 0xFFFFF) % 8 == b % 8 for b in range(n_blocks)
                  if units[2 * b] != NO_UNIT)
    assert on_home >= 0.9 * len(heavy)


def test_grouped_and_ungrouped_split_the_same_number_of_items(lib):
    for bh, seq, causal in [(14, 1024, True), (14, 2048, True), (48, 1024, False)]:
        assert plan(lib, bh, seq, causal, 64, 7)[2] == plan(lib, bh, seq, causal, 64, 1)[2]


def test_no_plan_without_a_cu_count_or_for_large_grids(lib):
    assert plan(lib, 48, 1024, False, 64, cu=0)[1] == 0
    assert plan(lib, 96, 4096, True, 64)[1] == 0  # 3072 items > 2 per CU
    assert plan(lib, 48, 1024, False, 64, cu=512)[1] == 0  # table holds <= 384 blocks


def test_bad_arguments_are_rejected(lib):
    nb, ns = ctypes.c_int(), ctypes.c_int()
    assert lib.fa_prefill_plan_units(0, 128, 1, 64, 1, 256, None, 0, ctypes.byref(nb),
                                     ctypes.byref(ns)) != 0
    assert lib.fa_prefill_plan_units(4, 128, 1, 96, 1, 256, None, 0, ctypes.byref(nb),
                                     ctypes.byref(ns)) != 0
