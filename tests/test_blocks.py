"""The native page allocator (luc_blocks_*, lucciola-rs_amd/csrc/luc_blocks.cpp)
through the C ABI, on the CPU: the reference's single-sequence behaviour
(KVCache free list and prepare_for_step, src/layers/kv_cache.rs:73-76,
106-122), then a model-based check of many sequences against a plain Python
statement of the allocation rules."""
import numpy as np
import pytest

from lucciola_rs_amd.engine import BlockManager
from lucciola_rs_amd.library import LucError

PAGE = 16


def test_single_sequence_matches_prepare_for_step():
    """Token by token, one sequence: the same pages as the reference's loop
    (pop from a free list filled in reverse when pos enters a new page)."""
    n = 40
    bm = BlockManager(n, 1, 64)
    free = list(range(n - 1, -1, -1))
    table = []
    for pos in range(300):
        if pos // PAGE >= len(table):
            table.append(free.pop())
        bm.reserve(0, pos + 1)
        row = bm.table()[0]
        assert list(row[: len(table)]) == table and not row[len(table):].any()
    assert bm.num_free == len(free) and bm.num_pages(0) == len(table)
    assert table == list(range(len(table)))  # a fresh pool hands out 0, 1, 2, ...


def test_multi_page_growth_and_no_shrink():
    bm = BlockManager(100, 2, 20)
    bm.reserve(0, 1)
    assert bm.num_pages(0) == 1
    bm.reserve(0, 5 * PAGE + 1)  # one call, five more pages
    assert bm.num_pages(0) == 6
    bm.reserve(0, 3)  # never shrinks
    assert bm.num_pages(0) == 6
    bm.reserve(1, 0)
    assert bm.num_pages(1) == 0


def test_out_of_pages_changes_nothing():
    bm = BlockManager(10, 3, 10)
    bm.reserve(0, 4 * PAGE)
    before = (bm.table().copy(), bm.num_free)
    with pytest.raises(LucError, match="LUC_E_NOMEM.*out of pages"):
        bm.reserve(1, 7 * PAGE)
    with pytest.raises(LucError, match="LUC_E_NOMEM"):
        bm.reserve_batch([1, 2], [3 * PAGE, 3 * PAGE + 1])  # 7 pages, 6 free: neither is given any
    assert np.array_equal(bm.table(), before[0]) and bm.num_free == before[1]
    bm.reserve_batch([1, 2], [3 * PAGE, 3 * PAGE])  # exactly the 6 free pages
    assert bm.num_free == 0


def test_invalid_arguments():
    bm = BlockManager(10, 2, 4)
    with pytest.raises(LucError, match="LUC_E_INVALID.*outside"):
        bm.reserve(2, 1)
    with pytest.raises(LucError, match="LUC_E_INVALID.*row holds 4"):
        bm.reserve(0, 4 * PAGE + 1)
    with pytest.raises(LucError, match="LUC_E_INVALID.*twice"):
        bm.reserve_batch([1, 1], [1, 1])
    with pytest.raises(LucError, match="LUC_E_INVALID.*negative"):
        bm.reserve(0, -1)
    with pytest.raises(LucError, match="LUC_E_INVALID"):
        bm.release(-1)
    with pytest.raises(LucError, match="LUC_E_INVALID"):
        BlockManager(0, 1, 1)
    assert bm.num_free == 10


def test_release_then_reserve_gives_the_same_pages():
    bm = BlockManager(64, 4, 16)
    bm.reserve(0, 50)
    bm.reserve(1, 100)
    row = bm.table()[1].copy()
    bm.release(1)
    bm.reserve(1, 100)
    assert np.array_equal(bm.table()[1], row)
    bm.release(3)  # releasing an empty sequence is a no-op
    assert bm.num_free == 64 - 4 - 7


class Model:
    """The allocation rules in plain Python."""

    def __init__(self, n, seqs, max_pages):
        self.free = list(range(n - 1, -1, -1))
        self.rows = [[] for _ in range(seqs)]
        self.max_pages = max_pages

    def reserve_batch(self, seqs, toks):
        extra = [max(0, -(-t // PAGE) - len(self.rows[s])) for s, t in zip(seqs, toks)]
        if any(-(-t // PAGE) > self.max_pages for t in toks):
            return "invalid"
        if sum(extra) > len(self.free):
            return "nomem"
        for s, e in zip(seqs, extra):
            for _ in range(e):
                self.rows[s].append(self.free.pop())
        return "ok"

    def release(self, s):
        self.free.extend(reversed(self.rows[s]))
        self.rows[s] = []


@pytest.mark.parametrize("seed", range(4))
def test_random_operations_against_the_rules(seed):
    rng = np.random.default_rng(seed)
    n, seqs, max_pages = 200, 12, 24
    bm, m = BlockManager(n, seqs, max_pages), Model(n, seqs, max_pages)
    for _ in range(600):
        op = rng.random()
        if op < 0.25:
            s = int(rng.integers(seqs))
            bm.release(s)
            m.release(s)
        else:
            k = int(rng.integers(1, 5))
            ss = rng.choice(seqs, size=k, replace=False).astype(np.int32)
            tt = rng.integers(0, max_pages * PAGE + 40, size=k).astype(np.int32)
            want = m.reserve_batch(list(ss), list(tt))
            try:
                bm.reserve_batch(ss, tt)
                got = "ok"
            except LucError as e:
                got = {-6: "nomem", -1: "invalid"}[e.code]
            assert got == want
        table = bm.table()
        for s in range(seqs):
            r = m.rows[s]
            assert list(table[s, : len(r)]) == r and not table[s, len(r):].any()
        assert bm.num_free == len(m.free)
        held = [p for r in m.rows for p in r]
        assert len(set(held)) == len(held) and len(held) + len(m.free) == n  # no page twice
