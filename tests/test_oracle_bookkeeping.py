"""Pins the CPU oracle of the spec-step bookkeeping (runs without a GPU).

Checks: the reference's BlockManager known-answer tests
(tests/test_block_manager.py:20-46), hand-worked FIFO scenarios of the
spec block (llm_engine.py:111-181), and conservation invariants over random
multi-step runs.
"""
import numpy as np
import pytest

from oracle.bookkeeping import BookState, Seq


def test_kat_allocate_reuses_cached_full_prefix_block():
    # tests/test_block_manager.py:20-31 (block_size 2)
    bm = BookState(num_blocks=4, block_size=2)
    s1, s2 = Seq([1, 2, 3]), Seq([1, 2, 9])
    bm.allocate(s1)
    bm.allocate(s2)
    shared = s1.block_table[0]
    assert s2.block_table[0] == shared
    assert s2.num_cached_tokens == 2
    assert bm.blocks[shared].ref_count == 2


def test_kat_deallocate_returns_blocks_to_free_pool():
    # tests/test_block_manager.py:34-46
    bm = BookState(num_blocks=3, block_size=2)
    s = Seq([1, 2, 3])
    bm.allocate(s)
    assert len(bm.free) == 1
    bm.deallocate(s)
    assert len(bm.free) == 3
    assert bm.used == set()
    assert s.block_table == [] and s.num_cached_tokens == 0


def test_prealloc_pops_front_and_skips_when_short():
    bm = BookState(num_blocks=6, block_size=4)
    a, b = Seq([1, 2, 3]), Seq([4, 5, 6, 7, 8])
    bm.allocate(a)  # block 0
    bm.allocate(b)  # blocks 1, 2
    assert list(bm.free) == [3, 4, 5]
    # gamma 3: a needs ceil((3+4)/4)=2 blocks (has 1) -> takes 3; b needs ceil(9/4)=3 (has 2) -> 4
    assert bm.prealloc([a, b], 3) == [1, 1]
    assert a.block_table == [0, 3] and b.block_table == [1, 2, 4]
    assert list(bm.free) == [5]
    # a second pre-allocation with gamma 6 needs 2 more blocks for a: skipped
    c = Seq([9])
    bm.allocate(c)  # takes 5
    assert bm.prealloc([a], 6) == [0]


def test_commit_trims_tail_blocks_in_reference_order():
    bm = BookState(num_blocks=8, block_size=2, eos=99)
    a, b = Seq([1, 2, 3]), Seq([4, 5, 6])
    bm.allocate(a)  # 0, 1
    bm.allocate(b)  # 2, 3
    bm.prealloc([a, b], 3)  # a: ceil(7/2)=4 -> 4,5 ; b: 6,7
    assert a.block_table == [0, 1, 4, 5] and b.block_table == [2, 3, 6, 7]
    # a accepts 1 draft + bonus (len 5 -> 3 blocks), b finishes on EOS
    app, _ = bm.commit([a, b], [[10, 11], [12, 99, 13]], 3)
    assert app == [2, 2]
    assert b.finished and b.block_table == []
    # finish releases b's table last-first, then trims pop a's tail
    assert list(bm.free) == [7, 6, 3, 2, 5]
    assert a.block_table == [0, 1, 4]


def test_dirty_ranges():
    bm = BookState(num_blocks=8, block_size=4)
    a = Seq([1, 2, 3, 4, 5])
    bm.allocate(a)
    bm.prealloc([a], 3)  # len 5 + 4 -> 3 blocks
    t = list(a.block_table)  # dirty slots refer to the table before the trim
    _, dirty0 = bm.commit([a], [[7, 8]], 3, dirty_mode=0)
    # old_len 5, new len 7: reference range [7, 9) (positions 7, 8)
    assert dirty0 == [[t[1] * 4 + 3, t[2] * 4 + 0]]
    b = Seq([1, 2, 3, 4, 5])
    bm2 = BookState(num_blocks=8, block_size=4)
    bm2.allocate(b)
    bm2.prealloc([b], 3)
    t = list(b.block_table)
    _, dirty1 = bm2.commit([b], [[7, 8]], 3, dirty_mode=1)
    # exact range [6, 8): position 6 (stale draft KV under the bonus) and 7
    assert dirty1 == [[t[1] * 4 + 2, t[1] * 4 + 3]]


@pytest.mark.parametrize("seed", range(4))
def test_random_runs_conserve_blocks(seed):
    rng = np.random.default_rng(seed)
    bm = BookState(num_blocks=40, block_size=4, eos=7)
    seqs = [Seq(list(rng.integers(0, 9, size=rng.integers(1, 12))), max_tokens=20)
            for _ in range(6)]
    for s in seqs:
        bm.allocate(s)
    for _ in range(10):
        gamma = int(rng.integers(1, 5))
        elig = bm.prealloc(seqs, gamma)
        batch = [s for s, e in zip(seqs, elig) if e]
        acc = [list(rng.integers(0, 9, size=rng.integers(1, gamma + 2))) for _ in batch]
        bm.commit(batch, acc, gamma)
        used = {b for s in seqs for b in s.block_table}
        assert len(bm.free) + len(used) == 40
        assert len(set(bm.free)) == len(bm.free)
        assert not (set(bm.free) & used)
        for s in seqs:
            if not s.finished:
                assert len(s.block_table) == (len(s) + 3) // 4
