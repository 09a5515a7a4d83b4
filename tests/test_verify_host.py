"""Host logic of the run_verify drop-in (runs without a GPU).

The staging of VerifyRunner (positions, slot mapping with -1 beyond the block
table, cu_seqlens) must equal the oracle's restatement of model_runner.py:
339-362, and the cleanup range must equal the oracle's dirty_mode 0 range
(model_runner.py:445-464).
"""
import importlib

import numpy as np
import pytest

from oracle.bookkeeping import BookState, Seq


def _vr():
    return importlib.import_module("hilda-vllm_amd.engine.verify")


def _sq():
    return importlib.import_module("hilda-vllm_amd.engine.sequence")


@pytest.mark.parametrize("seed", range(3))
def test_staging_matches_oracle(seed):
    vr, sq = _vr(), _sq()
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([4, 16, 256]))
    B = int(rng.integers(1, 12))
    bm = BookState(num_blocks=B * 40, block_size=bs)
    ours, theirs, drafts = [], [], []
    for _ in range(B):
        toks = list(map(int, rng.integers(0, 100, size=rng.integers(1, 5 * bs))))
        o = Seq(toks)
        bm.allocate(o)
        g = int(rng.integers(0, 6))
        if rng.random() < 0.7:  # most sequences are pre-allocated for the drafts
            bm.prealloc([o], g)
        s = sq.Sequence(toks)
        s.block_table = list(o.block_table)
        ours.append(s)
        theirs.append(o)
        drafts.append(list(map(int, rng.integers(0, 100, size=g))))
    runner = vr.VerifyRunner(None, block_size=bs, max_num_seqs=16, device="cpu")
    total, max_q, max_k, lens, bt = runner._stage(ours, drafts)
    ids, pos, slots, cq, ck = bm.prepare(theirs, drafts)
    assert total == len(ids)
    assert runner.gpu["input_ids"][:total].tolist() == ids
    assert runner.gpu["positions"][:total].tolist() == pos
    assert runner.gpu["slot_mapping"][:total].tolist() == slots
    assert runner.gpu["cu_seqlens_q"][:B + 1].tolist() == cq
    assert runner.gpu["cu_seqlens_k"][:B + 1].tolist() == ck
    assert max_q == max(len(d) + 1 for d in drafts)
    assert lens == [len(d) + 1 for d in drafts]
    for i, s in enumerate(ours):
        row = bt[i].tolist()
        assert row[:len(s.block_table)] == s.block_table
        assert all(v == -1 for v in row[len(s.block_table):])


def test_cleanup_range_matches_oracle():
    vr, sq = _vr(), _sq()
    bs = 4
    bm = BookState(num_blocks=16, block_size=bs)
    o = Seq([1, 2, 3, 4, 5])
    bm.allocate(o)
    bm.prealloc([o], 3)
    s = sq.Sequence([1, 2, 3, 4, 5])
    s.block_table = list(o.block_table)
    for t in (7, 8):
        s.append_token(t)
        o.token_ids.append(t)
    runner = vr.VerifyRunner(None, block_size=bs, device="cpu")  # no caches bound
    dirty = runner.cleanup_rejected_kv_slots([s], [([7, 8], 1)], 3)
    assert dirty == bm.dirty_slots(o, 2, 3, dirty_mode=0)


def test_sampling_params_validation():
    sq = _sq()
    with pytest.raises(ValueError):
        sq.SamplingParams(temperature=-1.0)
    with pytest.raises(ValueError):
        sq.SamplingParams(top_k=0)
    with pytest.raises(ValueError):
        sq.SamplingParams(top_p=0.0)
    assert sq.SamplingParams(temperature=0.0).temperature == 0.0
