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
    return importlib.import_module("tests.seq_fixture")


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


def _invalid_accept(monkeypatch, ops):
    """spec_accept as the single-launch kernel leaves it after a bounded wait ran
    out for sequence 1: num_accepted -1, out_len 0, tokens -1."""
    import torch

    def fake(lg, q, dt, T, ua, ur, **kw):
        B, g = dt.shape
        nacc = torch.tensor([g if b != 1 else -1 for b in range(B)], dtype=torch.int32)
        out = torch.cat([dt, torch.zeros((B, 1), dtype=torch.int64)], 1)
        out[1] = -1
        olen = (nacc + 1).clamp(min=0).to(torch.int32)
        return nacc, out, olen

    monkeypatch.setattr(ops, "spec_accept", fake)


def test_run_verify_raises_on_invalid_acceptance(monkeypatch):
    """VerifyRunner._accept reads the results back once; a -1 count must raise,
    not become an empty commit ([], -1)."""
    import torch
    vr, sq = _vr(), _sq()
    ops = importlib.import_module("hilda-vllm_amd.ops")
    _invalid_accept(monkeypatch, ops)
    runner = vr.VerifyRunner(None, device="cpu", record_breakdown=False)
    V, g = 64, 3
    seqs = [sq.Sequence([1, 2, 3]) for _ in range(3)]
    drafts = [[4, 5, 6]] * 3
    logits = torch.zeros((3 * (g + 1), V))
    probs = torch.full((3, g, V), 1.0 / V)
    with pytest.raises(RuntimeError, match="sequences \\[1\\]"):
        runner._accept(seqs, drafts, probs, logits, [g + 1] * 3, None)
    # the same call with valid outputs returns every sequence's tokens
    monkeypatch.setattr(ops, "spec_accept", lambda lg, q, dt, *a, **k: (
        torch.full((3,), g, dtype=torch.int32),
        torch.cat([dt, torch.full((3, 1), 9, dtype=torch.int64)], 1),
        torch.full((3,), g + 1, dtype=torch.int32)))
    res = runner._accept(seqs, drafts, probs, logits, [g + 1] * 3, None)
    assert res == [([4, 5, 6, 9], 3)] * 3


def test_spec_runner_raises_on_invalid_acceptance():
    """SpecRunner._after_step copies the step's totals to the host for the gamma
    controller; a -1 count of a sequence that took part must raise there, and a
    sequence that sat out (eligible 0) must not."""
    import types
    import torch
    srm = importlib.import_module("hilda-vllm_amd.engine.spec_runner")
    agm = importlib.import_module("hilda-vllm_amd.engine.adaptive_gamma")
    r = object.__new__(srm.SpecRunner)
    r.gamma = 3
    r.controller = agm.AdaptiveGamma(3, max_gamma=7)
    r.history = []
    G = types.SimpleNamespace(gamma=3, elig=torch.tensor([1, 1, 0], dtype=torch.int32),
                              last=(torch.tensor([2, -1, 0], dtype=torch.int32), None, None))
    r._per_gamma = {3: G}
    with pytest.raises(RuntimeError, match="invalid"):
        r._after_step()
    assert r.history == []
    G.last = (torch.tensor([2, 1, -1], dtype=torch.int32), None, None)
    r._after_step()
    assert r.history == [(3, 3, 6)]


def test_accept_error_flag_is_read_and_cleared(monkeypatch):
    """The sticky word at byte 8 of the acceptance workspace (set by the kernel
    when a wait ran out) is what SpecRunner.check reads for fixed-gamma runs.
    ops.workspace keys it by the ordinal of the tensors' device (0), and a device
    given without an index ("cuda", SpecRunner's default) must find that key."""
    import torch
    ops = importlib.import_module("hilda-vllm_amd.ops")
    ws = torch.zeros(256, dtype=torch.uint8)
    monkeypatch.setitem(ops._WS, (0, "spec_accept"), ws)
    assert not ops.accept_error("cuda")
    ws[8] = 1
    assert ops.accept_error("cuda")
    assert ops.accept_error(torch.device("cuda"))
    assert ops.accept_error("cuda:0", clear=True)
    assert not ops.accept_error("cuda")
    ws[8] = 1
    assert not ops.accept_error("cuda:1")  # another device's workspace is not this one


def test_workspace_key_resolves_the_device_index():
    ops = importlib.import_module("hilda-vllm_amd.ops")
    assert ops._dev_index("cuda:3") == 3
    assert ops._dev_index(2) == 2
    # no index: the current device (0 where no GPU is visible, as here on the CPU)
    expect = torch_current_device_or_zero()
    assert ops._dev_index("cuda") == expect


def torch_current_device_or_zero():
    import torch
    try:
        return torch.cuda.current_device()
    except (RuntimeError, AssertionError):
        return 0
