"""GPU parity of hs_spec_accept_commit_next: a speculative step's acceptance and
its bookkeeping (commit and rollback, the next step's pre-allocation, its draft
and verify staging) in one call.

At batch 1 with the single-launch acceptance the bookkeeping runs inside the
acceptance launch, in the workgroup that writes the outputs; otherwise the call
is the two launches. Each step runs the same inputs through hs_spec_accept +
hs_spec_commit_next on one device state and through the combined call on a
second one: outputs, state, eligibility and staging must be equal bit for bit.
The combined call's state is also checked against the CPU oracle of the
reference's bookkeeping (oracle/bookkeeping.py: llm_engine.py:111-181,
block_manager.py:84-92) after every step. Steps with zero acceptance uniforms
accept every draft (u < ratio with u = 0), so runs reach block boundaries, EOS
and max_tokens.
"""
import numpy as np
import pytest
import torch

from oracle.bookkeeping import BookState, Seq
from test_gpu_bookkeeping import assert_same_state, to_device

pytestmark = pytest.mark.gpu


def _stage(cuda, B, gamma):
    R = gamma + 1
    i64 = dict(dtype=torch.int64, device=cuda)
    i32 = dict(dtype=torch.int32, device=cuda)
    return (torch.full((B * R,), -7, **i64), torch.full((B * R,), -7, **i64),
            torch.full((B * R,), -7, **i32), torch.full((B + 1,), -7, **i32),
            torch.full((B + 1,), -7, **i32))


def _stage0(cuda, B):
    return _stage(cuda, B, 1)  # lookback: two rows per sequence


def _same(xs, ys, what):
    for i, (x, y) in enumerate(zip(xs, ys)):
        assert torch.equal(x, y), (what, i, x.cpu().tolist(), y.cpu().tolist())


@pytest.mark.parametrize("B,V,dtype,bs,seed", [
    (1, 151936, torch.bfloat16, 16, 0),
    (1, 151936, torch.bfloat16, 4, 1),
    (1, 32000, torch.float32, 256, 2),
    (1, 151936, torch.float32, 16, 3),
    (3, 151936, torch.bfloat16, 16, 4),
])
def test_accept_commit_next_matches_two_calls_and_oracle(hv, cuda, B, V, dtype, bs, seed):
    rng = np.random.default_rng(500 + seed)
    W, T = 96, 2048
    eos = int(rng.integers(1000, V))
    num_blocks = B * 12 + 6
    bm = BookState(num_blocks, bs, eos=eos)
    seqs = []
    for i in range(B):
        prompt = [int(x) for x in rng.integers(0, 900, size=int(rng.integers(1, 3 * bs)))]
        s = Seq(prompt, max_tokens=int(rng.integers(35, 70)), ignore_eos=bool(i == 2))
        bm.allocate(s)
        seqs.append(s)
    stA = to_device(hv, bm, seqs, W, T, cuda)
    stB = to_device(hv, bm, seqs, W, T, cuda)
    gammas = [int(g) for g in rng.choice([1, 2, 3, 5, 7], size=13)]
    elig_ref = bm.prealloc(seqs, gammas[0])
    eligA = hv.ops.spec_prealloc(stA, gammas[0])
    eligB = hv.ops.spec_prealloc(stB, gammas[0])
    assert eligB.cpu().tolist() == elig_ref
    print(f"B={B} V={V} {dtype} bs={bs} gammas={gammas} eos={eos}", flush=True)
    for step in range(len(gammas) - 1):
        g, gn = gammas[step], gammas[step + 1]
        R = g + 1
        logits = (torch.randn((B, R, V), device=cuda) * 3).to(dtype)
        q = torch.softmax(torch.randn((B, g, V), device=cuda) * 3, dim=-1)
        drafts = torch.from_numpy(rng.integers(0, 900, size=(B, g))).to(cuda)
        force = step % 3 != 1
        if step == 9:
            # the step ends the sequences at EOS: an accepted draft (even seeds), or
            # the bonus token drawn from a row peaked at EOS (odd seeds)
            force = True
            if seed % 2 == 0:
                drafts[:, int(rng.integers(0, g))] = eos
            else:
                logits[:, g, eos] = 60.0
        u_acc = (torch.zeros((B, g), device=cuda) if force
                 else torch.rand((B, g), device=cuda))
        u_res = torch.rand((B,), device=cuda)
        temps = torch.full((B,), 0.8, device=cuda)
        s0A, s0B = _stage0(cuda, B), _stage0(cuda, B)
        vA, vB = _stage(cuda, B, gn), _stage(cuda, B, gn)
        print(f"  step {step}: gamma {g} -> {gn}, forced {force}, lengths "
              f"{stB.context_lens.tolist()}", flush=True)
        a = hv.ops.spec_accept(logits, q, drafts, temps, u_acc, u_res)
        hv.ops.spec_commit_next(stA, g, a[1], a[2], eligA, gn, s0A, lookback=True,
                                stage_verify=vA)
        b = hv.ops.spec_accept(logits, q, drafts, temps, u_acc, u_res,
                               commit_next=dict(state=stB, eligible=eligB, next_gamma=gn,
                                                stage0=s0B, lookback=True, stage_verify=vB))
        torch.cuda.synchronize()
        _same(a, b, "outputs")
        assert int(b[0].min()) >= 0
        for f in stA.FIELDS:
            assert torch.equal(getattr(stA, f), getattr(stB, f)), (step, f)
        assert torch.equal(eligA, eligB)
        _same(s0A, s0B, "draft staging")
        _same(vA, vB, "verify staging")
        # the staging against the separate staging kernels on the committed state
        # (the verify rows' draft-token ids are the draft steps' to write)
        _same(hv.ops.draft_prepare(stB, None, 0, lookback=True), s0B, "draft staging vs kernel")
        vref = hv.ops.verify_prepare(stB, torch.zeros((B, gn), dtype=torch.int64, device=cuda),
                                     gn)
        Rn = gn + 1
        assert torch.equal(vref[0][0::Rn], vB[0][0::Rn])
        _same(vref[1:], vB[1:], "verify staging vs kernel")
        # the oracle: commit the eligible sequences' emitted tokens, then pre-allocate
        out, olen = b[1].cpu().numpy(), b[2].cpu().numpy()
        batch = [s for s, e in zip(seqs, elig_ref) if e]
        acc = [out[i, :olen[i]].tolist() for i, e in enumerate(elig_ref) if e]
        bm.commit(batch, acc, g)
        elig_ref = bm.prealloc(seqs, gn)
        assert eligB.cpu().tolist() == elig_ref, step
        assert_same_state(stB, bm, seqs)
        if all(s.finished for s in seqs):
            break


def test_accept_commit_next_failed_wait_leaves_state(hv, cuda):
    """A zero wait budget makes the batch-1 launch's waits give up: the sequence gets
    num_accepted -1 and out_len 0, the bookkeeping does not run (state, eligibility
    and staging keep their values), every kernel exits, and the next call with the
    default budget is correct again."""
    rng = np.random.default_rng(9)
    V, g, bs = 151936, 3, 16
    bm = BookState(20, bs, eos=V - 1)
    s = Seq([int(x) for x in rng.integers(0, 900, size=21)], max_tokens=50)
    bm.allocate(s)
    st = to_device(hv, bm, [s], 32, 512, cuda)
    ref = to_device(hv, bm, [s], 32, 512, cuda)
    elig = hv.ops.spec_prealloc(st, g)
    hv.ops.spec_prealloc(ref, g)
    logits = (torch.randn((1, g + 1, V), device=cuda) * 3).to(torch.bfloat16)
    q = torch.softmax(torch.randn((1, g, V), device=cuda) * 3, dim=-1)
    drafts = torch.from_numpy(rng.integers(0, 900, size=(1, g))).to(cuda)
    temps = torch.full((1,), 0.8, device=cuda)
    u_acc, u_res = torch.rand((1, g), device=cuda), torch.rand((1,), device=cuda)
    s0, v = _stage0(cuda, 1), _stage(cuda, 1, g)
    s0c, vc = [t.clone() for t in s0], [t.clone() for t in v]
    elig0 = elig.clone()
    cn = dict(state=st, eligible=elig, next_gamma=g, stage0=s0, lookback=True, stage_verify=v)
    hv.ops.accept_error(cuda, clear=True)
    hv.ops.accept_wait_budget(cuda, 0)
    try:
        nacc, out, olen = hv.ops.spec_accept(logits, q, drafts, temps, u_acc, u_res,
                                             commit_next=cn)
        torch.cuda.synchronize()
    finally:
        hv.ops.accept_wait_budget(cuda, None)
    assert int(nacc[0]) == -1 and int(olen[0]) == 0
    assert hv.ops.accept_error(cuda, clear=True)
    for f in st.FIELDS:
        assert torch.equal(getattr(st, f), getattr(ref, f)), f
    assert torch.equal(elig, elig0)
    _same(s0, s0c, "draft staging")
    _same(v, vc, "verify staging")
    # the default budget again: the combined call equals the two calls
    b = hv.ops.spec_accept(logits, q, drafts, temps, u_acc, u_res, commit_next=cn)
    eref = elig0.clone()
    s0r, vr = _stage0(cuda, 1), _stage(cuda, 1, g)
    a = hv.ops.spec_accept(logits, q, drafts, temps, u_acc, u_res)
    hv.ops.spec_commit_next(ref, g, a[1], a[2], eref, g, s0r, lookback=True, stage_verify=vr)
    torch.cuda.synchronize()
    _same(a, b, "outputs")
    assert int(b[0][0]) >= 0
    for f in st.FIELDS:
        assert torch.equal(getattr(st, f), getattr(ref, f)), f
    assert torch.equal(elig, eref)
    _same(s0, s0r, "draft staging")
    _same(v, vr, "verify staging")
    assert not hv.ops.accept_error(cuda)
