"""GPU tests of the run_verify / cleanup_rejected_kv_slots drop-in
(hilda-vllm_amd/engine/verify.py, mirroring model_runner.py:321-481).

* The accept decisions and emitted tokens equal the CPU oracle's on the
  logits the verify forward produced (same explicit uniforms), bit-exact.
* The verify logits equal those of a plain prefill over prompt + drafts in a
  fresh cache (pins the staging: positions, slots, cu_seqlens, block tables).
* Mixed draft counts (including a sequence without drafts) and greedy
  batches give the oracle's results.
* cleanup zeroes exactly the token rows of the reference's dirty range.
"""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BS = 32


def _mods():
    q3 = importlib.import_module("hilda-vllm_amd.engine.qwen3_host")
    vr = importlib.import_module("hilda-vllm_amd.engine.verify")
    sq = importlib.import_module("tests.seq_fixture")
    ctx = importlib.import_module("hilda-vllm_amd.utils.context")
    return q3, vr, sq, ctx


def _model(q3, cuda, seed=41):
    g = q3.Qwen3Geometry(num_layers=2, hidden=512, num_heads=4, num_kv_heads=2, ffn=1024,
                         vocab=3000, max_position=4096)
    return q3.Qwen3Host(g, device=cuda, seed=seed), g


def _bind(model, g, cuda, nb=64):
    kv = torch.zeros((2, g.num_layers, nb, BS, g.num_kv_heads, g.head_dim), dtype=torch.bfloat16,
                     device=cuda)
    for i, a in enumerate(model.attention_layers()):
        a.k_cache, a.v_cache = kv[0, i], kv[1, i]
    return kv


def _prefill(model, ctx, seqs, cuda):
    ids, pos, slots, cu = [], [], [], [0]
    for s in seqs:
        n = len(s)
        ids += s.token_ids
        pos += list(range(n))
        slots += [s.block_table[p // BS] * BS + p % BS for p in range(n)]
        cu.append(cu[-1] + n)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    W = max(len(s.block_table) for s in seqs)
    bt = torch.full((len(seqs), W), -1, dtype=torch.int32)
    for i, s in enumerate(seqs):
        bt[i, :len(s.block_table)] = torch.tensor(s.block_table)
    ctx.set_context(True, cu_t, cu_t, max(len(s) for s in seqs), max(len(s) for s in seqs),
                    torch.tensor(slots, dtype=torch.int32, device=cuda), None, bt.to(cuda))
    with torch.inference_mode():
        h = model(torch.tensor(ids, device=cuda), torch.tensor(pos, device=cuda))
    ctx.reset_context()
    return h


def _make_seqs(sq, prompts, gamma, temperature=0.8, first_block=0):
    seqs, nxt = [], first_block
    for p in prompts:
        s = sq.Sequence(p, sq.SamplingParams(temperature=temperature))
        s.block_size = BS
        need = (len(p) + gamma + 1 + BS - 1) // BS  # pre-allocation (llm_engine.py:111-128)
        s.block_table = list(range(nxt, nxt + need))
        nxt += need
        seqs.append(s)
    return seqs


def _draft_inputs(rng, B, gammas, V, cuda):
    drafts = [list(map(int, rng.integers(0, V, size=g))) for g in gammas]
    probs = []
    for g in gammas:
        rows = []
        for _ in range(g):
            x = torch.from_numpy(rng.normal(0, 2, size=V).astype(np.float32))
            rows.append(torch.softmax(x, 0).to(cuda))
        probs.append(rows)
    return drafts, probs


def _oracle_accept(orc, logits_rows, probs_rows, drafts, temps, ua, ur, mode):
    lg = logits_rows.float().cpu().numpy()[None]
    q = np.stack([p.cpu().numpy() for p in probs_rows])[None] if probs_rows else None
    return orc.spec_accept(lg, q, np.array([drafts], np.int64), np.array([temps], np.float32),
                           ua[None], ur[None], mode=mode)


def test_run_verify_matches_oracle_and_prefill(orc, cuda):
    q3, vr, sq, ctx = _mods()
    model, g = _model(q3, cuda)
    kv = _bind(model, g, cuda)
    rng = np.random.default_rng(3)
    gamma = 3
    prompts = [list(map(int, rng.integers(0, g.vocab, size=n))) for n in (5, 40, 70)]
    seqs = _make_seqs(sq, prompts, gamma)
    _prefill(model, ctx, seqs, cuda)
    drafts, probs = _draft_inputs(rng, 3, [gamma] * 3, g.vocab, cuda)
    ua = rng.random((3, gamma)).astype(np.float32)
    ur = rng.random(3).astype(np.float32)
    runner = vr.VerifyRunner(model, block_size=BS, max_num_seqs=8, kv_caches=[kv], device=cuda)
    print("run_verify B=3 gamma=3", flush=True)
    res = runner.run_verify(seqs, drafts, probs, uniforms=(ua, ur))
    assert set(runner.last_verify_breakdown) == {"prep_time_s", "forward_time_s",
                                                 "lmhead_time_s", "sampling_time_s"}
    logits = runner.last_logits
    for i in range(3):
        ref = _oracle_accept(orc, logits[4 * i:4 * i + 4], probs[i], drafts[i], 0.8, ua[i], ur[i],
                             "reference")
        n = int(ref["num_accepted"][0])
        assert res[i][1] == n
        assert res[i][0] == ref["out_tokens"][0, :n + 1].tolist()
        assert res[i][0][:n] == drafts[i][:n]
    # verify logits == a plain prefill of prompt + drafts in a fresh cache
    model2, _ = _model(q3, cuda)
    _bind(model2, g, cuda)
    full = _make_seqs(sq, [p + d for p, d in zip(prompts, drafts)], 0)
    h = _prefill(model2, ctx, full, cuda)
    with torch.inference_mode():
        lg_full = model2.compute_logits(h)
    off = 0
    for i, s in enumerate(full):
        want = lg_full[off + len(s) - 4: off + len(s)].float()
        got = logits[4 * i:4 * i + 4].float()
        off += len(s)
        err = (got - want).abs().max().item()
        assert err <= 0.03 * want.abs().max().item() + 0.02, (i, err)
        assert torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), 0) > 0.999


def test_run_verify_mixed_draft_counts(orc, cuda):
    q3, vr, sq, ctx = _mods()
    model, g = _model(q3, cuda, seed=42)
    kv = _bind(model, g, cuda)
    rng = np.random.default_rng(4)
    gammas = [3, 0, 2, 3]
    prompts = [list(map(int, rng.integers(0, g.vocab, size=n))) for n in (33, 8, 64, 12)]
    seqs = _make_seqs(sq, prompts, 3)
    _prefill(model, ctx, seqs, cuda)
    drafts, probs = _draft_inputs(rng, 4, gammas, g.vocab, cuda)
    ua = rng.random((4, 3)).astype(np.float32)
    ur = rng.random(4).astype(np.float32)
    runner = vr.VerifyRunner(model, block_size=BS, max_num_seqs=8, kv_caches=[kv], device=cuda,
                             record_breakdown=False)
    print("run_verify mixed gammas", gammas, flush=True)
    res = runner.run_verify(seqs, drafts, probs, uniforms=(ua, ur))
    logits = runner.last_logits
    off = 0
    for i, gm in enumerate(gammas):
        rows = logits[off:off + gm + 1]
        off += gm + 1
        if gm == 0:
            r = orc.sampler(rows.float().cpu().numpy(), np.array([0.8], np.float32),
                            mode="reference", uniforms=ur[i:i + 1])
            assert res[i] == ([int(r["tokens"][0])], 0)
            continue
        ref = _oracle_accept(orc, rows, probs[i], drafts[i], 0.8, ua[i, :gm], ur[i], "reference")
        n = int(ref["num_accepted"][0])
        assert res[i] == (ref["out_tokens"][0, :n + 1].tolist(), n)


def test_run_verify_greedy(orc, cuda):
    q3, vr, sq, ctx = _mods()
    model, g = _model(q3, cuda, seed=43)
    _bind(model, g, cuda)
    rng = np.random.default_rng(5)
    prompts = [list(map(int, rng.integers(0, g.vocab, size=n))) for n in (20, 50)]
    seqs = _make_seqs(sq, prompts, 3, temperature=0.0)
    _prefill(model, ctx, seqs, cuda)
    runner = vr.VerifyRunner(model, block_size=BS, max_num_seqs=4, device=cuda)
    drafts = [list(map(int, rng.integers(0, g.vocab, size=3))) for _ in range(2)]
    print("run_verify greedy", flush=True)
    # Re-verifying seq 0 with the target's own argmax choices fixes one more draft per
    # call (row j depends on drafts[:j]); after 3 updates all of them are accepted.
    for it in range(4):
        res = runner.run_verify(seqs, drafts, None)
        logits = runner.last_logits.float()
        for i in range(2):
            am = logits[4 * i:4 * i + 4].argmax(-1).tolist()
            n = 0
            while n < 3 and drafts[i][n] == am[n]:
                n += 1
            assert res[i] == (drafts[i][:n] + [am[n]], n), (it, i)
        if it < 3:
            drafts[0] = logits[0:3].argmax(-1).tolist()
    assert res[0][1] == 3


def test_cleanup_rejected_kv_slots(cuda):
    q3, vr, sq, ctx = _mods()
    model, g = _model(q3, cuda, seed=44)
    kv = _bind(model, g, cuda)
    kv.normal_()
    dkv = torch.randn((2, 1, 64, BS, g.num_kv_heads, g.head_dim), device=cuda).to(torch.bfloat16)
    before, dbefore = kv.clone(), dkv.clone()
    seqs = _make_seqs(sq, [[1] * 30, [2] * 62], 3)
    results = [([7, 8], 1), ([9], 0)]  # tokens appended by the commit
    for s, (acc, _) in zip(seqs, results):
        for t in acc:
            s.append_token(t)
    runner = vr.VerifyRunner(model, block_size=BS, max_num_seqs=4, kv_caches=[kv, dkv],
                             device=cuda)
    dirty = runner.cleanup_rejected_kv_slots(seqs, results, 3)
    # seq 0: old 30, kept 2 -> positions [32, 34); seq 1: old 62, kept 1 -> [63, 66)
    bt0, bt1 = seqs[0].block_table, seqs[1].block_table
    want = [bt0[1] * BS + 0, bt0[1] * BS + 1] + [bt1[1] * BS + 31] + \
        [bt1[2] * BS + 0, bt1[2] * BS + 1]
    assert dirty == want
    torch.cuda.synchronize()
    for c, ref in ((kv, before), (dkv, dbefore)):
        flat = ref.view(2, ref.shape[1], -1, g.num_kv_heads, g.head_dim)
        flat[:, :, want] = 0
        assert torch.equal(c, ref)
