"""End-to-end speculative decoding on the GPU with small Qwen3-shaped models.

Properties checked (model weights are random, so these are invariants rather
than reference outputs):
  * greedy acceptance with draft == target accepts (almost) every draft;
  * every step emits between 1 and gamma+1 tokens and the device bookkeeping
    stays consistent (block count, free list conservation);
  * replaying the captured HIP graphs gives the same tokens as eager steps.
"""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _mods():
    q3 = importlib.import_module("hilda-vllm_amd.engine.qwen3_host")
    sr = importlib.import_module("hilda-vllm_amd.engine.spec_runner")
    return q3, sr


def _hv():
    return importlib.import_module("hilda-vllm_amd")


def _small(q3, layers=2, hidden=512, heads=4, kv=2, vocab=3000):
    return q3.Qwen3Geometry(num_layers=layers, hidden=hidden, num_heads=heads, num_kv_heads=kv,
                            ffn=1024, vocab=vocab, max_position=4096)


def _check_state(runner):
    """Block accounting between steps: every sequence holds ceil(len / block) blocks,
    or, when the last commit already pre-allocated the next step (chained steps),
    ceil((len + gamma + 1) / block)."""
    st = runner.state
    nb = st.num_seq_blocks.cpu()
    lens = st.context_lens.cpu()
    extra = runner.gamma + 1 if runner._staged else 0
    for b in range(runner.B):
        need = (int(lens[b]) + extra + runner.bs - 1) // runner.bs
        assert int(nb[b]) == need
    used = int(nb.sum())
    assert int(st.free_hdr[1]) + used == runner.num_blocks


def test_greedy_self_draft_accepts_all(cuda):
    q3, sr = _mods()
    g = _small(q3)
    target = q3.Qwen3Host(g, device=cuda, seed=11)
    draft = q3.Qwen3Host(g, share_from=target)
    runner = sr.SpecRunner(target, draft, batch=2, gamma=3, max_model_len=512, block_size=32,
                           temperature=0.0, mode="greedy", device=cuda)
    runner.load_prompts([[5, 6, 7, 8, 9], list(range(40, 77))])
    runner.prefill()
    l0 = runner.lengths()
    steps = 12
    for _ in range(steps):
        runner.step()
    torch.cuda.synchronize()
    l1 = runner.lengths()
    emitted = sum(a - b for a, b in zip(l1, l0))
    assert emitted >= 0.9 * steps * 2 * 4, (l0, l1)
    _check_state(runner)


@pytest.mark.parametrize("kv", ["auto", "fp8"])
def test_natural_sampling_steps(cuda, kv):
    q3, sr = _mods()
    gt = _small(q3, layers=3)
    gd = _small(q3, layers=1)
    target = q3.Qwen3Host(gt, device=cuda, seed=12)
    draft = q3.Qwen3Host(gd, device=cuda, seed=13)
    B, gamma = 3, 4
    runner = sr.SpecRunner(target, draft, batch=B, gamma=gamma, max_model_len=600, block_size=32,
                           temperature=0.8, mode="reference", kv_cache_dtype=kv, device=cuda)
    runner.load_prompts([[1] * 3, list(range(100, 170)), [7, 8]])
    runner.prefill()
    prev = runner.lengths()
    for _ in range(15):
        runner.step()
        cur = runner.lengths()
        for a, b in zip(cur, prev):
            assert 1 <= a - b <= gamma + 1
        prev = cur
    _check_state(runner)


def test_graph_replay_matches_eager(cuda):
    q3, sr = _mods()
    gt = _small(q3, layers=2)
    gd = _small(q3, layers=1)

    def make():
        target = q3.Qwen3Host(gt, device=cuda, seed=21)
        draft = q3.Qwen3Host(gd, device=cuda, seed=22)
        r = sr.SpecRunner(target, draft, batch=2, gamma=3, max_model_len=400, block_size=32,
                          temperature=0.7, mode="reference", device=cuda)
        r.load_prompts([[3, 4, 5, 6], list(range(200, 240))])
        torch.manual_seed(5)
        r.prefill()
        return r

    eager = make()
    torch.manual_seed(77)
    eager.step()  # same warm-up as the graph runner
    for _ in range(6):
        eager.step()
    graph = make()
    torch.manual_seed(77)
    graph.step()
    graph.capture()
    for _ in range(6):
        graph.replay()
    torch.cuda.synchronize()
    assert graph.lengths() == eager.lengths()
    for b in range(2):
        assert graph.tokens(b) == eager.tokens(b)


@pytest.mark.parametrize("batch", [1, 3])
def test_chained_steps_match_separate_bookkeeping(cuda, batch):
    """hs_spec_commit_next (the commit, then the next step's pre-allocation and first
    draft-step staging in one launch; with one sequence also the next verify staging,
    the draft tokens written straight into the verify input ids) against
    hs_spec_commit + hs_spec_prealloc + hs_draft_prepare (+ hs_verify_prepare) as
    separate launches: the same tokens every step, and at the end the same device
    state and staging once the separate runner has pre-allocated and staged its next
    step too (llm_engine.py:111-195, model_runner.py:294-310, 339-362)."""
    q3, sr = _mods()
    gt = _small(q3, layers=2)
    gd = _small(q3, layers=1)
    prompts = [[3, 4, 5, 6], list(range(200, 262)), [9] * 30][-batch:]

    def make(chain):
        target = q3.Qwen3Host(gt, device=cuda, seed=31)
        draft = q3.Qwen3Host(gd, device=cuda, seed=32)
        r = sr.SpecRunner(target, draft, batch=batch, gamma=3, max_model_len=300, block_size=32,
                          temperature=0.9, mode="reference", device=cuda, chain_steps=chain)
        r.load_prompts(prompts)
        torch.manual_seed(7)
        r.prefill()
        return r

    sep, chn = make(False), make(True)
    assert chn._stage_verify == (batch == 1) and not sep._stage_verify
    for step in range(8):
        torch.manual_seed(100 + step)
        sep.step()
        torch.manual_seed(100 + step)
        chn.step()
        print(f"chained step {step} (B={batch}): lengths {chn.lengths()}", flush=True)
        assert chn.lengths() == sep.lengths()
        for b in range(batch):
            assert chn.tokens(b) == sep.tokens(b)
        _check_state(chn)
        _check_state(sep)
    hv = _hv()
    G = sep._g()
    hv.ops.spec_prealloc(sep.state, G.gamma, out=G.elig)
    stage = hv.ops.draft_prepare(sep.state, None, 0, lookback=True)
    vstage = hv.ops.verify_prepare(sep.state, G.draft_tokens, G.gamma)
    torch.cuda.synchronize()
    for f in sep.state.FIELDS:
        assert torch.equal(getattr(sep.state, f), getattr(chn.state, f)), f
    assert torch.equal(G.elig, chn._g().elig)
    for x, y in zip(stage, chn.d_stage0):
        assert torch.equal(x, y)
    if batch == 1:
        # the staged verify rows: all but the draft tokens' ids, which the next
        # draft phase writes
        R = G.gamma + 1
        ids, *rest = chn._g().v_stage
        assert torch.equal(ids[0::R], vstage[0][0::R])
        for x, y in zip(vstage[1:], rest):
            assert torch.equal(x, y)


def test_filtered_topk_graph_replay_matches_eager(cuda):
    """Filtered mode with top-k 50 / top-p 0.9 at the full 151936-token vocabulary:
    the runner passes the top-k <= 64 promise, so acceptance runs as the single
    top-k launch inside the captured verify graph; replays must reproduce eager
    steps token for token, and every step emits 1..gamma+1 tokens."""
    q3, sr = _mods()
    gt = _small(q3, layers=2, vocab=151936)
    gd = _small(q3, layers=1, vocab=151936)

    def make():
        target = q3.Qwen3Host(gt, device=cuda, seed=23)
        draft = q3.Qwen3Host(gd, device=cuda, seed=24)
        r = sr.SpecRunner(target, draft, batch=2, gamma=3, max_model_len=400, block_size=32,
                          temperature=0.9, top_k=50, top_p=0.9, mode="filtered", device=cuda)
        assert r.topk_le64
        r.load_prompts([[3, 4, 5, 6], list(range(200, 240))])
        torch.manual_seed(6)
        r.prefill()
        return r

    eager = make()
    torch.manual_seed(78)
    prev = eager.lengths()
    for _ in range(7):
        eager.step()
        cur = eager.lengths()
        assert all(1 <= a - b <= 4 for a, b in zip(cur, prev)), (prev, cur)
        prev = cur
    graph = make()
    torch.manual_seed(78)
    graph.step()
    graph.capture()
    for _ in range(6):
        graph.replay()
    torch.cuda.synchronize()
    graph.check()
    assert graph.lengths() == eager.lengths()
    for b in range(2):
        assert graph.tokens(b) == eager.tokens(b)


def test_reference_mode_with_filters_keeps_unfiltered_draft_probs(cuda, orc):
    """Reference mode with top-k 50 / top-p 0.9 (model_runner.py:312-313 and
    :387-428): draft tokens come from the filtered Sampler, the draft
    probabilities are the unfiltered softmax(logits/T), and the acceptance
    compares them with the unfiltered target. Each step's draft rows have more
    than 50 nonzero probabilities, each draft token ranks among its row's 50
    largest, the acceptance equals the C oracle in reference mode on the step's
    own inputs, and graph replays reproduce eager steps."""
    q3, sr = _mods()
    gt = _small(q3, layers=2, vocab=151936)
    gd = _small(q3, layers=1, vocab=151936)

    def make():
        target = q3.Qwen3Host(gt, device=cuda, seed=31)
        draft = q3.Qwen3Host(gd, device=cuda, seed=32)
        r = sr.SpecRunner(target, draft, batch=2, gamma=3, max_model_len=400, block_size=32,
                          temperature=0.8, top_k=50, top_p=0.9, mode="reference", device=cuda)
        assert r.draft_out_kind == 2 and r.draft_mode == "filtered" and not r.topk_le64
        r.load_prompts([[3, 4, 5, 6], list(range(300, 330))])
        torch.manual_seed(8)
        r.prefill()
        return r

    def check_step(r):
        G = r._g()
        q = G.draft_probs.cpu()
        toks = G.draft_tokens.cpu()
        for b in range(r.B):
            for j in range(G.gamma):
                row = q[b, j]
                assert int((row > 0).sum()) > 50
                assert abs(float(row.double().sum()) - 1.0) < 1e-4
                assert int((row > row[int(toks[b, j])]).sum()) < 50
        _accept_matches_oracle(r, orc)

    eager = make()
    torch.manual_seed(91)
    for _ in range(5):
        eager.step()
        torch.cuda.synchronize()
        check_step(eager)
    graph = make()
    torch.manual_seed(91)
    graph.step()
    graph.capture()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        check_step(graph)
    graph.check()
    assert graph.lengths() == eager.lengths()
    for b in range(2):
        assert graph.tokens(b) == eager.tokens(b)


def test_fused_layer_matches_eager(cuda):
    """Fused kernels (RMSNorm inside the projections, qk-norm + RoPE + KV store,
    SwiGLU epilogue) vs the eager restatement of qwen3.py:72-185 (same attention
    kernel on both sides), at prefill size and at a 4-row verify pass."""
    q3, sr = _mods()
    g = _small(q3, layers=3, hidden=1024, heads=8, kv=4)
    target = q3.Qwen3Host(g, device=cuda, seed=31)
    draft = q3.Qwen3Host(g, share_from=target, num_layers=1)
    runner = sr.SpecRunner(target, draft, batch=1, gamma=2, max_model_len=256, block_size=32,
                           device=cuda)
    prompt = list(range(10, 60))
    runner.load_prompts([prompt])
    ids = torch.tensor(prompt, device=cuda)
    pos = torch.arange(len(prompt), device=cuda)
    slots = torch.tensor([int(runner.state.block_tables[0, i // 32]) * 32 + i % 32
                          for i in range(len(prompt))], dtype=torch.int32, device=cuda)
    cu = torch.tensor([0, len(prompt)], dtype=torch.int32, device=cuda)
    ctx = importlib.import_module("hilda-vllm_amd.utils.context")
    with torch.inference_mode():
        ctx.set_context(True, cu, cu, len(prompt), len(prompt), slots, None,
                        runner.state.block_tables)
        ref = target(ids, pos, reference=True).float()
        got = target(ids, pos).float()
        ctx.reset_context()
    torch.cuda.synchronize()
    err = (got - ref).abs()
    assert err.max() <= 0.05 * ref.abs().max() + 0.02, float(err.max())
    assert torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), dim=0) > 0.999
    # a 4-row verify pass (positions 50..53) runs the skinny projections with the
    # RMSNorm prologue; the reference pass stores its own K/V first, the fused pass
    # then overwrites those slots with its own
    n0 = len(prompt)
    ids4 = torch.tensor([5, 6, 7, 8], device=cuda)
    pos4 = torch.arange(n0, n0 + 4, device=cuda)
    slots4 = torch.tensor([int(runner.state.block_tables[0, i // 32]) * 32 + i % 32
                           for i in range(n0, n0 + 4)], dtype=torch.int32, device=cuda)
    cq = torch.tensor([0, 4], dtype=torch.int32, device=cuda)
    ck = torch.tensor([0, n0 + 4], dtype=torch.int32, device=cuda)
    with torch.inference_mode():
        ctx.set_context(True, cq, ck, 4, n0 + 4, slots4, None, runner.state.block_tables)
        ref4 = target(ids4, pos4, reference=True).float()
        got4 = target(ids4, pos4).float()
        ctx.reset_context()
    torch.cuda.synchronize()
    err4 = (got4 - ref4).abs()
    assert err4.max() <= 0.05 * ref4.abs().max() + 0.02, float(err4.max())
    assert torch.nn.functional.cosine_similarity(got4.flatten(), ref4.flatten(), dim=0) > 0.999


@pytest.mark.parametrize("draft_kind", ["self", "random"])
def test_adaptive_gamma_fp8_block_pressure(cuda, draft_kind):
    """Config 4 at test scale: adaptive gamma, FP8 target cache, a block pool too
    small for every sequence at once (some sequences must wait), sequences of
    different max_tokens finishing and releasing their blocks."""
    q3, sr = _mods()
    AG = importlib.import_module("hilda-vllm_amd.engine.adaptive_gamma").AdaptiveGamma
    g = _small(q3, layers=2)
    target = q3.Qwen3Host(g, device=cuda, seed=61)
    if draft_kind == "self":
        draft = q3.Qwen3Host(g, share_from=target)
        mode, temp, g0 = "greedy", 0.0, 3
    else:
        draft = q3.Qwen3Host(_small(q3, layers=1), device=cuda, seed=62)
        mode, temp, g0 = "reference", 0.9, 5
    B, bs = 6, 32
    # five short sequences that never outgrow their two prompt blocks (even with the
    # lookahead of gamma 8) and one long sequence whose prompt fills its three blocks:
    # with no spare block it needs a fourth at once and waits until the short ones
    # finish and release theirs
    prompts = [list(range(10 + i, 10 + i + n)) for i, n in enumerate([33, 34, 35, 36, 37, 95])]
    max_tokens = [12, 14, 10, 16, 8, 200]
    num_blocks = 13  # exactly the prompt blocks
    runner = sr.SpecRunner(target, draft, batch=B, gamma=g0, max_model_len=400, block_size=bs,
                           kv_cache_dtype="fp8", num_blocks=num_blocks, temperature=temp,
                           mode=mode, adaptive=True, device=cuda)
    runner.load_prompts(prompts)
    st = runner.state
    st.max_tokens.copy_(torch.tensor(max_tokens, dtype=torch.int32))
    runner.prefill()
    waited = 0
    for step in range(400):
        fin = st.finished.cpu()
        if bool(fin.all()):
            break
        runner.step_graph()
        G = runner._per_gamma[runner.history[-1][0]]
        elig = G.elig.cpu()
        waited += int(((elig == 0) & (fin == 0)).sum())
        _check_blocks(runner)
    torch.cuda.synchronize()
    assert bool(st.finished.cpu().all()), "sequences did not finish"
    lens = runner.lengths()
    assert lens == [len(p) + m for p, m in zip(prompts, max_tokens)]
    assert int(st.free_hdr[1]) == num_blocks  # every block released
    assert waited > 0, "the block pool never ran short"
    # the gamma trajectory is the controller's on the recorded totals
    ctl = AG(g0, max_gamma=8)
    for k, (gk, acc, prop) in enumerate(runner.history):
        assert gk == ctl.gamma, (k, runner.history[:k + 1])
        assert 0 <= acc <= prop
        ctl.update(acc, prop)
    gammas = [h[0] for h in runner.history]
    print("gamma trajectory", gammas, flush=True)
    if draft_kind == "self":
        assert max(gammas) > g0, gammas  # high acceptance raises gamma
    else:
        assert min(gammas) < g0, gammas  # low acceptance lowers it


def _check_blocks(runner):
    st = runner.state
    nb = st.num_seq_blocks.cpu()
    lens = st.context_lens.cpu()
    fin = st.finished.cpu()
    for b in range(runner.B):
        if fin[b]:
            assert int(nb[b]) == 0
        else:
            assert int(nb[b]) == (int(lens[b]) + runner.bs - 1) // runner.bs
    assert int(st.free_hdr[1]) + int(nb.sum()) == runner.num_blocks


def test_preemption_frees_blocks_and_recomputes(cuda):
    """A pool that cannot hold every sequence to its end: when no sequence gets its
    blocks the longest is preempted (scheduler.py:313-320: blocks back to the free
    list, the sequence out of the batch) and readmitted once the free list holds its
    whole length, its K/V recomputed by prefill. Every sequence must still reach its
    max_tokens with the block accounting exact after every step."""
    q3, sr = _mods()
    g = _small(q3, layers=2)
    target = q3.Qwen3Host(g, device=cuda, seed=71)
    draft = q3.Qwen3Host(g, share_from=target)
    B, bs = 4, 32
    prompts = [list(range(20 + i, 20 + i + n)) for i, n in enumerate([33, 35, 37, 39])]
    max_tokens = [150, 150, 150, 150]  # 6 blocks each at the end, 24 in all
    num_blocks = 12                      # the 8 prompt blocks and 4 more
    runner = sr.SpecRunner(target, draft, batch=B, gamma=3, max_model_len=400, block_size=bs,
                           kv_cache_dtype="fp8", num_blocks=num_blocks, temperature=0.0,
                           mode="greedy", adaptive=True, device=cuda)
    runner.load_prompts(prompts)
    st = runner.state
    st.max_tokens.copy_(torch.tensor(max_tokens, dtype=torch.int32))
    runner.prefill()
    preempted = readmitted = 0
    for step in range(600):
        if runner.preempted:
            readmitted += runner.readmit()
            _check_blocks(runner)
        fin = st.finished.cpu()
        if bool(fin.all()) and not runner.preempted:
            break
        runner.step_graph()
        G = runner._per_gamma[runner.history[-1][0]]
        fin = st.finished.cpu()
        if int(G.elig.sum()) == 0 and not bool(fin.all()):
            lens = st.context_lens.cpu().masked_fill(fin.bool(), -1)
            runner.preempt(int(torch.argmax(lens)))
            preempted += 1
        _check_blocks(runner)
    torch.cuda.synchronize()
    print(f"preempted {preempted} readmitted {readmitted} steps {step}", flush=True)
    assert bool(st.finished.cpu().all()) and not runner.preempted, "sequences did not finish"
    assert runner.lengths() == [len(p) + m for p, m in zip(prompts, max_tokens)]
    assert preempted > 0 and readmitted == preempted
    assert int(st.free_hdr[1]) == num_blocks


def test_config4_shape_adaptive_fp8_to_8192(cuda):
    """Config 4's shape: B = 32, prompts ~ U[32, 128], every sequence decoding to an
    8192-token context in an FP8 target cache of 256-token blocks (32-entry block
    tables) whose pool holds 3/4 of the final need, gamma adapted in [1, 7]. The
    models keep config 3's head geometry (16 Q / 8 KV heads of 128) at two layers
    and a 3000-token vocabulary so the run fits a test; the draft is the target's
    first layer. Invariants after every step: block accounting; at the end:
    completion, every block released, no invalid acceptance output, and the gamma
    trajectory equal to the controller's on the recorded totals."""
    import numpy as np
    q3, sr = _mods()
    AG = importlib.import_module("hilda-vllm_amd.engine.adaptive_gamma").AdaptiveGamma
    g = q3.Qwen3Geometry(num_layers=2, hidden=1024, num_heads=16, num_kv_heads=8, ffn=1024,
                         vocab=3000, max_position=8704)
    target = q3.Qwen3Host(g, device=cuda, seed=81)
    draft = q3.Qwen3Host(g, share_from=target, num_layers=1)
    B, bs, ctx = 32, 256, 8192
    rng = np.random.default_rng(82)
    plens = rng.integers(32, 129, size=B)
    prompts = [rng.integers(0, 3000, size=n).tolist() for n in plens]
    need = B * -(-(ctx + 8) // bs)
    num_blocks = int(0.75 * need)
    runner = sr.SpecRunner(target, draft, batch=B, gamma=3, max_model_len=ctx + 16,
                           block_size=bs, kv_cache_dtype="fp8", num_blocks=num_blocks,
                           temperature=0.6, mode="reference", adaptive=True, max_gamma=7,
                           device=cuda)
    assert runner.W >= 32
    runner.load_prompts(prompts)
    st = runner.state
    st.max_tokens.copy_(torch.tensor([ctx - int(n) for n in plens], dtype=torch.int32))
    runner.prefill()
    scales = runner.kv_scales()
    assert all(0 < k < 1 and 0 < v < 1 for k, v in scales), scales  # calibrated amax/448
    preempted = readmitted = steps = checked = 0
    while steps < 20000:
        if runner.preempted:
            readmitted += runner.readmit()
            _check_blocks(runner)
        fin = st.finished.cpu()
        if bool(fin.all()) and not runner.preempted:
            break
        len0 = st.context_lens.cpu()
        runner.step_graph()
        G = runner._per_gamma[runner.history[-1][0]]
        fin1 = st.finished.cpu()
        if bool((fin1 == fin).all()):
            # the controller's totals are this step's: every participating sequence
            # appended its accepted drafts plus one token (also at the step that
            # captured a new gamma's graphs)
            appended = int((st.context_lens.cpu() - len0).sum())
            assert runner.history[-1][1] == appended - int(G.elig.sum()), (
                steps, runner.history[-1], appended)
            checked += 1
        fin = fin1
        if int(G.elig.sum()) == 0 and not bool(fin.all()):
            lens = st.context_lens.cpu().masked_fill(fin.bool(), -1)
            runner.preempt(int(torch.argmax(lens)))
            preempted += 1
        _check_blocks(runner)
        steps += 1
        if steps % 500 == 0:
            print(f"config4 shape: step {steps} tokens {sum(runner.lengths())} "
                  f"gamma {runner.gamma} preempted {preempted}", flush=True)
    torch.cuda.synchronize()
    runner.check()
    print(f"config4 shape: {steps} steps ({checked} with totals checked), preempted "
          f"{preempted}, readmitted {readmitted}", flush=True)
    assert bool(st.finished.cpu().all()) and not runner.preempted, "sequences did not finish"
    assert runner.lengths() == [ctx] * B
    assert int(st.free_hdr[1]) == num_blocks
    assert preempted > 0 and readmitted == preempted
    ctl = AG(3, max_gamma=7)
    for k, (gk, acc, prop) in enumerate(runner.history):
        assert gk == ctl.gamma, (k, runner.history[max(0, k - 3):k + 1])
        assert 1 <= gk <= 7 and 0 <= acc <= prop
        ctl.update(acc, prop)
    gammas = [h[0] for h in runner.history]
    print("gamma histogram", {k: gammas.count(k) for k in sorted(set(gammas))}, flush=True)


def _accept_matches_oracle(r, orc):
    """The acceptance of the runner's last step against the C oracle on that step's
    own inputs (model_runner.py:387-428): its target logits, draft probabilities and
    tokens, temperatures and uniforms, read back after the step; accepted counts,
    emitted tokens and lengths must be equal."""
    G = r._g()
    B, g, V = r.B, G.gamma, r.V
    logits = G.logits.float().cpu().numpy().reshape(B, g + 1, V)
    ref = orc.spec_accept(logits, G.draft_probs.cpu().numpy(),
                          G.draft_tokens.cpu().numpy(), r.temps.cpu().numpy(),
                          G.u_acc.cpu().numpy(), r.u_res.cpu().numpy())
    nacc, out, olen = (t.cpu().numpy() for t in G.last)
    np.testing.assert_array_equal(nacc, ref["num_accepted"])
    np.testing.assert_array_equal(olen, ref["out_len"])
    for b in range(B):
        n = int(olen[b])
        np.testing.assert_array_equal(out[b, :n], ref["out_tokens"][b, :n])
    return nacc


@pytest.mark.parametrize("draft_kind", ["qwen3-0.6b", "forced"])
def test_config3_real_geometry_graph_matches_eager(cuda, orc, draft_kind):
    """Config 3 at its real geometry: random-init Qwen3-8B target (36 layers,
    hidden 4096, 32 / 8 heads, FFN 12288, vocab 151936) with the Qwen3-0.6B draft
    or the forced-acceptance draft (the target's first 28 layers and LM head),
    batch 1, gamma 3, T 0.6, a 64-token prompt, max_model_len 4096 (the
    reference's). Six steps replayed from the captured HIP graphs emit the same
    tokens as six eager steps; every step's acceptance (eager and replayed)
    equals the C oracle on the step's own logits, draft probabilities and
    uniforms; every step emits 1 to gamma + 1 tokens; the forced draft has
    drafts accepted."""
    q3, sr = _mods()
    print(f"config 3 real geometry, draft {draft_kind}", flush=True)
    target = q3.Qwen3Host(q3.QWEN3_8B, device=cuda, seed=1)
    draft = (q3.Qwen3Host(q3.QWEN3_8B, share_from=target, num_layers=28)
             if draft_kind == "forced" else q3.Qwen3Host(q3.QWEN3_0_6B, device=cuda, seed=2))
    prompt = torch.randint(0, 10000, (64,), generator=torch.Generator().manual_seed(0)).tolist()

    def run(graphs):
        r = sr.SpecRunner(target, draft, batch=1, gamma=3, max_model_len=4096, temperature=0.6,
                          mode="reference", device=cuda)
        r.load_prompts([prompt])
        torch.manual_seed(3)
        r.prefill()
        torch.manual_seed(77)
        r.step()
        _accept_matches_oracle(r, orc)
        if graphs:
            r.capture()
        lens = [r.lengths()[0]]
        for _ in range(6):
            r.replay() if graphs else r.step()
            torch.cuda.synchronize()
            _accept_matches_oracle(r, orc)
            lens.append(r.lengths()[0])
        r.check()
        toks = r.tokens(0)
        del r
        torch.cuda.empty_cache()
        return lens, toks

    lens_e, toks_e = run(False)
    lens_g, toks_g = run(True)
    assert lens_g == lens_e and toks_g == toks_e
    steps = [b - a for a, b in zip(lens_e, lens_e[1:])]
    assert all(1 <= s <= 4 for s in steps), steps
    if draft_kind == "forced":
        assert sum(steps) > len(steps), steps  # some drafts accepted


def test_fp8_calibration_matches_bf16_cache_amax(cuda):
    """FP8 scale calibration (prefill without given scales) attends over each layer's
    own bf16 K/V rows, so every layer's amax is taken on the activations of an exact
    cache: the scales equal headroom * amax / 448 of the K and V rows that a
    bf16-cache run of the same model and prompt stores, layer by layer. After a few
    steps, kv_saturation() reports the share of clipped codes (in [0, 1))."""
    q3, sr = _mods()
    g = _small(q3, layers=3)
    target = q3.Qwen3Host(g, device=cuda, seed=21)
    draft = q3.Qwen3Host(g, device=cuda, seed=22)
    prompt = torch.randint(0, 3000, (40,), generator=torch.Generator().manual_seed(4)).tolist()
    print("fp8 calibration vs bf16 cache amax", flush=True)

    def runner(kv):
        r = sr.SpecRunner(target, draft, batch=1, gamma=3, max_model_len=256, temperature=0.6,
                          mode="reference", kv_cache_dtype=kv, device=cuda)
        r.load_prompts([prompt])
        torch.manual_seed(1)
        r.prefill()
        torch.cuda.synchronize()
        return r

    r8 = runner("fp8")
    scales = r8.kv_scales()
    rb = runner("auto")
    bt = rb.state.block_tables[0].cpu().tolist()
    slots = [bt[p // rb.bs] * rb.bs + p % rb.bs for p in range(len(prompt))]
    idx = torch.tensor(slots, device=cuda)
    for i, (ks, vs) in enumerate(scales):
        kr = rb.kv[0, i].reshape(-1, g.num_kv_heads, g.head_dim)[idx]
        vr = rb.kv[1, i].reshape(-1, g.num_kv_heads, g.head_dim)[idx]
        ek = kr.float().abs().amax().item() * r8.FP8_HEADROOM / 448.0
        ev = vr.float().abs().amax().item() * r8.FP8_HEADROOM / 448.0
        assert abs(ks - ek) <= 1e-6 * ek and abs(vs - ev) <= 1e-6 * ev, (i, ks, ek, vs, ev)
    for _ in range(3):
        r8.step()
    sat = r8.kv_saturation()
    assert 0.0 <= sat < 1.0
    print(f"fp8 saturated share after 3 steps: {sat:.2e}", flush=True)
