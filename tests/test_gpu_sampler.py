"""GPU parity of the fused acceptance sampler and the row sampler.

Every test runs the HIP kernels through the C ABI (hilda-vllm_amd.ops) and
compares with the CPU oracle on identical seeded inputs. Accept counts, token
IDs, row maxima and normalisers are expected bit-exact (both sides evaluate
the same arithmetic); probabilities are checked bit-exact as well, which
implies the 1e-5 relative bound of the specification.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _to_dev(w, cuda):
    if w["dtype"] == "bf16":
        lg = torch.from_numpy(w["logits_bits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        lg = torch.from_numpy(w["logits"]).to(cuda)
    t = {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(cuda)
         for k in ["draft_probs", "draft_tokens", "temperatures", "top_ks", "top_ps",
                   "u_accept", "u_resample"]}
    return lg, t


def _run_both(hv, orc, w, cuda, mode):
    lg, t = _to_dev(w, cuda)
    nacc, out, olen, stats = hv.ops.spec_accept(
        lg, t["draft_probs"], t["draft_tokens"], t["temperatures"], t["u_accept"],
        t["u_resample"], mode=mode, top_ks=t["top_ks"], top_ps=t["top_ps"], row_stats=True)
    torch.cuda.synchronize()
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode=mode, top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    return (nacc.cpu().numpy(), out.cpu().numpy(), olen.cpu().numpy(), stats.cpu().numpy()), ref


def _assert_same(got, ref, check_stats=True):
    nacc, out, olen, stats = got
    np.testing.assert_array_equal(nacc, ref["num_accepted"])
    np.testing.assert_array_equal(out, ref["out_tokens"])
    np.testing.assert_array_equal(olen, ref["out_len"])
    if check_stats:
        np.testing.assert_array_equal(stats, ref["row_stats"])


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_config0_reference_mode(hv, orc, cuda, seed):
    w = hv.synthetic.accept_workload(1, 3, seed=seed)
    print(f"config0 reference seed={seed}", flush=True)
    got, ref = _run_both(hv, orc, w, cuda, "reference")
    _assert_same(got, ref)


@pytest.mark.parametrize("seed", [0, 5])
def test_config0_filtered_mode(hv, orc, cuda, seed):
    w = hv.synthetic.accept_workload(1, 3, seed=seed, top_k=50, top_p=0.9, mode="filtered")
    print(f"config0 filtered seed={seed}", flush=True)
    got, ref = _run_both(hv, orc, w, cuda, "filtered")
    _assert_same(got, ref)


@pytest.mark.parametrize("gamma", [1, 3, 5])
def test_config1_batched_bf16_filtered(hv, orc, cuda, gamma):
    w = hv.synthetic.accept_workload(8, gamma, seed=100 + gamma, dtype="bf16",
                                     per_seq_settings=True, mode="filtered")
    print(f"config1 filtered B=8 gamma={gamma}", flush=True)
    got, ref = _run_both(hv, orc, w, cuda, "filtered")
    _assert_same(got, ref)


@pytest.mark.parametrize("gamma", [1, 3, 5])
def test_config1_batched_bf16_reference(hv, orc, cuda, gamma):
    w = hv.synthetic.accept_workload(8, gamma, seed=200 + gamma, dtype="bf16",
                                     per_seq_settings=True)
    got, ref = _run_both(hv, orc, w, cuda, "reference")
    _assert_same(got, ref)


def test_config1_greedy(hv, orc, cuda):
    w = hv.synthetic.accept_workload(8, 3, seed=300, dtype="bf16")
    # make some drafts match the argmax so that acceptance paths vary
    am = w["logits"].argmax(-1)
    for b in range(8):
        w["draft_tokens"][b, : b % 4] = am[b, : b % 4]
    got, ref = _run_both(hv, orc, w, cuda, "greedy")
    _assert_same(got, ref, check_stats=False)


def test_all_reject_positions_with_small_vocab(hv, orc, cuda):
    """Sweeps the uniforms so that every first-reject position 0..gamma occurs."""
    rng = np.random.default_rng(7)
    B, g, V = 64, 4, 3000  # V not a multiple of the 2048 chunk
    w = hv.synthetic.accept_workload(B, g, vocab=V, seed=7)
    w["u_accept"] = np.sort(rng.random((B, g), dtype=np.float32), axis=0)
    got, ref = _run_both(hv, orc, w, cuda, "reference")
    _assert_same(got, ref)
    assert len(set(ref["num_accepted"].tolist())) >= 3


@pytest.mark.parametrize("B,g,dtype", [(1, 1, "f32"), (1, 3, "bf16"), (1, 7, "f32"),
                                       (2, 5, "bf16"), (3, 2, "f32")])
def test_small_batch_single_launch_every_reject_position(hv, orc, cuda, B, g, dtype):
    """Batches whose grid fits one workgroup per CU (B <= 3 at V = 151936) run the
    single-launch kernel with grid barriers between its phases. The acceptance
    uniforms force every first-reject position 0..gamma in turn (u = 0 accepts any
    draft with nonzero target probability, u = 1 rejects), so both the residual and
    the bonus draw run on it; every call reuses the same barrier state."""
    V = 151936 if B == 1 else 50000
    base = hv.synthetic.accept_workload(B, g, vocab=V, seed=500 + 10 * B + g, dtype=dtype,
                                        per_seq_settings=(B > 1))
    for r in range(g + 1):
        w = dict(base)
        u = np.zeros((B, g), np.float32)
        if r < g:
            u[:, r] = 1.0
        w["u_accept"] = u
        w["u_resample"] = ((np.arange(B, dtype=np.float32) + 0.5 + r) / (B + g + 1)).astype(
            np.float32)
        print(f"single-launch B={B} gamma={g} {dtype} reject at {r}", flush=True)
        got, ref = _run_both(hv, orc, w, cuda, "reference")
        _assert_same(got, ref)
        assert (ref["num_accepted"] == r).all()


def test_single_launch_ignores_matching_stale_words_elsewhere(hv, orc, cuda):
    """The single-launch kernel's epoch-tagged words live in a fixed region after the
    sync word (64 KiB at offset 256), written by no other kernel. Every other word of
    the shared workspace is filled with a value whose high half is the next launch's
    epoch, as stale chain data of another shape could eventually be; the call must
    still match the oracle and report no timed-out wait."""
    V = 151936
    w = hv.synthetic.accept_workload(1, 3, seed=77, dtype="bf16")
    got, ref = _run_both(hv, orc, w, cuda, "reference")  # sets up the shared workspace
    _assert_same(got, ref)
    nbytes = hv._lib.lib().hs_spec_accept_workspace_size(1, 3, V)
    ws = hv.ops.workspace(cuda, nbytes, "spec_accept")
    rng = np.random.default_rng(5)
    for step in range(2):
        torch.cuda.synchronize()
        sync = ws[:16].cpu().numpy().view(np.uint64)
        assert int(sync[1]) & 0xffffffff == 0  # no wait ran out so far
        nxt = (int(sync[0]) >> 32) + 1
        words = ws[256 + 65536:].view(torch.int64)
        low = torch.from_numpy(rng.integers(0, 2**32, size=words.numel(), dtype=np.int64))
        words.copy_(((nxt << 32) | low).to(cuda))
        w2 = hv.synthetic.accept_workload(1, 3, seed=78 + step, dtype="bf16")
        print(f"stale words carry epoch {nxt}", flush=True)
        got, ref = _run_both(hv, orc, w2, cuda, "reference")
        _assert_same(got, ref)
    torch.cuda.synchronize()
    assert int(ws[:16].cpu().numpy().view(np.uint64)[1]) & 0xffffffff == 0


def test_draft_equal_to_target_accepts_everything(hv, orc, cuda):
    B, g, V = 4, 3, 5000
    w = hv.synthetic.accept_workload(B, g, vocab=V, seed=8)
    P = orc.sampler(w["logits"].reshape(-1, V))["probs"].reshape(B, g + 1, V)
    w["draft_probs"] = np.ascontiguousarray(P[:, :g])
    w["u_accept"][:] = np.float32(0.9999999)
    got, ref = _run_both(hv, orc, w, cuda, "reference")
    _assert_same(got, ref)
    assert (ref["num_accepted"] == g).all()


def test_residual_fallback_when_draft_equals_target(hv, orc, cuda):
    B, g, V = 2, 2, 4099
    w = hv.synthetic.accept_workload(B, g, vocab=V, seed=9)
    P = orc.sampler(w["logits"].reshape(-1, V))["probs"].reshape(B, g + 1, V)
    w["draft_probs"] = np.ascontiguousarray(P[:, :g])
    w["u_accept"][:] = 1.0  # forces a reject at row 0 with an all-zero residual
    got, ref = _run_both(hv, orc, w, cuda, "reference")
    _assert_same(got, ref)
    assert (ref["num_accepted"] == 0).all()


def test_unaligned_rows_use_scalar_path(hv, orc, cuda):
    B, g, V = 3, 2, 1001
    w = hv.synthetic.accept_workload(B, g, vocab=V, seed=10)
    lg, t = _to_dev(w, cuda)
    # embed rows in a wider buffer with an odd stride
    big = torch.zeros((B * (g + 1), V + 3), dtype=torch.float32, device=cuda)
    big[:, 1:V + 1] = lg.reshape(B * (g + 1), V)
    view = big[:, 1:V + 1].reshape(B, g + 1, V)
    nacc, out, olen = hv.ops.spec_accept(view, t["draft_probs"], t["draft_tokens"],
                                         t["temperatures"], t["u_accept"], t["u_resample"])
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"])
    np.testing.assert_array_equal(nacc.cpu().numpy(), ref["num_accepted"])
    np.testing.assert_array_equal(out.cpu().numpy(), ref["out_tokens"])


@pytest.mark.parametrize("mode", ["reference", "filtered"])
def test_sampler_probs_and_tokens(hv, orc, cuda, mode):
    rng = np.random.default_rng(11)
    rows, V = 6, 151936
    logits = (rng.standard_normal((rows, V), dtype=np.float32) * 2)
    temps = np.array([1.0, 0.6, 1.2, 0.9, 1.0, 0.5], np.float32)
    tk = np.array([50, 0, 20, 1, 0, 5000], np.int32)
    tp = np.array([0.9, 0.8, 1.0, 1.0, 0.5, 0.95], np.float32)
    u = rng.random(rows, dtype=np.float32)
    r = hv.ops.sample_rows(torch.from_numpy(logits).to(cuda), torch.from_numpy(temps).to(cuda),
                           torch.from_numpy(tk).to(cuda), torch.from_numpy(tp).to(cuda),
                           mode=mode, uniforms=torch.from_numpy(u).to(cuda), want_probs=True,
                           row_stats=True)
    ref = orc.sampler(logits, temps, tk, tp, mode=mode, uniforms=u)
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), ref["probs"])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sampler_unfiltered_probs_beside_filtered_draw(hv, orc, cuda, dtype):
    """out_kind 2 (model_runner.py:312-313: the draft token from the filtered
    Sampler, the draft probabilities from the unfiltered softmax(logits/T)): the
    tokens equal the oracle's filtered draw and the probabilities the oracle's
    reference-mode (unfiltered) rows, bit for bit; rows without a filter (k 0,
    p 1) included, and the same call in reference mode equals out_kind 0."""
    rng = np.random.default_rng(21)
    rows, V = 6, 151936
    logits = (rng.standard_normal((rows, V), dtype=np.float32) * 2)
    if dtype == "bf16":
        lg = torch.from_numpy(logits).to(cuda).to(torch.bfloat16)
        logits = lg.float().cpu().numpy()
    else:
        lg = torch.from_numpy(logits).to(cuda)
    temps = np.array([1.0, 0.6, 1.2, 0.9, 1.0, 0.5], np.float32)
    tk = np.array([50, 0, 20, 1, 0, 5000], np.int32)
    tp = np.array([0.9, 0.8, 1.0, 1.0, 1.0, 0.95], np.float32)
    u = rng.random(rows, dtype=np.float32)
    dev = {k: torch.from_numpy(v).to(cuda) for k, v in
           dict(t=temps, k=tk, p=tp, u=u).items()}
    r = hv.ops.sample_rows(lg, dev["t"], dev["k"], dev["p"], mode="filtered",
                           uniforms=dev["u"], want_probs=True, out_kind=2)
    filt = orc.sampler(logits, temps, tk, tp, mode="filtered", uniforms=u)
    full = orc.sampler(logits, temps, mode="reference", uniforms=u)
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), filt["tokens"])
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), full["probs"])
    assert (filt["probs"] == 0).any() and not (full["probs"][:, :100] == 0).all()
    r2 = hv.ops.sample_rows(lg, dev["t"], mode="reference", uniforms=dev["u"], want_probs=True,
                            out_kind=2)
    np.testing.assert_array_equal(r2["tokens"].cpu().numpy(), full["tokens"])
    np.testing.assert_array_equal(r2["probs"].cpu().numpy(), full["probs"])


def test_sampler_masked_logits_match_reference_kats(hv, cuda):
    """tests/test_sampler.py:6-44 of the reference, through the GPU filter."""
    x = torch.tensor([[5.0, 4.0, 3.0, 2.0]], device=cuda)
    one = torch.ones(1, device=cuda)
    r = hv.ops.sample_rows(x, one, torch.tensor([2], device=cuda), torch.ones(1, device=cuda),
                           mode="filtered", want_probs=True, out_kind=1)
    m = r["probs"][0].cpu()
    assert torch.isneginf(m[2]) and torch.isneginf(m[3]) and m[0] == 5.0 and m[1] == 4.0
    lg = torch.log(torch.tensor([[0.5, 0.3, 0.15, 0.05]], dtype=torch.float32)).to(cuda)
    for p, expect in [(0.81, [True, True, False, False]), (0.8, [True, False, False, False])]:
        r = hv.ops.sample_rows(lg, one, torch.zeros(1, dtype=torch.int32, device=cuda),
                               torch.tensor([p], device=cuda), mode="filtered", want_probs=True,
                               out_kind=1)
        assert torch.isfinite(r["probs"][0].cpu()).tolist() == expect


def test_sampler_greedy_with_ties(hv, orc, cuda):
    rng = np.random.default_rng(12)
    logits = rng.integers(-2, 2, size=(5, 40000)).astype(np.float32)
    r = hv.ops.sample_rows(torch.from_numpy(logits).to(cuda), mode="greedy")
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), logits.argmax(-1))


@pytest.mark.parametrize("k,p", [(1000, 1.0), (7000, 0.9), (0, 0.3), (3, 1.0)])
def test_filter_ties_in_bf16(hv, orc, cuda, k, p):
    """bf16-rounded logits tie often; the kept set must break ties by index."""
    rng = np.random.default_rng(13 + k)
    V = 151936
    x = (rng.standard_normal((2, V), dtype=np.float32) * 2)
    bits = hv.synthetic.f32_to_bf16_bits(x)
    xf = hv.synthetic.bf16_bits_to_f32(bits)
    lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    T = np.ones(2, np.float32)
    tk = np.full(2, k, np.int32)
    tp = np.full(2, p, np.float32)
    u = np.array([0.3, 0.7], np.float32)
    r = hv.ops.sample_rows(lg, torch.from_numpy(T).to(cuda), torch.from_numpy(tk).to(cuda),
                           torch.from_numpy(tp).to(cuda), mode="filtered",
                           uniforms=torch.from_numpy(u).to(cuda), want_probs=True)
    ref = orc.sampler(xf, T, tk, tp, mode="filtered", uniforms=u)
    got = r["probs"].cpu().numpy()
    np.testing.assert_array_equal(got > 0, ref["probs"] > 0)
    np.testing.assert_array_equal(got, ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])


def test_repeated_calls_reuse_workspace(hv, orc, cuda):
    w = hv.synthetic.accept_workload(4, 3, vocab=20000, seed=14)
    outs = [_run_both(hv, orc, w, cuda, "reference")[0][1] for _ in range(3)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


def test_shape_changes_share_workspace(hv, orc, cuda):
    """Calls of different (B, gamma, V) reuse one workspace; the ticket
    counters must still start from zero on every call."""
    shapes = [(8, 5, 30000), (2, 1, 4097), (16, 3, 2048), (1, 7, 151936), (8, 1, 30000)]
    for i, (B, g, V) in enumerate(shapes):
        w = hv.synthetic.accept_workload(B, g, vocab=V, seed=400 + i)
        got, ref = _run_both(hv, orc, w, cuda, "reference")
        _assert_same(got, ref)


def _degenerate_rows(V, rng):
    rows = [np.zeros(V, np.float32),                                    # all tied
            rng.integers(0, 2, size=V).astype(np.float32),              # two values
            np.where(rng.random(V) < 0.5, -np.inf, rng.standard_normal(V) * 3).astype(np.float32),
            np.concatenate([[40.0], np.full(V - 1, -5.0)]).astype(np.float32),  # one spike
            (rng.standard_normal(V) * 0.05).astype(np.float32)]        # nearly flat
    return np.stack(rows)


@pytest.mark.parametrize("k,p", [(0, 0.9), (0, 0.5), (20, 1.0), (50, 0.9), (100, 0.8), (0, 0.999)])
def test_filter_paths_on_degenerate_rows(hv, orc, cuda, k, p):
    """Rows that overflow the LDS candidate capacity (ties, flat logits) take the
    radix fallback; -inf entries and spikes exercise the bucket edges."""
    rng = np.random.default_rng(31 + k)
    V = 151936
    x = _degenerate_rows(V, rng)
    R = x.shape[0]
    T = np.full(R, 0.8, np.float32)
    tk = np.full(R, k, np.int32)
    tp = np.full(R, p, np.float32)
    u = rng.random(R).astype(np.float32)
    print(f"degenerate rows k={k} p={p}", flush=True)
    r = hv.ops.sample_rows(torch.from_numpy(x).to(cuda), torch.from_numpy(T).to(cuda),
                           torch.from_numpy(tk).to(cuda), torch.from_numpy(tp).to(cuda),
                           mode="filtered", uniforms=torch.from_numpy(u).to(cuda),
                           want_probs=True, row_stats=True)
    ref = orc.sampler(x, T, tk, tp, mode="filtered", uniforms=u)
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])


@pytest.mark.parametrize("k,p", [(20, 0.9), (50, 0.5), (0, 0.95), (0, 0.8), (75, 0.99)])
def test_filter_fast_paths_random_rows(hv, orc, cuda, k, p):
    """Chunk-maximum gather (k <= chunks) and (M - x) bucket (top-p alone) paths
    on N(0, 2^2) bf16 rows at several temperatures."""
    rng = np.random.default_rng(51 + k)
    V = 151936
    R = 6
    x = rng.standard_normal((R, V), dtype=np.float32) * 2
    bits = hv.synthetic.f32_to_bf16_bits(x)
    xf = hv.synthetic.bf16_bits_to_f32(bits)
    lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    T = np.array([0.5, 0.7, 0.9, 1.0, 1.2, 2.0], np.float32)
    tk = np.full(R, k, np.int32)
    tp = np.full(R, p, np.float32)
    u = rng.random(R).astype(np.float32)
    r = hv.ops.sample_rows(lg, torch.from_numpy(T).to(cuda), torch.from_numpy(tk).to(cuda),
                           torch.from_numpy(tp).to(cuda), mode="filtered",
                           uniforms=torch.from_numpy(u).to(cuda), want_probs=True, row_stats=True)
    ref = orc.sampler(xf, T, tk, tp, mode="filtered", uniforms=u)
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])


@pytest.mark.parametrize("dtype,unaligned", [("bf16", False), ("f32", False), ("bf16", True)])
def test_filter_segmented_passes_many_rows(hv, orc, cuda, dtype, unaligned):
    """128 rows, 108 of them top-p alone: the filter passes give each workgroup a segment of
    4-5 consecutive chunks of one row (histograms accumulate over the segment), and the
    temperatures put the boundary bucket both below and above the refinement threshold.
    Unaligned rows send the top-k rows through the same segmented pass."""
    rng = np.random.default_rng(71)
    V, R = 151936, 128
    x = rng.standard_normal((R, V), dtype=np.float32) * 2
    if dtype == "bf16":
        bits = hv.synthetic.f32_to_bf16_bits(x)
        xf = hv.synthetic.bf16_bits_to_f32(bits)
        lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        xf = x
        lg = torch.from_numpy(x).to(cuda)
    if unaligned:  # odd row stride, rows 2 bytes past a 16-byte boundary
        big = torch.zeros((R, V + 3), dtype=lg.dtype, device=cuda)
        big[:, 1:V + 1] = lg
        lg = big[:, 1:V + 1]
    T = rng.choice(np.array([0.6, 0.8, 1.0, 1.3], np.float32), R)
    tk = np.zeros(R, np.int32)
    tk[:8] = 20
    tk[8:12] = 50
    tp = rng.choice(np.array([0.5, 0.8, 0.9, 0.95], np.float32), R)
    tp[:12] = 1.0
    tp[120:] = 1.0
    u = rng.random(R).astype(np.float32)
    print(f"segmented filter passes {dtype} unaligned={unaligned}", flush=True)
    r = hv.ops.sample_rows(lg, torch.from_numpy(T).to(cuda), torch.from_numpy(tk).to(cuda),
                           torch.from_numpy(tp).to(cuda), mode="filtered",
                           uniforms=torch.from_numpy(u).to(cuda), want_probs=True, row_stats=True)
    ref = orc.sampler(xf, T, tk, tp, mode="filtered", uniforms=u)
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])


@pytest.mark.parametrize("rows,dtype,temps", [(1, "bf16", [0.6]), (1, "f32", [1.0]),
                                              (2, "f32", [1.3, 0.6]),
                                              (3, "bf16", [0.6, 1.0, 2.0])])
def test_sampler_single_launch_matches_chain_and_oracle(hv, orc, cuda, rows, dtype, temps):
    """The single-launch row sampler (a few rows, reference mode: the draft step's
    softmax(logits / T) and token, model_runner.py:312-313) writes the same
    probabilities, tokens and row statistics as the launch chain, bit for bit, and
    both equal the C oracle; the probabilities go to a strided view as the draft
    phase writes them (draft_probs[:, j] of [rows, gamma, V]). Uniforms include
    the range ends."""
    V = 151936
    rng = np.random.default_rng(100 + rows)
    logits = rng.standard_normal((rows, V), dtype=np.float32) * 2
    if dtype == "bf16":
        bits = hv.synthetic.f32_to_bf16_bits(logits)
        logits = (bits.astype(np.uint32) << 16).view(np.float32)
        lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        lg = torch.from_numpy(logits).to(cuda)
    T = np.array(temps, np.float32)
    for u_case in ("random", "ends"):
        u = rng.random(rows, dtype=np.float32) if u_case == "random" else \
            np.array([0.0, np.float32(1.0) - np.float32(2 ** -24), 0.5][:rows], np.float32)
        ref = orc.sampler(logits, T, np.zeros(rows, np.int32), np.ones(rows, np.float32),
                          mode="reference", uniforms=u)
        got = []
        for chain in (False, True):
            big = torch.full((rows, 3, V), float("nan"), device=cuda)
            tok = torch.full((rows,), -7, dtype=torch.int64, device=cuda)
            print(f"sampler rows={rows} {dtype} u={u_case} chain={chain}", flush=True)
            r = hv.ops.sample_rows(lg, torch.from_numpy(T).to(cuda), mode="reference",
                                   uniforms=torch.from_numpy(u).to(cuda), probs_out=big[:, 1],
                                   tokens_out=tok, row_stats=True, chain_only=chain)
            torch.cuda.synchronize()
            assert torch.isnan(big[:, 0]).all() and torch.isnan(big[:, 2]).all()
            got.append((big[:, 1].cpu().numpy(), tok.cpu().numpy(),
                        r["row_stats"].cpu().numpy()))
        for probs, toks, stats in got:
            np.testing.assert_array_equal(toks, ref["tokens"])
            np.testing.assert_array_equal(stats, ref["row_stats"])
            np.testing.assert_array_equal(probs, ref["probs"])
    assert not hv.ops.accept_error(cuda)
