"""GPU parity of the single-launch filtered acceptance (every top-k in [1, 64]).

hs_spec_accept with HS_ACCEPT_TOPK_LE64 runs small filtered batches as one
launch (k_accept_small_topk): chunk maxima give a threshold under each row's
top-k, the chunks publish their candidates, and workgroup 0 sorts them, cuts
top-k and top-p and draws over the kept set. Accept counts, emitted tokens
and row statistics must equal the C oracle bit for bit, as for the chain.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

V = 151936


def _dev(w, cuda):
    if w["dtype"] == "bf16":
        lg = torch.from_numpy(w["logits_bits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        lg = torch.from_numpy(w["logits"]).to(cuda)
    t = {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(cuda)
         for k in ["draft_probs", "draft_tokens", "temperatures", "top_ks", "top_ps",
                   "u_accept", "u_resample"]}
    return lg, t


def _check(hv, orc, w, cuda, expect_valid=True):
    lg, t = _dev(w, cuda)
    nacc, out, olen, stats = hv.ops.spec_accept(
        lg, t["draft_probs"], t["draft_tokens"], t["temperatures"], t["u_accept"],
        t["u_resample"], mode="filtered", top_ks=t["top_ks"], top_ps=t["top_ps"],
        row_stats=True, topk_le64=True)
    torch.cuda.synchronize()
    got = nacc.cpu().numpy(), out.cpu().numpy(), olen.cpu().numpy(), stats.cpu().numpy()
    if not expect_valid:
        return got
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode="filtered", top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    np.testing.assert_array_equal(got[0], ref["num_accepted"])
    np.testing.assert_array_equal(got[1], ref["out_tokens"])
    np.testing.assert_array_equal(got[2], ref["out_len"])
    np.testing.assert_array_equal(got[3], ref["row_stats"])
    return ref


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 5, 8])
def test_config0_single_launch(hv, orc, cuda, seed):
    """Config 0: B = 1, gamma = 3, f32 logits, T = 1, top-k 50, top-p 0.9."""
    print(f"config0 top-k single launch seed={seed}", flush=True)
    w = hv.synthetic.accept_workload(1, 3, seed=seed, top_k=50, top_p=0.9, mode="filtered")
    _check(hv, orc, w, cuda)


@pytest.mark.parametrize("B,g,dtype,k,p,T", [
    (1, 1, "f32", 1, 1.0, 1.0), (1, 3, "bf16", 50, 0.9, 0.8), (1, 7, "f32", 64, 0.5, 1.3),
    (2, 5, "bf16", 20, 0.8, 0.6), (3, 3, "f32", 64, 1.0, 1.0), (3, 2, "bf16", 7, 0.95, 1.1)])
def test_every_reject_position(hv, orc, cuda, B, g, dtype, k, p, T):
    """Drafts at each target row's argmax (always kept), acceptance uniforms that
    force the first reject at every position 0..gamma in turn (u = 0 accepts a
    kept draft, u = 1 rejects), so residual and bonus draws both run."""
    base = hv.synthetic.accept_workload(B, g, seed=600 + 10 * B + g, dtype=dtype,
                                        temperature=T, top_k=k, top_p=p, mode="filtered")
    am = base["logits"].argmax(-1)
    base["draft_tokens"] = np.ascontiguousarray(am[:, :g]).astype(np.int64)
    for r in range(g + 1):
        w = dict(base)
        u = np.zeros((B, g), np.float32)
        if r < g:
            u[:, r] = 1.0
        w["u_accept"] = u
        w["u_resample"] = ((np.arange(B, dtype=np.float32) + 0.5 + r) / (B + g + 1)).astype(
            np.float32)
        print(f"top-k single launch B={B} gamma={g} {dtype} k={k} p={p} reject at {r}",
              flush=True)
        ref = _check(hv, orc, w, cuda)
        assert (ref["num_accepted"] == r).all()


def test_crowded_chunk_and_tied_rows(hv, orc, cuda):
    """Row 0: every value of one chunk above the rest (that chunk has 2048
    candidates: the workgroup sorts them in LDS and publishes its 64 largest).
    Row 1: all logits equal (ties broken by index: every chunk before the k-th
    overflows, and workgroup 0 merges ~3000 candidates 192 at a time). Row 2:
    bf16-style ties at a few values. Row 3: a plain row."""
    g = 3
    w = hv.synthetic.accept_workload(1, g, seed=77, top_k=50, top_p=0.9, mode="filtered")
    x = w["logits"]
    rng = np.random.default_rng(78)
    x[0, 0] = rng.standard_normal(V).astype(np.float32)
    x[0, 0, 5 * 2048:6 * 2048] = 10.0 + np.arange(2048, dtype=np.float32) / 1024
    x[0, 1] = 0.0
    x[0, 2] = rng.integers(-3, 4, size=V).astype(np.float32)
    w["logits"] = np.ascontiguousarray(x)
    for r in range(g + 1):
        u = np.zeros((1, g), np.float32)
        if r < g:
            u[:, r] = 1.0
        w2 = dict(w)
        w2["u_accept"] = u
        w2["draft_tokens"] = np.array([[5 * 2048 + 2047, 3, int(x[0, 2].argmax())]], np.int64)
        print(f"crowded/tied rows reject at {r}", flush=True)
        ref = _check(hv, orc, w2, cuda)
        assert int(ref["num_accepted"][0]) == r


def test_broken_promise_marks_outputs_invalid(hv, orc, cuda):
    """A sequence with top-k 0 (off) or 65 under HS_ACCEPT_TOPK_LE64 gets
    num_accepted -1 and out_len 0; the others of the batch are unaffected, and the
    next call on the same workspace is correct."""
    w = hv.synthetic.accept_workload(3, 3, seed=90, top_k=50, top_p=0.9, mode="filtered")
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode="filtered", top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    w["top_ks"] = np.array([50, 0, 65], np.int32)
    nacc, out, olen, _ = _check(hv, orc, w, cuda, expect_valid=False)
    assert nacc.tolist()[1:] == [-1, -1] and olen.tolist()[1:] == [0, 0]
    assert int(nacc[0]) == int(ref["num_accepted"][0])
    np.testing.assert_array_equal(out[0], ref["out_tokens"][0])
    assert (out[1:] == -1).all()
    w = hv.synthetic.accept_workload(1, 3, seed=91, top_k=30, top_p=0.8, mode="filtered")
    _check(hv, orc, w, cuda)
    assert not hv.ops.accept_error(cuda)


def test_shared_workspace_across_paths(hv, orc, cuda):
    """Reference single launch, top-k single launch, the filtered chain (per-sequence
    settings, top-k 0 present) and the top-k launch again, on one workspace."""
    calls = [
        ("reference", hv.synthetic.accept_workload(1, 3, seed=95, dtype="bf16")),
        ("topk", hv.synthetic.accept_workload(2, 4, seed=96, top_k=40, top_p=0.9,
                                              mode="filtered")),
        ("chain", hv.synthetic.accept_workload(4, 3, seed=97, dtype="bf16",
                                               per_seq_settings=True, mode="filtered")),
        ("topk", hv.synthetic.accept_workload(1, 3, seed=98, dtype="bf16", top_k=64, top_p=1.0,
                                              mode="filtered")),
    ]
    for kind, w in calls:
        print(f"shared workspace: {kind}", flush=True)
        if kind == "topk":
            _check(hv, orc, w, cuda)
            continue
        lg, t = _dev(w, cuda)
        mode = "reference" if kind == "reference" else "filtered"
        nacc, out, olen = hv.ops.spec_accept(lg, t["draft_probs"], t["draft_tokens"],
                                             t["temperatures"], t["u_accept"], t["u_resample"],
                                             mode=mode, top_ks=t["top_ks"], top_ps=t["top_ps"])
        ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"],
                              w["temperatures"], w["u_accept"], w["u_resample"], mode=mode,
                              top_ks=w["top_ks"], top_ps=w["top_ps"])
        np.testing.assert_array_equal(nacc.cpu().numpy(), ref["num_accepted"])
        np.testing.assert_array_equal(out.cpu().numpy(), ref["out_tokens"])
    assert not hv.ops.accept_error(cuda)
