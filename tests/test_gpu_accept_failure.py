"""Failure path of the single-launch acceptance's bounded waits.

The single-launch kernels (k_accept_small, k_accept_small_topk) exchange data
between workgroups through tagged words and wait for them with a bounded
number of polls. The budget is set from the host (ops.accept_wait_budget, the
workspace word at byte 12): with a budget of 0 a workgroup gives up at its
first poll that finds the data missing, so the failure path runs while every
kernel still exits normally. Each call must then return within milliseconds,
every sequence must be either equal to the C oracle (model_runner.py:387-428)
or marked invalid (num_accepted -1, out_len 0) with the sticky error word set,
and the next call on the same workspace with the default budget must be
correct.
"""
import time

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(hv, kind):
    if kind.startswith("reference"):
        B = int(kind.split("-b")[1])
        w = hv.synthetic.accept_workload(B, 3, seed=300 + B, dtype="bf16", temperature=0.6)
        return w, "reference", False
    B = int(kind.split("-b")[1])
    w = hv.synthetic.accept_workload(B, 3, seed=400 + B, top_k=50, top_p=0.9, mode="filtered")
    return w, "filtered", True


def _call(hv, w, mode, topk, cuda):
    if w["dtype"] == "bf16":
        lg = torch.from_numpy(w["logits_bits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        lg = torch.from_numpy(w["logits"]).to(cuda)
    t = {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(cuda)
         for k in ["draft_probs", "draft_tokens", "temperatures", "top_ks", "top_ps",
                   "u_accept", "u_resample"]}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nacc, out, olen = hv.ops.spec_accept(lg, t["draft_probs"], t["draft_tokens"],
                                         t["temperatures"], t["u_accept"], t["u_resample"],
                                         mode=mode, top_ks=t["top_ks"], top_ps=t["top_ps"],
                                         topk_le64=topk)
    torch.cuda.synchronize()
    return nacc.cpu().numpy(), out.cpu().numpy(), olen.cpu().numpy(), time.perf_counter() - t0


@pytest.mark.parametrize("kind", ["reference-b1", "reference-b3", "topk-b1", "topk-b2"])
def test_zero_wait_budget(hv, orc, cuda, kind):
    ops = hv.ops
    w, mode, topk = _inputs(hv, kind)
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode=mode, top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    B = w["draft_tokens"].shape[0]
    _call(hv, w, mode, topk, cuda)  # the workspace exists, with the default budget
    ops.accept_error(cuda, clear=True)
    print(f"zero wait budget {kind}", flush=True)
    ops.accept_wait_budget(cuda, 0)
    invalid = 0
    try:
        for rep in range(4):
            nacc, out, olen, dt = _call(hv, w, mode, topk, cuda)
            assert dt < 0.25, dt  # every wait gave up at once
            for b in range(B):
                if nacc[b] < 0:
                    invalid += 1
                    assert olen[b] == 0
                else:
                    assert nacc[b] == ref["num_accepted"][b]
                    assert olen[b] == ref["out_len"][b]
                    np.testing.assert_array_equal(out[b], ref["out_tokens"][b])
        err = ops.accept_error(cuda)
        if invalid:
            assert err  # marked outputs come with the sticky error word
    finally:
        ops.accept_wait_budget(cuda, None)
    print(f"invalid sequences over 4 calls: {invalid} of {4 * B}", flush=True)
    ops.accept_error(cuda, clear=True)
    # the default budget again: correct on the same workspace
    nacc, out, olen, _ = _call(hv, w, mode, topk, cuda)
    np.testing.assert_array_equal(nacc, ref["num_accepted"])
    np.testing.assert_array_equal(out, ref["out_tokens"])
    np.testing.assert_array_equal(olen, ref["out_len"])
    assert not ops.accept_error(cuda)


def test_sampler_zero_wait_budget(hv, orc, cuda):
    """The single-launch row sampler under a zero wait budget: each row's token is
    the oracle's or -1 (with the sticky error word set), each call returns at
    once, and the default budget afterwards gives the oracle's tokens."""
    ops = hv.ops
    V, rows = 151936, 3
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((rows, V), dtype=np.float32) * 2
    T = np.array([0.6, 1.0, 0.8], np.float32)
    u = rng.random(rows, dtype=np.float32)
    ref = orc.sampler(logits, T, np.zeros(rows, np.int32), np.ones(rows, np.float32),
                      mode="reference", uniforms=u)
    lg = torch.from_numpy(logits).to(cuda)
    Tt, ut = torch.from_numpy(T).to(cuda), torch.from_numpy(u).to(cuda)

    def call():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = ops.sample_rows(lg, Tt, mode="reference", uniforms=ut, want_probs=True)
        toks = r["tokens"].cpu().numpy()
        return toks, time.perf_counter() - t0

    call()
    ops.accept_error(cuda, clear=True)
    print("sampler zero wait budget", flush=True)
    ops.accept_wait_budget(cuda, 0, kind="sampler")
    invalid = 0
    try:
        for _ in range(4):
            toks, dt = call()
            assert dt < 0.25, dt
            for b in range(rows):
                if toks[b] < 0:
                    invalid += 1
                else:
                    assert toks[b] == ref["tokens"][b]
        if invalid:
            assert ops.accept_error(cuda)
    finally:
        ops.accept_wait_budget(cuda, None, kind="sampler")
    ops.accept_error(cuda, clear=True)
    toks, _ = call()
    np.testing.assert_array_equal(toks, ref["tokens"])
    assert not ops.accept_error(cuda)
