"""Pins the CPU oracle of the acceptance sampler (runs without a GPU).

Checks come from outside the oracle's own formulas:
  * the reference's known-answer tests, tests/test_sampler.py:6-44;
  * textbook facts (exp accuracy against float64, exact fixed-point values,
    round-to-nearest-even of integers computed with Python integers);
  * the speculative-sampling theorem: for any draft distribution the emitted
    token is distributed as the target distribution (integrated over the
    uniforms on a grid);
  * special cases that fix the outcome: q == p always accepts, p_t == 0
    always rejects, an all-zero residual falls back to P[r];
  * an independent torch restatement of Sampler._apply_top_k/_apply_top_p
    (sort + softmax + cumsum) on random rows.
"""
import math

import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- number formats
def test_exp_accuracy_and_special_values(orc):
    ys = np.concatenate([np.linspace(-86.0, 0.0, 20001, dtype=np.float32),
                         -np.logspace(-8, 1.9, 2000).astype(np.float32)])
    got = np.array([orc.exp_f32(float(y)) for y in ys], dtype=np.float64)
    ref = np.exp(ys.astype(np.float64))
    rel = np.abs(got - ref) / ref
    assert rel.max() < 2.5e-7, rel.max()
    assert orc.exp_f32(0.0) == 1.0
    assert orc.exp_f32(-86.5) == 0.0
    assert orc.exp_f32(float("nan")) == 0.0
    assert orc.exp_f32(float("-inf")) == 0.0
    # smallest kept value is a normal float
    assert orc.exp_f32(-86.0) > np.finfo(np.float32).tiny


def test_fixed_point_closed_forms(orc):
    assert orc.fx44(1.0) == 1 << 44
    assert orc.fx44(0.5) == 1 << 43
    assert orc.fx44(2.0 ** -44) == 1
    assert orc.fx44(2.0 ** -45) == 0
    assert orc.fx44(3 * 2.0 ** -44) == 3
    assert orc.fx44(0.0) == 0 and orc.fx44(-1.0) == 0
    x = np.float32(0.3)
    assert orc.fx44(float(x)) == math.floor(float(x) * 2 ** 44)


def _rne_u64_to_f32(n: int) -> float:
    if n == 0:
        return 0.0
    sh = max(n.bit_length() - 24, 0)
    m, rem = n >> sh, n & ((1 << sh) - 1)
    half = 1 << (sh - 1) if sh else 0
    if sh and (rem > half or (rem == half and m & 1)):
        m += 1
    return float(m << sh)


@pytest.mark.parametrize("n", [1, 2 ** 24 - 1, 2 ** 24, 2 ** 24 + 1, 2 ** 24 + 2, 2 ** 24 + 3,
                               2 ** 25 + 2, 2 ** 25 + 6, 2 ** 44 + 2 ** 20, (1 << 62) - 1,
                               123456789012345, 98765432109876543])
def test_u64_to_f32_round_to_nearest_even(orc, n):
    assert orc.f32_of_u64(n) == _rne_u64_to_f32(n)


def test_order_key_is_monotone(orc):
    vals = np.array([-np.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.0, 7.25, np.inf], np.float32)
    keys = [orc.key_f32(float(v)) for v in vals]
    assert keys == sorted(keys)
    assert orc.key_f32(-0.0) == orc.key_f32(0.0)


# ---------------------------------------------------- reference KATs (sampler.py)
def test_kat_top_k_masks_lower_ranked_logits(orc):
    # tests/test_sampler.py:6-18
    keep, n, _, _ = orc.filter_keep(np.array([5.0, 4.0, 3.0, 2.0], np.float32), top_k=2)
    assert keep.tolist() == [True, True, False, False] and n == 2


def test_kat_top_p_masks_tail_outside_probability_mass(orc):
    # tests/test_sampler.py:21-31
    logits = torch.log(torch.tensor([0.5, 0.3, 0.15, 0.05], dtype=torch.float32)).numpy()
    keep, _, _, _ = orc.filter_keep(logits, top_p=0.81)
    assert keep.tolist() == [True, True, False, False]


def test_kat_top_p_uses_strict_boundary(orc):
    # tests/test_sampler.py:34-44
    logits = torch.log(torch.tensor([0.5, 0.3, 0.15, 0.05], dtype=torch.float32)).numpy()
    keep, _, _, _ = orc.filter_keep(logits, top_p=0.8)
    assert keep.tolist() == [True, False, False, False]


def test_masked_logits_survive_unchanged(orc):
    # masked_fill keeps the surviving logits bit-for-bit (sampler.py:36,48)
    x = np.array([1.5, -2.0, 3.25, 0.5, 3.25], np.float32)
    keep, n, _, _ = orc.filter_keep(x, top_k=2)
    # tie at 3.25: lower index first
    assert keep.tolist() == [False, False, True, False, True] and n == 2
    keep, n, _, _ = orc.filter_keep(x, top_k=1)
    assert keep.tolist() == [False, False, True, False, False]


def _torch_filter(x: torch.Tensor, k: int, p: float) -> np.ndarray:
    """Independent restatement of Sampler._apply_top_k/_apply_top_p in torch
    (descending sort, softmax, cumsum, strict <, keep rank 0)."""
    V = x.shape[-1]
    x = x.clone().unsqueeze(0)
    if 0 < k < V:
        s, idx = torch.sort(x, dim=-1, descending=True, stable=True)
        keep_s = torch.arange(V).unsqueeze(0) < k
        s = s.masked_fill(~keep_s, float("-inf"))
        x = torch.empty_like(x).scatter(1, idx, s)
    if p < 1.0:
        s, idx = torch.sort(x, dim=-1, descending=True, stable=True)
        cp = torch.cumsum(torch.softmax(s, dim=-1), dim=-1)
        keep_s = cp < p
        keep_s[:, 0] = True
        s = s.masked_fill(~keep_s, float("-inf"))
        x = torch.empty_like(x).scatter(1, idx, s)
    return torch.isfinite(x[0]).numpy()


@pytest.mark.parametrize("seed,k,p,T", [(1, 50, 1.0, 1.0), (2, 0, 0.9, 1.0), (3, 20, 0.8, 0.7),
                                        (4, 0, 0.5, 1.3), (5, 1000, 0.95, 0.9)])
def test_filter_matches_torch_restatement(orc, seed, k, p, T):
    rng = np.random.default_rng(seed)
    V = 20000
    logits = (rng.standard_normal(V) * 2).astype(np.float32)
    keep, n, M, S = orc.filter_keep(logits, temperature=T, top_k=k, top_p=p)
    x = torch.from_numpy(logits) / T
    ref = _torch_filter(x, k, p)
    diff = np.nonzero(keep != ref)[0]
    if diff.size:
        # only a boundary element whose cumulative mass is within 1e-6 of p may differ
        s, idx = torch.sort(x, descending=True, stable=True)
        if 0 < k < V:
            s = s[:k]
            idx = idx[:k]
        cp = torch.cumsum(torch.softmax(s.double(), 0), 0).numpy()
        pos = {int(i): r for r, i in enumerate(idx.tolist())}
        for d in diff:
            assert abs(cp[pos[int(d)]] - p) < 1e-6, (d, cp[pos[int(d)]])
    assert abs(int(keep.sum()) - int(ref.sum())) <= 1


# ----------------------------------------------------------- acceptance oracle
def _tiny_case(V=6, gamma=1, seed=0):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((1, gamma + 1, V)) * 1.5).astype(np.float32)
    dlog = logits[:, :gamma] + rng.standard_normal((1, gamma, V)).astype(np.float32)
    q = np.exp(dlog - dlog.max(-1, keepdims=True))
    q = (q / q.sum(-1, keepdims=True)).astype(np.float32)
    return logits, q


def test_law_of_emitted_token_equals_target(orc):
    """Speculative sampling theorem: P(first emitted token = i) == P0[i]."""
    V, G = 6, 512
    logits, q = _tiny_case(V)
    P0 = orc.sampler(logits[0, :1])["probs"][0].astype(np.float64)
    for d in range(V):
        B = G * G
        ua = ((np.arange(G) + 0.5) / G).astype(np.float32)
        ur = ((np.arange(G) + 0.5) / G).astype(np.float32)
        UA, UR = np.meshgrid(ua, ur, indexing="ij")
        res = orc.spec_accept(np.broadcast_to(logits, (B, 2, V)), np.broadcast_to(q, (B, 1, V)),
                              np.full((B, 1), d, np.int64), np.ones(B, np.float32),
                              UA.reshape(B, 1), UR.reshape(B), mode="reference")
        first = res["out_tokens"][:, 0]
        law = np.bincount(first, minlength=V) / B
        # the draft token d was proposed; mix over the draft law q[d]
        if d == 0:
            total = np.zeros(V)
        total += q[0, 0, d] * law
    assert np.abs(total - P0).max() < 4e-3, (total, P0)


def test_equal_distributions_always_accept(orc):
    V, gamma = 300, 3
    rng = np.random.default_rng(7)
    logits = (rng.standard_normal((1, gamma + 1, V)) * 2).astype(np.float32)
    P = orc.sampler(logits[0])["probs"]
    q = P[None, :gamma].copy()
    dtok = rng.integers(0, V, size=(1, gamma))
    res = orc.spec_accept(logits, q, dtok, np.ones(1), np.full((1, gamma), 0.999999, np.float32),
                          np.array([0.3], np.float32))
    assert res["num_accepted"][0] == gamma and res["out_len"][0] == gamma + 1
    assert res["out_tokens"][0, :gamma].tolist() == dtok[0].tolist()


def test_zero_target_mass_always_rejects(orc):
    V, gamma = 300, 2
    rng = np.random.default_rng(8)
    logits = (rng.standard_normal((1, gamma + 1, V)) * 2).astype(np.float32)
    logits[0, 0, 17] = -np.inf
    q = np.full((1, gamma, V), 1.0 / V, np.float32)
    res = orc.spec_accept(logits, q, np.array([[17, 3]]), np.ones(1),
                          np.zeros((1, gamma), np.float32), np.array([0.5], np.float32))
    assert res["num_accepted"][0] == 0
    assert res["out_tokens"][0, 0] != 17 and res["out_tokens"][0, 1] == -1


def test_empty_residual_falls_back_to_target(orc):
    V, gamma = 257, 1
    rng = np.random.default_rng(9)
    logits = (rng.standard_normal((1, 2, V)) * 2).astype(np.float32)
    P = orc.sampler(logits[0])["probs"]
    q = P[None, :1].copy()  # Q == P: residual is all zero
    u = np.float32(0.61)
    res = orc.spec_accept(logits, q, np.array([[5]]), np.ones(1), np.array([[1.0]], np.float32),
                          np.array([u]))
    assert res["num_accepted"][0] == 0
    w = np.array([orc.fx44(float(v)) for v in P[0]], dtype=object)
    W = int(sum(w))
    t = (min(int(u * 2 ** 24), 2 ** 24 - 1) * W) >> 24
    c = np.cumsum(w)
    expect = int(np.nonzero(c > t)[0][0])
    assert res["out_tokens"][0, 0] == expect


def test_bonus_draw_is_inverse_cdf(orc):
    V = 5000
    rng = np.random.default_rng(10)
    logits = (rng.standard_normal((1, V)) * 2).astype(np.float32)
    for u in [0.0, 1e-7, 0.25, 0.5, 0.999, 0.99999994]:
        r = orc.sampler(logits, uniforms=np.array([u], np.float32))
        w = [orc.fx44(float(v)) for v in r["probs"][0]]
        W = sum(w)
        t = (min(int(np.float32(u) * np.float32(2 ** 24)), 2 ** 24 - 1) * W) >> 24
        expect = int(np.searchsorted(np.cumsum(np.array(w, dtype=np.float64)), t, side="right"))
        # exact check with python ints
        acc = 0
        for i, wi in enumerate(w):
            acc += wi
            if acc > t:
                exact = i
                break
        assert r["tokens"][0] == exact
        assert abs(expect - exact) <= 1


def test_greedy_is_first_argmax(orc):
    rng = np.random.default_rng(11)
    V, gamma = 1000, 3
    logits = rng.integers(-3, 3, size=(2, gamma + 1, V)).astype(np.float32)  # many ties
    am = logits.argmax(-1)
    dtok = am[:, :gamma].copy()
    dtok[1, 1] += 1
    res = orc.spec_accept(logits, None, dtok, None, None, None, mode="greedy")
    assert res["num_accepted"].tolist() == [gamma, 1]
    assert res["out_tokens"][0].tolist() == am[0].tolist()
    assert res["out_tokens"][1].tolist() == [am[1, 0], am[1, 1], -1, -1]


def test_reference_probs_match_torch_softmax(orc):
    rng = np.random.default_rng(12)
    V = 151936
    logits = (rng.standard_normal((3, V)) * 2).astype(np.float32)
    T = np.array([1.0, 0.6, 1.3], np.float32)
    got = orc.sampler(logits, temperatures=T)["probs"]
    ref = torch.softmax(torch.from_numpy(logits) / torch.from_numpy(T)[:, None], -1).numpy()
    rel = np.abs(got - ref) / np.maximum(ref, 1e-30)
    big = ref > 1e-30
    assert rel[big].max() < 1e-5
