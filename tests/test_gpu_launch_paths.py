"""Cross-checks between the launch paths of hs_spec_accept, and every branch of
the filter chain against the CPU oracle (mini_vllm/layers/sampler.py:27-49,
mini_vllm/engine/model_runner.py:391-428).

Small batches run as one launch (k_accept_small in reference mode,
k_accept_small_topk in filtered mode with top-k <= 64); chain_only=True forces
the launch chain on the same inputs, and both must give the same bits."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

V = 151936


def _dev(w, cuda, keys):
    return {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(cuda) for k in keys}


def _logits(w, cuda):
    if w["dtype"] == "bf16":
        return torch.from_numpy(w["logits_bits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    return torch.from_numpy(w["logits"]).to(cuda)


@pytest.mark.parametrize("B,gamma,dtype,mode", [
    (1, 3, "bf16", "reference"), (2, 5, "bf16", "reference"), (3, 7, "f32", "reference"),
    (1, 1, "f32", "reference"), (1, 3, "f32", "filtered"), (2, 3, "bf16", "filtered")])
def test_single_launch_matches_chain(hv, orc, cuda, B, gamma, dtype, mode):
    print(f"single launch vs chain B={B} gamma={gamma} {dtype} {mode}", flush=True)
    kw = dict(temperature=1.0, top_k=50, top_p=0.9) if mode == "filtered" else dict(
        temperature=0.6)
    w = hv.synthetic.accept_workload(B, gamma, seed=3300 + 10 * B + gamma, dtype=dtype,
                                     mode=mode, **kw)
    lg = _logits(w, cuda)
    t = _dev(w, cuda, ["draft_probs", "draft_tokens", "temperatures", "u_accept",
                       "u_resample", "top_ks", "top_ps"])
    got = []
    for chain in (False, True):
        r = hv.ops.spec_accept(lg, t["draft_probs"], t["draft_tokens"], t["temperatures"],
                               t["u_accept"], t["u_resample"], mode=mode, top_ks=t["top_ks"],
                               top_ps=t["top_ps"], row_stats=True,
                               topk_le64=(mode == "filtered"), chain_only=chain)
        got.append([x.cpu().numpy() for x in r])
    hv.ops.check_accepted(torch.from_numpy(got[0][0]))
    for a, b in zip(*got):
        np.testing.assert_array_equal(a, b)
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode=mode, top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    np.testing.assert_array_equal(got[0][0], ref["num_accepted"])
    np.testing.assert_array_equal(got[0][1], ref["out_tokens"])


def _plateau_row(rng, n_plat, values):
    """A row whose top-p 0.9 crossing lies in a plateau of n_plat bf16 values just
    below one spike (the coarse boundary bucket then holds about n_plat elements)."""
    x = (rng.standard_normal(V) - 12.0).astype(np.float32)
    pos = rng.choice(V, size=n_plat + 1, replace=False)
    x[pos[0]] = 10.0
    x[pos[1:]] = rng.choice(np.asarray(values, np.float32), size=n_plat)
    return x


def _filter_rows(hv, rng):
    """Rows covering every branch of the filter chain in one call: ordinary
    top-p / top-k / both / neither rows, boundary buckets of ~1000 and ~10000
    elements (listed whole, refined into fine sub-buckets, fine bucket listed by
    the third pass), top-k above the chunk count (radix path), rows with -inf
    entries, rows of one repeated value (ties everywhere), nearly flat rows and
    top-p near its limits."""
    rows, T, K, P = [], [], [], []

    def add(x, t, k, p):
        rows.append(np.asarray(x, np.float32))
        T.append(t)
        K.append(k)
        P.append(p)

    for i in range(10):
        base = rng.standard_normal(V).astype(np.float32) * 2.0
        add(base, 0.6 + 0.06 * i, 0, 0.9)
        add(base, 1.0, [20, 50, 64, 5, 1][i % 5], 1.0)
        add(base, 0.8, 50, 0.8)
    add(rng.standard_normal(V) * 2.0, 1.0, 0, 1.0)
    add(rng.standard_normal(V) * 2.0, 0.7, 200, 0.9)
    add(rng.standard_normal(V) * 2.0, 1.1, 1000, 1.0)
    add(_plateau_row(rng, 1000, [9.0, 8.9375]), 1.0, 0, 0.9)
    add(_plateau_row(rng, 10000, [9.0, 8.9375]), 1.0, 0, 0.9)
    add(_plateau_row(rng, 10000, [8.9375]), 1.0, 0, 0.9)
    add(_plateau_row(rng, 3000, [8.9375, 8.875]), 0.9, 0, 0.9)
    x = np.where(rng.random(V) < 0.5, -np.inf, rng.standard_normal(V) * 3)
    add(x, 1.0, 0, 0.95)
    add(x, 1.0, 30, 1.0)
    add(np.full(V, 0.5), 1.0, 0, 0.5)
    add(np.full(V, 0.5), 1.0, 40, 1.0)
    add(rng.standard_normal(V) * 0.01, 1.0, 0, 0.9)
    # top-p near its limits: p close to 1 (wide boundary region), a peaked row
    # (boundary at the top bucket), logits spread far beyond the skipped
    # buckets, a maximum far from 0, a nearly flat row at p = 0.99
    add(rng.standard_normal(V) * 2.0, 0.6, 0, 0.999)
    add(rng.standard_normal(V) * 8.0, 1.0, 0, 0.5)
    add(rng.standard_normal(V) * 6.0, 1.0, 0, 0.95)
    add(rng.standard_normal(V) * 2.0 + 300000.0, 1.0, 0, 0.9)
    add(rng.standard_normal(V) * 0.01, 1.0, 0, 0.99)
    bits = hv.synthetic.f32_to_bf16_bits(np.stack(rows))
    return (bits, hv.synthetic.bf16_bits_to_f32(bits), np.array(T, np.float32),
            np.array(K, np.int32), np.array(P, np.float32))


def test_filter_chain_every_branch_vs_oracle(hv, orc, cuda):
    rng = np.random.default_rng(515)
    bits, xf, T, K, P = _filter_rows(hv, rng)
    R = bits.shape[0]
    u = rng.random(R).astype(np.float32)
    lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    args = [torch.from_numpy(a).to(cuda) for a in (T, K, P)]
    print(f"filter chain branches rows={R}", flush=True)
    r = hv.ops.sample_rows(lg, *args, mode="filtered", uniforms=torch.from_numpy(u).to(cuda),
                           want_probs=True, row_stats=True)
    m = hv.ops.sample_rows(lg, *args, mode="filtered", want_probs=True, out_kind=1)
    ref = orc.sampler(xf, T, K, P, mode="filtered", uniforms=u)
    probs = r["probs"].cpu().numpy()
    np.testing.assert_array_equal(probs, ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])
    # masked logits: x / T inside the kept set, -inf outside (sampler.py:36-37,48-49)
    masked = m["probs"].cpu().numpy()
    kept = np.isfinite(masked)
    np.testing.assert_array_equal(kept, probs > 0)
    xs = (xf / T[:, None]).astype(np.float32)
    np.testing.assert_array_equal(masked[kept], xs[kept])


@pytest.mark.parametrize("mode", ["reference", "filtered"])
def test_wave_and_scalar_chains_agree(hv, orc, cuda, mode):
    """B = 64, gamma = 3, per-sequence settings: the chain's wave-per-chunk kernels
    (aligned rows) and its workgroup-per-chunk kernels (draft probabilities at an odd
    row stride, so no row is 16-byte aligned) give the same bits, and the oracle's
    decisions."""
    B, gamma = 64, 3
    print(f"wave vs scalar chain B={B} gamma={gamma} {mode}", flush=True)
    w = hv.synthetic.accept_workload(B, gamma, seed=4242, dtype="bf16", mode=mode,
                                     per_seq_settings=True)
    lg = _logits(w, cuda)
    t = _dev(w, cuda, ["draft_probs", "draft_tokens", "temperatures", "u_accept",
                       "u_resample", "top_ks", "top_ps"])
    padded = torch.zeros((B * gamma, V + 1), dtype=torch.float32, device=cuda)
    padded[:, :V] = t["draft_probs"].reshape(B * gamma, V)
    q_odd = padded[:, :V].reshape(B, gamma, V)
    assert q_odd.stride(1) == V + 1
    got = []
    for q in (t["draft_probs"], q_odd):
        r = hv.ops.spec_accept(lg, q, t["draft_tokens"], t["temperatures"], t["u_accept"],
                               t["u_resample"], mode=mode, top_ks=t["top_ks"],
                               top_ps=t["top_ps"], row_stats=True)
        got.append([x.cpu().numpy() for x in r])
    for a, b in zip(*got):
        np.testing.assert_array_equal(a, b)
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode=mode, top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    np.testing.assert_array_equal(got[0][0], ref["num_accepted"])
    np.testing.assert_array_equal(got[0][1], ref["out_tokens"])


def _edge_targets(hv, rng, B, gamma):
    """Target logit patterns [B, gamma+1, V] (bf16) whose numerators leave the
    range [2^-96, 2^60] in which x / T is taken as a corrected product: exact
    zeros of both signs, tiny normals and subnormals, the range ends and their
    neighbours, huge values, -inf entries; spread over a whole row or confined
    to one chunk (so that fast and fallback chunks meet in one row), including
    the row's last, partial chunk."""
    f = hv.synthetic.f32_to_bf16_bits
    tb = f((rng.standard_normal((B, gamma + 1, V)) * 2.0).astype(np.float32))

    def put(b, j, idx, vals):
        tb[b, j, idx] = np.asarray(vals, np.uint16)

    spread = lambda n: rng.choice(V, size=n, replace=False)
    in_chunk = lambda c, n: c * 2048 + rng.choice(min(2048, V - c * 2048), size=n, replace=False)
    put(0, 0, spread(400), [0x0000] * 200 + [0x8000] * 200)
    put(1, 1, spread(150), f(np.r_[np.full(50, 1e-35), np.full(50, -1e-35),
                                  np.full(25, 1e-40), np.full(25, -1e-40)].astype(np.float32)))
    put(2, 2, in_chunk(10, 8), [0x0F80, 0x8F80, 0x0F7F, 0x8F7F, 0x5D80, 0xDD80, 0x5D81, 0xDD81])
    put(3, 0, in_chunk(74, 6), f(np.array([-1e25, -3e19, 0.0, -0.0, 1e-38, -np.inf],
                                          np.float32)))
    put(4, 3, spread(V // 2), [0xFF80] * (V // 2))  # -inf
    put(5, 1, in_chunk(0, 4), [0x0000, 0x0001, 0x8001, 0x4780])  # 0, +-min subnormal, 2^16
    put(6, 0, in_chunk(40, 3), f(np.array([1e30, -1e30, 0.0], np.float32)))
    return tb


@pytest.mark.parametrize("mode", ["reference", "filtered"])
def test_temperature_division_range_edges(hv, orc, cuda, mode):
    """x / T where the numerators leave the corrected product's exact range:
    the chain (row statistics, partial sums, final search), the single launch
    and the row sampler agree with the oracle bit for bit. Temperatures include
    1 (no division), 2^-12 and 2^21 (outside the corrected product's divisor
    range) and ordinary values."""
    B, gamma = 8, 3
    print(f"division range edges B={B} gamma={gamma} {mode}", flush=True)
    rng = np.random.default_rng(2718)
    w = hv.synthetic.accept_workload(B, gamma, seed=2718, dtype="bf16", mode=mode,
                                     per_seq_settings=True)
    tb = _edge_targets(hv, rng, B, gamma)
    xf = hv.synthetic.bf16_bits_to_f32(tb)
    temps = w["temperatures"].copy()
    temps[5], temps[6], temps[7] = 2.0 ** -12, 1.0, 2.0 ** 21
    lg = torch.from_numpy(tb.view(np.int16)).to(cuda).view(torch.bfloat16)
    t = _dev(w, cuda, ["draft_probs", "draft_tokens", "u_accept", "u_resample", "top_ks",
                       "top_ps"])
    tt = torch.from_numpy(temps).to(cuda)
    ref = orc.spec_accept(xf, w["draft_probs"], w["draft_tokens"], temps, w["u_accept"],
                          w["u_resample"], mode=mode, top_ks=w["top_ks"], top_ps=w["top_ps"])
    for chain in (False, True):
        r = hv.ops.spec_accept(lg, t["draft_probs"], t["draft_tokens"], tt, t["u_accept"],
                               t["u_resample"], mode=mode, top_ks=t["top_ks"],
                               top_ps=t["top_ps"], row_stats=True, chain_only=chain)
        got = [x.cpu().numpy() for x in r]
        np.testing.assert_array_equal(got[0], ref["num_accepted"])
        np.testing.assert_array_equal(got[1], ref["out_tokens"])
        np.testing.assert_array_equal(got[3].reshape(-1, 2), ref["row_stats"].reshape(-1, 2))
    rows = B * (gamma + 1)
    rt = np.repeat(temps, gamma + 1)
    rk = np.repeat(w["top_ks"], gamma + 1).astype(np.int32)
    rp = np.repeat(w["top_ps"], gamma + 1).astype(np.float32)
    u = rng.random(rows).astype(np.float32)
    s = hv.ops.sample_rows(lg.reshape(rows, V), *[torch.from_numpy(a).to(cuda) for a in (rt, rk, rp)],
                           mode=mode, uniforms=torch.from_numpy(u).to(cuda), want_probs=True,
                           row_stats=True)
    sref = orc.sampler(xf.reshape(rows, V), rt, rk, rp, mode=mode, uniforms=u)
    np.testing.assert_array_equal(s["probs"].cpu().numpy(), sref["probs"])
    np.testing.assert_array_equal(s["tokens"].cpu().numpy(), sref["tokens"])
    np.testing.assert_array_equal(s["row_stats"].cpu().numpy(), sref["row_stats"])
