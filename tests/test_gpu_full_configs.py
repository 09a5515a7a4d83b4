"""GPU parity at the full sizes of configs 1 and 4 (and the filter's bucket paths).

* Config 4 attention: the verify shapes of adaptive-gamma batched decoding with
  an FP8 target cache (e4m3fn with per-tensor amax/448 scales, 256-token
  blocks, contexts up to 8192 keys, so 32-entry block tables, 2..9 query rows
  per sequence, B = 32, 32 Q / 8 KV heads) and its bf16 draft cache (16 Q / 8 KV
  heads). The whole batch runs on the GPU; a subset of sequences (the longest,
  the shortest, one at a block boundary and a few others) goes through the
  float64 oracle, within the 2e-2 bound of the specification.
* Long contexts through the per-tile grid with key splits (B = 2, 8192 keys).
* Config 1 at full size: hs_spec_accept against the C oracle at B = 64,
  gamma = 3 and B = 256, gamma = 5, V = 151936, bf16 logits, per-sequence
  temperature / top-k / top-p, in reference, filtered and greedy modes; accept
  counts and tokens bit-exact.
* The top-p filter's boundary-bucket paths: a coarse boundary bucket of ~1000
  elements (appended whole by the second pass) and of ~10000 (refined into fine
  buckets, third pass), f32 and bf16 rows.
* Attention.forward under the reference's decode context
  (model_runner.py:310: set_context(False, slot_mapping, context_lens,
  block_tables), no max_seqlen_k).
"""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.fixture(scope="module")
def attn(orc):
    from oracle import attn as A
    return A


def _bf16(hv, x, dev):
    bits = hv.synthetic.f32_to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)


def _ragged_queries(w, ql):
    """Keep the first ql[b] query rows of every sequence (cu_seqlens_q rebuilt)."""
    B = len(ql)
    keep = np.concatenate([np.arange(w["cu_seqlens_q"][b], w["cu_seqlens_q"][b] + ql[b])
                           for b in range(B)])
    w["q"] = np.ascontiguousarray(w["q"][keep])
    w["cu_seqlens_q"] = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    w["max_seqlen_q"] = int(np.max(ql))
    return w


def _oracle_subset(attn, w, kref, vref, sel):
    """float64 oracle output for sequences `sel` only, from a compact copy of their
    blocks (block ids remapped), as rows in the order of the selected sequences."""
    bt = w["block_tables"]
    lens = w["lens"]
    bs = w["block_size"]
    blocks, tables = [], []
    for b in sel:
        n = (int(lens[b]) + bs - 1) // bs
        tables.append(list(range(len(blocks), len(blocks) + n)))
        blocks.extend(int(x) for x in bt[b, :n])
    W = max(len(t) for t in tables)
    sbt = np.full((len(sel), W), -1, np.int32)
    for i, t in enumerate(tables):
        sbt[i, :len(t)] = t
    kc = kref[blocks]
    vc = vref[blocks]
    cq, ck = w["cu_seqlens_q"], w["cu_seqlens_k"]
    rows = np.concatenate([np.arange(cq[b], cq[b + 1]) for b in sel])
    qn = np.array([cq[b + 1] - cq[b] for b in sel])
    kn = np.array([ck[b + 1] - ck[b] for b in sel])
    scq = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    sck = np.concatenate([[0], np.cumsum(kn)]).astype(np.int32)
    ref = attn.paged_attention(w["q"][rows], kc, vc, sbt, scq, sck, w["softmax_scale"])
    return rows, ref


def _run_subset(hv, attn, w, dev, kv, sel, workspace=True):
    if kv == "fp8":
        ks = float(np.nanmax(np.abs(w["k_cache"]))) / 448.0
        vs = float(np.nanmax(np.abs(w["v_cache"]))) / 448.0
        kq = attn.e4m3fn_quantize(w["k_cache"], ks)
        vq = attn.e4m3fn_quantize(w["v_cache"], vs)
        kc = torch.from_numpy(kq).to(dev).view(torch.float8_e4m3fn)
        vc = torch.from_numpy(vq).to(dev).view(torch.float8_e4m3fn)
        table = attn.e4m3fn_table().astype(np.float64)

        class Deq:  # dequantises only the blocks the oracle gathers
            def __init__(self, codes, scale):
                self.codes, self.scale = codes, scale

            def __getitem__(self, idx):
                return table[self.codes[idx]] * self.scale

        kref, vref = Deq(kq, ks), Deq(vq, vs)
    else:
        ks = vs = 1.0
        kc = _bf16(hv, w["k_cache"], dev)
        vc = _bf16(hv, w["v_cache"], dev)
        kref, vref = w["k_cache"], w["v_cache"]
    q = _bf16(hv, w["q"], dev)
    out = hv.ops.verify_attention(
        q, kc, vc, torch.from_numpy(w["block_tables"]).to(dev),
        torch.from_numpy(w["cu_seqlens_q"]).to(dev), torch.from_numpy(w["cu_seqlens_k"]).to(dev),
        w["max_seqlen_q"], w["max_seqlen_k"], w["softmax_scale"], k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    rows, ref = _oracle_subset(attn, w, kref, vref, sel)
    err = np.abs(got[rows] - ref)
    bad = err > TOL + TOL * np.abs(ref)
    assert not bad.any(), (err.max(), np.argwhere(bad)[:5])
    return float(err.max())


def _config4_lens(rng, B):
    lens = rng.integers(1024, 8193, size=B)
    lens[:6] = [8192, 8191, 7937, 4096, 2049, 1024]  # the maximum, block edges, short
    return lens


@pytest.mark.parametrize("which", ["target-fp8", "draft-bf16"])
def test_config4_attention_to_8192_keys(hv, attn, cuda, which):
    hq, kv = (32, "fp8") if which == "target-fp8" else (16, "bf16")
    rng = np.random.default_rng(40 + hq)
    B = 32
    lens = _config4_lens(rng, B)
    print(f"config4 attention {which} B={B} max {lens.max()} keys", flush=True)
    w = hv.synthetic.attention_workload(batch=B, q_len=9, num_q_heads=hq, num_kv_heads=8,
                                        lens=lens, seed=41 + hq, spare_blocks=5)
    assert w["block_tables"].shape == (B, 32)
    ql = rng.integers(2, 10, size=B)
    ql[:3] = [9, 2, 8]
    w = _ragged_queries(w, ql)
    sel = [0, 1, 2, 3, 4, 5, 17, 31]
    err = _run_subset(hv, attn, w, cuda, kv, sel)
    print(f"max err {err:.3e}", flush=True)


@pytest.mark.parametrize("kv", ["fp8", "bf16"])
def test_long_context_split_grid(hv, attn, cuda, kv):
    """Two sequences of up to 8192 keys: too few tiles for the one-workgroup-per-CU
    launch, so the per-tile grid splits the keys and merges the splits."""
    print(f"long context split grid {kv}", flush=True)
    w = hv.synthetic.attention_workload(batch=2, q_len=4, num_q_heads=32, num_kv_heads=8,
                                        lens=[8192, 5000], seed=45)
    _run_subset(hv, attn, w, cuda, kv, [0, 1])


# ---------------------------------------------------------------- config 1, full size
def _accept_both(hv, orc, w, cuda, mode):
    lg = torch.from_numpy(w["logits_bits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    t = {k: torch.from_numpy(np.ascontiguousarray(w[k])).to(cuda)
         for k in ["draft_probs", "draft_tokens", "temperatures", "top_ks", "top_ps",
                   "u_accept", "u_resample"]}
    nacc, out, olen = hv.ops.spec_accept(lg, t["draft_probs"], t["draft_tokens"],
                                         t["temperatures"], t["u_accept"], t["u_resample"],
                                         mode=mode, top_ks=t["top_ks"], top_ps=t["top_ps"])
    torch.cuda.synchronize()
    del lg, t
    ref = orc.spec_accept(w["logits"], w["draft_probs"], w["draft_tokens"], w["temperatures"],
                          w["u_accept"], w["u_resample"], mode=mode, top_ks=w["top_ks"],
                          top_ps=w["top_ps"])
    np.testing.assert_array_equal(nacc.cpu().numpy(), ref["num_accepted"])
    np.testing.assert_array_equal(out.cpu().numpy(), ref["out_tokens"])
    np.testing.assert_array_equal(olen.cpu().numpy(), ref["out_len"])
    return ref


@pytest.mark.parametrize("B,gamma", [(64, 1), (64, 3), (64, 5), (256, 1), (256, 3), (256, 5)])
@pytest.mark.parametrize("mode", ["reference", "filtered", "greedy"])
def test_config1_full_size(hv, orc, cuda, B, gamma, mode):
    """Config 1 over its grid B in {64, 256} x gamma in {1, 3, 5} (B = 8 is in
    test_gpu_sampler.py): bf16 logits, per-sequence T / top-k / top-p, the three
    modes; accepted counts, emitted tokens and lengths bit-exact vs the C oracle."""
    print(f"config1 full size B={B} gamma={gamma} {mode}", flush=True)
    w = hv.synthetic.accept_workload(B, gamma, seed=7000 + B + gamma, dtype="bf16",
                                     per_seq_settings=True,
                                     mode="filtered" if mode == "filtered" else "reference")
    if mode == "greedy":
        # drafts that match the target's argmax for a varying prefix of each sequence
        am = w["logits"].argmax(-1)
        for b in range(B):
            n = b % (gamma + 1)
            w["draft_tokens"][b, :n] = am[b, :n]
    ref = _accept_both(hv, orc, w, cuda, mode)
    # every first-reject position occurs, so both residual and bonus draws ran
    if mode != "filtered" or B == 256:
        assert len(set(ref["num_accepted"].tolist())) >= min(gamma + 1, 3)


# ---------------------------------------------------------------- filter bucket paths
def _plateau_rows(V, n_plat, rng, bf16):
    """Rows whose top-p 0.9 crossing falls inside a plateau of n_plat elements just
    below one spike at 10: (M - x) * 8 of every plateau element lies in [8, 9), so
    the coarse bucket holding the crossing has n_plat elements. f32 plateaus spread
    over (8.88, 8.98]; bf16 plateaus take the representable values 9 and 8.9375
    (ties, broken by index)."""
    rows = []
    for r in range(2):
        x = (rng.standard_normal(V) - 12.0).astype(np.float32)
        pos = rng.choice(V, size=n_plat + 1, replace=False)
        x[pos[0]] = 10.0
        if bf16:
            vals = np.array([9.0, 8.9375], np.float32) if r == 0 else np.array([8.9375],
                                                                                 np.float32)
            x[pos[1:]] = rng.choice(vals, size=n_plat)
        else:
            x[pos[1:]] = (8.98 - (0.1 if r == 0 else 0.05) * rng.random(n_plat)).astype(
                np.float32)
        rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("n_plat", [1000, 10000])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_filter_boundary_bucket_paths(hv, orc, cuda, n_plat, dtype):
    """Boundary bucket above 256 elements: up to 4096 it is appended whole by the
    second pass, above that it is refined into fine sub-buckets whose boundary one
    the third pass appends. The bucket's size is checked on the host from the
    same bucket rule ((M - x) * 8 with x = logit / T)."""
    rng = np.random.default_rng(90 + n_plat)
    V = 151936
    x = _plateau_rows(V, n_plat, rng, dtype == "bf16")
    if dtype == "bf16":
        bits = hv.synthetic.f32_to_bf16_bits(x)
        xf = hv.synthetic.bf16_bits_to_f32(bits)
        lg = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        xf = x
        lg = torch.from_numpy(x).to(cuda)
    R = xf.shape[0]
    T = np.ones(R, np.float32)
    tk = np.zeros(R, np.int32)
    tp = np.full(R, 0.9, np.float32)
    for r in range(R):  # host-side size of the boundary bucket
        xs = np.sort(xf[r].astype(np.float64))[::-1]
        p = np.exp(xs - xs[0])
        c = np.cumsum(p) / p.sum()
        cross = xs[int(np.searchsorted(c, 0.9))]
        bucket = np.floor((xs[0] - xf[r].astype(np.float64)) * 8)
        c1 = int((bucket == np.floor((xs[0] - cross) * 8)).sum())
        assert (256 < c1 <= 4096) if n_plat == 1000 else (c1 > 4096), c1
    u = rng.random(R).astype(np.float32)
    print(f"boundary bucket n={n_plat} {dtype}", flush=True)
    r = hv.ops.sample_rows(lg, torch.from_numpy(T).to(cuda), torch.from_numpy(tk).to(cuda),
                           torch.from_numpy(tp).to(cuda), mode="filtered",
                           uniforms=torch.from_numpy(u).to(cuda), want_probs=True,
                           row_stats=True)
    ref = orc.sampler(xf, T, tk, tp, mode="filtered", uniforms=u)
    np.testing.assert_array_equal(r["probs"].cpu().numpy(), ref["probs"])
    np.testing.assert_array_equal(r["tokens"].cpu().numpy(), ref["tokens"])
    np.testing.assert_array_equal(r["row_stats"].cpu().numpy(), ref["row_stats"])
    kept = (ref["probs"] > 0).sum(-1)
    assert (kept > 1).all() and (kept < n_plat + 1).all(), kept


# ---------------------------------------------------------------- drop-in decode context
def test_attention_forward_under_reference_decode_context(hv, attn, cuda):
    """Attention.forward as the reference's decode path calls it: the context has
    slot_mapping, context_lens and block_tables only (no cu_seqlens, no
    max_seqlen_k, model_runner.py:310,815,853) and the module has no
    max_model_len; the launch is sized by the block-table width."""
    A = importlib.import_module("hilda-vllm_amd.layers.attention")
    C = importlib.import_module("hilda-vllm_amd.utils.context")
    B, Hq, Hkv, D, bs = 5, 16, 8, 128, 256
    lens = np.array([1, 77, 256, 300, 700])
    w = hv.synthetic.attention_workload(batch=B, q_len=1, num_q_heads=Hq, num_kv_heads=Hkv,
                                        lens=lens, seed=96)
    # the step's token (last position) is stored by forward itself: take its K/V out
    # of the reference cache and let forward write them
    kc = _bf16(hv, np.nan_to_num(w["k_cache"]), cuda)
    vc = _bf16(hv, np.nan_to_num(w["v_cache"]), cuda)
    bt = w["block_tables"]
    last = lens - 1
    slots = np.array([int(bt[b, last[b] // bs]) * bs + last[b] % bs for b in range(B)],
                     np.int32)
    knew = w["k_cache"][slots // bs, slots % bs].copy()
    vnew = w["v_cache"][slots // bs, slots % bs].copy()
    kc.view(-1, Hkv, D)[torch.from_numpy(slots).long().to(cuda)] = 0
    vc.view(-1, Hkv, D)[torch.from_numpy(slots).long().to(cuda)] = 0
    layer = A.Attention(Hq, D, D ** -0.5, Hkv)
    layer.k_cache, layer.v_cache = kc, vc
    assert layer.max_model_len == 0
    C.set_context(False, slot_mapping=torch.from_numpy(slots).to(cuda),
                  context_lens=torch.from_numpy(lens.astype(np.int32)).to(cuda),
                  block_tables=torch.from_numpy(bt).to(cuda))
    try:
        out = layer(_bf16(hv, w["q"], cuda), _bf16(hv, knew, cuda), _bf16(hv, vnew, cuda))
    finally:
        C.reset_context()
    torch.cuda.synchronize()
    ref = attn.paged_attention(w["q"], w["k_cache"], w["v_cache"], bt, w["cu_seqlens_q"],
                               w["cu_seqlens_k"], w["softmax_scale"])
    got = out.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(got - ref)
    assert not (err > TOL + TOL * np.abs(ref)).any(), err.max()
