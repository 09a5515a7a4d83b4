"""Fused decoder-layer kernels vs the unfused kernels they replace.

* hs_linear_rmsnorm (RMSNorm / add + RMSNorm inside the projection) against
  hs_rmsnorm followed by hs_linear and against an fp32 PyTorch restatement of
  layernorm.py:18-36 + F.linear. The new residual bf16(x + residual) is one
  fp32 add and one rounding on both sides: bit-exact. The outputs may differ
  where the fused kernel's sum of squares (summed in another order) moves a
  normalised value across a bf16 rounding boundary: |err| <= 1e-2 * scale, the
  bound of the plain projection test.
* hs_qk_norm_rope_store against hs_qk_norm_rope + hs_store_kvcache: the same
  per-lane arithmetic, so q and both caches (bf16 and FP8) are bit-exact,
  including tokens whose slot is -1 (nothing stored).
* hs_qk_norm_rope_attend against hs_qk_norm_rope_store + hs_verify_attention:
  outputs and both caches bit-exact, for the fused launch and the shapes that
  run as two launches.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _norm_ref(x, res, w, eps):
    """layernorm.py:18-36 in fp32 with the reference's two roundings."""
    xf = x.float() if res is None else x.float() + res.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return ((xf * inv).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("K,N,swiglu", [(4096, 6144, False), (1024, 4096, False),
                                        (4096, 12288, True), (1024, 3072, True),
                                        (4096, 151936, False)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_linear_rmsnorm_matches_unfused(hv, cuda, M, K, N, swiglu, with_residual):
    ops = hv.ops
    g = torch.Generator(device=cuda).manual_seed(M * 7 + K + N + with_residual)
    x = (torch.randn((M, K), generator=g, device=cuda) * 3).to(torch.bfloat16)
    res = (torch.randn((M, K), generator=g, device=cuda) * 5).to(torch.bfloat16) \
        if with_residual else None
    nw = (1 + 0.1 * torch.randn(K, generator=g, device=cuda)).to(torch.bfloat16)
    rows = 2 * N if swiglu else N
    w = (torch.randn((rows, K), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    eps = 1e-6
    print(f"linear_rmsnorm M={M} K={K} N={N} swiglu={swiglu} res={with_residual}", flush=True)
    res_before = None if res is None else res.clone()
    y, new_res = ops.linear_rmsnorm(x, nw, eps, w, residual=res, swiglu=swiglu)
    # unfused chain: rmsnorm kernel (residual updated in place) + skinny projection
    res_u = None if res is None else res.clone()
    xn = ops.rmsnorm(x, nw, eps, residual=res_u)
    y_u = ops.linear(xn, w, swiglu=swiglu)
    torch.cuda.synchronize()
    if res is None:
        assert new_res is x
    else:
        assert torch.equal(res, res_before), "the input residual must not be modified"
        assert torch.equal(new_res, res_u)
        assert torch.equal(new_res, (x.float() + res_before.float()).to(torch.bfloat16))
    # fp32 reference of the whole chain
    xr = _norm_ref(x, res_before, nw, eps).float()
    ref = xr @ w.float().t()
    if swiglu:
        ref = torch.nn.functional.silu(ref[:, :N]) * ref[:, N:]
    scale = ref.abs().max().item()
    assert (y.float() - ref).abs().max().item() <= 1e-2 * scale
    assert (y.float() - y_u.float()).abs().max().item() <= 1e-2 * scale


def test_linear_rmsnorm_fallback_rows(hv, cuda):
    """More than 8 rows: hs_rmsnorm + library GEMM, residual updated in place."""
    ops = hv.ops
    g = torch.Generator(device=cuda).manual_seed(5)
    x = torch.randn((16, 1024), generator=g, device=cuda).to(torch.bfloat16)
    res = torch.randn((16, 1024), generator=g, device=cuda).to(torch.bfloat16)
    nw = torch.ones(1024, device=cuda, dtype=torch.bfloat16)
    w = (torch.randn((512, 1024), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    expect_res = (x.float() + res.float()).to(torch.bfloat16)
    xr = _norm_ref(x, res, nw, 1e-6).float()
    y, new_res = ops.linear_rmsnorm(x, nw, 1e-6, w, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(new_res, expect_res)
    ref = xr @ w.float().t()
    assert (y.float() - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()


def _rope_table(max_pos, device):
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32, device=device) / 128))
    f = torch.outer(torch.arange(max_pos, dtype=torch.float32, device=device), inv)
    return torch.cat([f.cos(), f.sin()], -1).contiguous()


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("N,Hq,Hkv", [(4, 32, 8), (1, 16, 8), (37, 8, 4)])
def test_qk_norm_rope_store_matches_separate(hv, cuda, kv, N, Hq, Hkv):
    ops = hv.ops
    g = torch.Generator(device=cuda).manual_seed(N * 100 + Hq + Hkv)
    qkv = (torch.randn((N, (Hq + 2 * Hkv) * 128), generator=g, device=cuda) * 2).to(
        torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, generator=g, device=cuda)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g, device=cuda)).to(torch.bfloat16)
    cs = _rope_table(4096, cuda)
    pos = torch.randint(0, 4096, (N,), generator=g, device=cuda)
    nb, bs = 6, 16
    slots = torch.randperm(nb * bs, generator=g, device=cuda)[:N].to(torch.int32)
    slots[::3] = -1  # tokens without a slot store nothing
    dt = torch.bfloat16 if kv == "bf16" else torch.float8_e4m3fn
    ksc, vsc = (1.0, 1.0) if kv == "bf16" else (0.05, 0.03)
    print(f"qk_norm_rope_store kv={kv} N={N} Hq={Hq} Hkv={Hkv}", flush=True)

    def caches():
        fill = torch.randint(0, 255, (2, nb, bs, Hkv, 128), generator=g, device=cuda,
                             dtype=torch.uint8)
        if dt == torch.bfloat16:
            fill = fill.to(torch.int16).view(torch.bfloat16)
            return fill[0].clone(), fill[1].clone()
        fill = fill & 0x77  # finite e4m3 codes
        return fill[0].clone().view(dt), fill[1].clone().view(dt)

    kc1, vc1 = caches()
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1, k1 = ops.qk_norm_rope(qkv, Hq, Hkv, qw, kw, cs, pos, 1e-6)
    v = qkv[:, (Hq + Hkv) * 128:].reshape(N, Hkv, 128)
    ops.store_kvcache(k1, v, kc1, vc1, slots, k_scale=ksc, v_scale=vsc)
    q2 = ops.qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, cs, pos, 1e-6, kc2, vc2, slots,
                                k_scale=ksc, v_scale=vsc)
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    u8 = lambda t: t.view(torch.uint8)  # noqa: E731
    assert torch.equal(u8(kc1), u8(kc2))
    assert torch.equal(u8(vc1), u8(vc2))


# (name, Hq, Hkv, query lengths, earlier keys per sequence, block size,
# declared max_seqlen_k or None for the longest): the verify step of the 8B
# target, decode of the 0.6B draft (one sequence with no earlier key: its
# first window holds the new key), a batch over several blocks, a padding
# token (slot -1), G = 1, RoPE positions that differ from the key index, and
# two shapes that run as two launches (two query tiles; the balanced launch
# of a large batch). Batch-1 cases: verify, decode, the draft's two-token
# first step, new keys straddling two 32-key windows or starting one, all
# keys new, a padding token and a slot elsewhere than the key's table entry.
# A declared max_seqlen_k of 4101 (max_model_len 4096 plus the verify tokens)
# plans five 1024-key splits: contexts within one split run as one workgroup
# per kv head, longer ones merge their splits in the kernel (one sequence,
# new keys on both sides of a split edge, and two sequences of different
# lengths).
_ATTEND_CASES = [
    ("verify-8b", 32, 8, [4], [316], 256, None),
    ("decode-06b", 16, 8, [1, 1, 1], [76, 299, 0], 256, None),
    ("verify-batch", 32, 8, [4, 4, 4, 4], [1, 36, 300, 700], 32, None),
    ("padding-slot", 16, 8, [2, 2], [10, 20], 32, None),
    ("g1", 8, 8, [4], [100], 256, None),
    ("pos-offset", 32, 8, [4, 4], [60, 200], 256, None),
    ("two-tiles", 32, 8, [5, 3], [50, 100], 256, None),
    ("balanced", 32, 8, [4] * 32, [1500 + 17 * i for i in range(32)], 256, None),
    ("decode-b1", 16, 8, [1], [299], 256, None),
    ("lookback-b1", 16, 8, [2], [100], 256, None),
    ("straddle-b1", 32, 8, [4], [318], 256, None),
    ("window-start-b1", 32, 8, [4], [320], 256, None),
    ("first-window-b1", 32, 8, [4], [0], 256, None),
    ("padding-b1", 32, 8, [4], [200], 256, None),
    ("slot-elsewhere-b1", 32, 8, [4], [200], 256, None),
    ("mml4096-b1", 32, 8, [4], [316], 256, 4101),
    ("mml4096-long-b1", 32, 8, [4], [2600], 256, 4101),
    ("mml4096-decode-b2", 16, 8, [1, 1], [1500, 3000], 256, 4101),
    ("mml4096-split-edge-b1", 32, 8, [4], [1022], 256, 4101),
]


def _attend_inputs(cuda, kv, case):
    """Inputs of one fused-attention case: the qkv rows of the query tokens,
    norm weights, the RoPE table, positions and slots of the tokens, a random
    block table and random caches (bf16, or finite e4m3fn codes)."""
    name, Hq, Hkv, qls, ctxs, bs, max_k_decl = case
    B = len(qls)
    g = torch.Generator(device=cuda).manual_seed(sum(qls) * 1000 + sum(ctxs) + Hq + bs)
    lks = [c + q for c, q in zip(ctxs, qls)]
    nblk = [(lk + bs - 1) // bs for lk in lks]
    nb = sum(nblk) + 3
    perm = torch.randperm(nb, generator=g, device=cuda).to(torch.int32)
    W = max(nblk)
    bt = torch.full((B, W), -1, dtype=torch.int32, device=cuda)
    o = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    spare = perm[o:].tolist()  # blocks in no table
    btc = bt.cpu()
    pos, slots = [], []
    for b in range(B):
        for i in range(qls[b]):
            p = ctxs[b] + i
            # RoPE positions other than the key index (the kernel's cos/sin guess)
            pos.append(p + 7 if name == "pos-offset" else p)
            slots.append(int(btc[b, p // bs]) * bs + p % bs)
    if name in ("padding-slot", "padding-b1"):
        slots[1] = -1  # a padding token: nothing stored, the cache keeps its old row
    if name == "slot-elsewhere-b1":
        slots[2] = spare[0] * bs + 5  # stored elsewhere; its key reads the table's row
    N = len(pos)
    cu_q = torch.tensor([0] + list(torch.tensor(qls).cumsum(0)), dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0] + list(torch.tensor(lks).cumsum(0)), dtype=torch.int32, device=cuda)
    qkv = (torch.randn((N, (Hq + 2 * Hkv) * 128), generator=g, device=cuda) * 2).to(
        torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(128, generator=g, device=cuda)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(128, generator=g, device=cuda)).to(torch.bfloat16)
    dt = torch.bfloat16 if kv == "bf16" else torch.float8_e4m3fn
    ksc, vsc = (1.0, 1.0) if kv == "bf16" else (0.05, 0.03)
    if dt == torch.bfloat16:
        kc = torch.randn((nb, bs, Hkv, 128), generator=g, device=cuda).to(dt)
        vc = torch.randn((nb, bs, Hkv, 128), generator=g, device=cuda).to(dt)
    else:
        fill = torch.randint(0, 255, (2, nb, bs, Hkv, 128), generator=g, device=cuda,
                             dtype=torch.uint8) & 0x77  # finite e4m3 codes
        kc, vc = fill[0].clone().view(dt), fill[1].clone().view(dt)
    return dict(B=B, Hq=Hq, Hkv=Hkv, bs=bs, qls=qls, lks=lks, bt=bt, cu_q=cu_q, cu_k=cu_k,
                pos=torch.tensor(pos, dtype=torch.int64, device=cuda),
                slots=torch.tensor(slots, dtype=torch.int32, device=cuda), qkv=qkv, qw=qw,
                kw=kw, cs=_rope_table(4096, cuda), kc=kc, vc=vc, ksc=ksc, vsc=vsc,
                max_q=max(qls), max_k=max_k_decl or max(lks))


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("case", _ATTEND_CASES, ids=[c[0] for c in _ATTEND_CASES])
def test_qk_norm_rope_attend_matches_two_launches(hv, cuda, kv, case):
    """hs_qk_norm_rope_attend against hs_qk_norm_rope_store + hs_verify_attention
    (+ the split combine): the fused prologue uses the same per-lane arithmetic,
    the attention the same kernel body over the same 32-key windows, and the
    splits merge with the combine's arithmetic, so the outputs and both caches
    are bit-exact."""
    ops = hv.ops
    x = _attend_inputs(cuda, kv, case)
    Hq, Hkv = x["Hq"], x["Hkv"]
    kc1, vc1 = x["kc"], x["vc"]
    kc2, vc2 = kc1.clone(), vc1.clone()
    scale = 128 ** -0.5
    print(f"qk_norm_rope_attend {case[0]} kv={kv} B={x['B']} max_k={x['max_k']}", flush=True)
    q = ops.qk_norm_rope_store(x["qkv"], Hq, Hkv, x["qw"], x["kw"], x["cs"], x["pos"], 1e-6, kc1,
                               vc1, x["slots"], k_scale=x["ksc"], v_scale=x["vsc"])
    out1 = ops.verify_attention(q, kc1, vc1, x["bt"], x["cu_q"], x["cu_k"], x["max_q"],
                                x["max_k"], scale, k_scale=x["ksc"], v_scale=x["vsc"])
    out2 = ops.qk_norm_rope_attend(x["qkv"], Hq, Hkv, x["qw"], x["kw"], x["cs"], x["pos"], 1e-6,
                                   kc2, vc2, x["slots"], x["bt"], x["cu_q"], x["cu_k"],
                                   x["max_q"], x["max_k"], scale, k_scale=x["ksc"],
                                   v_scale=x["vsc"])
    # a second call on the same workspace (split tickets left at zero)
    out3 = ops.qk_norm_rope_attend(x["qkv"], Hq, Hkv, x["qw"], x["kw"], x["cs"], x["pos"], 1e-6,
                                   kc2, vc2, x["slots"], x["bt"], x["cu_q"], x["cu_k"],
                                   x["max_q"], x["max_k"], scale, k_scale=x["ksc"],
                                   v_scale=x["vsc"])
    torch.cuda.synchronize()
    u8 = lambda t: t.view(torch.uint8)  # noqa: E731
    assert torch.equal(u8(kc1), u8(kc2))
    assert torch.equal(u8(vc1), u8(vc2))
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(out1.view(torch.int16), out3.view(torch.int16))


def _norm_rope_ref(x, w, cos_sin, pos, eps):
    """q/k RMSNorm + neox RoPE on the CPU in fp32: layernorm.py:18-25 (normalise in
    fp32, round to bf16, multiply by the bf16 weight) then rotary_embedding.py:8-16,
    39-50 (cos/sin rows of the positions, fp32 rotation, rounded to bf16).
    x [N, H, 128] bf16."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    xn = (xf * torch.rsqrt(var + eps)).to(torch.bfloat16) * w
    cs = cos_sin[pos]
    cos, sin = cs[:, None, :64], cs[:, None, 64:]
    x1, x2 = xn.float().chunk(2, -1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(torch.bfloat16)


_ORACLE_CASES = [c for c in _ATTEND_CASES
                 if c[0] in ("verify-8b", "decode-b1", "lookback-b1", "decode-06b",
                             "straddle-b1", "mml4096-b1", "mml4096-long-b1",
                             "mml4096-decode-b2")]


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("case", _ORACLE_CASES, ids=[c[0] for c in _ORACLE_CASES])
def test_qk_norm_rope_attend_matches_oracle(hv, cuda, kv, case):
    """hs_qk_norm_rope_attend against the CPU oracle of the same step: the q/k
    RMSNorm + RoPE of qwen3.py:82-85 restated in fp32 torch (layernorm.py:18-25,
    rotary_embedding.py:39-50), the K/V store of attention.py:59-90 (e4m3fn codes
    through the oracle codec for fp8) and the paged causal attention of
    attention.py:145-160 in float64 (oracle/attn.py). V rows and the cache rows
    the call must not touch are bit-exact; the stored K rows agree with the
    restatement to one bf16 ulp (one e4m3 step) where the two sums of squares
    round differently; outputs agree within 2e-2."""
    from oracle import attn as oa
    ops = hv.ops
    x = _attend_inputs(cuda, kv, case)
    Hq, Hkv, bs = x["Hq"], x["Hkv"], x["bs"]
    kc0, vc0 = x["kc"].cpu(), x["vc"].cpu()
    kc, vc = x["kc"], x["vc"]
    scale = 128 ** -0.5
    print(f"qk_norm_rope_attend vs oracle {case[0]} kv={kv}", flush=True)
    out = ops.qk_norm_rope_attend(x["qkv"], Hq, Hkv, x["qw"], x["kw"], x["cs"], x["pos"], 1e-6,
                                  kc, vc, x["slots"], x["bt"], x["cu_q"], x["cu_k"], x["max_q"],
                                  x["max_k"], scale, k_scale=x["ksc"], v_scale=x["vsc"])
    torch.cuda.synchronize()
    # oracle: norm + RoPE on the CPU, the store, then the float64 attention
    qkv = x["qkv"].cpu()
    N = qkv.shape[0]
    pos = x["pos"].cpu()
    cs = x["cs"].cpu()
    q = _norm_rope_ref(qkv[:, :Hq * 128].view(N, Hq, 128), x["qw"].cpu(), cs, pos, 1e-6)
    k = _norm_rope_ref(qkv[:, Hq * 128:(Hq + Hkv) * 128].view(N, Hkv, 128), x["kw"].cpu(), cs,
                       pos, 1e-6)
    v = qkv[:, (Hq + Hkv) * 128:].reshape(N, Hkv, 128)
    slots = x["slots"].cpu().numpy()
    if kv == "bf16":
        kref, vref = kc0.float().numpy().copy(), vc0.float().numpy().copy()
        kstore, vstore = k.float().numpy(), v.float().numpy()
    else:
        kref, vref = kc0.view(torch.uint8).numpy().copy(), vc0.view(torch.uint8).numpy().copy()
        kstore = oa.e4m3fn_quantize(k.float().numpy(), x["ksc"])
        vstore = oa.e4m3fn_quantize(v.float().numpy(), x["vsc"])
    oa.store_kvcache(kstore, vstore, kref, vref, slots)
    got_k = kc.cpu().float().numpy() if kv == "bf16" else kc.cpu().view(torch.uint8).numpy()
    got_v = vc.cpu().float().numpy() if kv == "bf16" else vc.cpu().view(torch.uint8).numpy()
    assert np.array_equal(got_v, vref)
    # K: rows the call stores may differ from the restatement by one bf16 ulp / e4m3 step
    if kv == "bf16":
        diff = np.abs(got_k - kref)
        tol = np.abs(kref) * 2.0 ** -7 + 1e-30
        assert (diff <= tol).all()
    else:
        dec = oa.e4m3fn_table()
        diff = np.abs(dec[got_k].astype(np.float64) - dec[kref].astype(np.float64))
        assert (diff <= np.abs(dec[kref]) * 0.125 + 2.0 ** -9).all()
    assert (got_k != kref).mean() < 1e-3
    if kv == "bf16":
        kd, vd = got_k, got_v
    else:
        kd, vd = oa.dequant(got_k, x["ksc"]), oa.dequant(got_v, x["vsc"])
    ref = oa.paged_attention(q.float().numpy(), kd, vd, x["bt"].cpu().numpy(),
                             x["cu_q"].cpu().numpy(), x["cu_k"].cpu().numpy(), scale)
    err = np.abs(out.float().cpu().numpy() - ref).max()
    assert err <= 2e-2 * max(1.0, np.abs(ref).max()), err
