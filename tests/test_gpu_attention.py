"""GPU parity of the paged verify attention and the KV-cache store.

The HIP kernels run through the C ABI and are compared with the float64
oracle (oracle/attn.py) on identical inputs. Attention outputs are bf16 and
must agree within 2e-2 (absolute + relative); the BF16 store is a bit-exact
copy and the FP8 store must equal the oracle's codec bit for bit.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.fixture(scope="module")
def attn(orc):
    from oracle import attn as A
    return A


def _bf16(x, dev):
    from importlib import import_module
    hv = import_module("hilda-vllm_amd")
    bits = hv.synthetic.f32_to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)


def _run(hv, attn, w, cuda, kv="bf16", q_strided=False):
    dev = cuda
    if kv == "fp8":
        ks = float(np.nanmax(np.abs(w["k_cache"]))) / 448.0
        vs = float(np.nanmax(np.abs(w["v_cache"]))) / 448.0
        kq = attn.e4m3fn_quantize(w["k_cache"], ks)
        vq = attn.e4m3fn_quantize(w["v_cache"], vs)
        kc = torch.from_numpy(kq).to(dev).view(torch.float8_e4m3fn)
        vc = torch.from_numpy(vq).to(dev).view(torch.float8_e4m3fn)
        kref = attn.dequant(kq, ks)
        vref = attn.dequant(vq, vs)
    else:
        ks = vs = 1.0
        kc = _bf16(w["k_cache"], dev)
        vc = _bf16(w["v_cache"], dev)
        kref, vref = w["k_cache"], w["v_cache"]
    q = _bf16(w["q"], dev)
    if q_strided:  # q as the first slice of a fused qkv projection
        N, Hq, D = q.shape
        big = torch.zeros((N, Hq + 2 * 8, D), dtype=torch.bfloat16, device=dev)
        big[:, :Hq] = q
        q = big[:, :Hq]
    out = hv.ops.verify_attention(
        q, kc, vc, torch.from_numpy(w["block_tables"]).to(dev),
        torch.from_numpy(w["cu_seqlens_q"]).to(dev), torch.from_numpy(w["cu_seqlens_k"]).to(dev),
        w["max_seqlen_q"], w["max_seqlen_k"], w["softmax_scale"], k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    ref = attn.paged_attention(w["q"], kref, vref, w["block_tables"], w["cu_seqlens_q"],
                               w["cu_seqlens_k"], w["softmax_scale"])
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    bad = err > TOL + TOL * np.abs(ref)
    assert not bad.any(), (err.max(), np.argwhere(bad)[:5])
    return err.max()


def test_config2_bf16(hv, attn, cuda):
    print("config2 bf16 B=64", flush=True)
    w = hv.synthetic.attention_workload(seed=0)
    _run(hv, attn, w, cuda)


def test_config2_fp8(hv, attn, cuda):
    print("config2 fp8 B=64", flush=True)
    w = hv.synthetic.attention_workload(seed=1)
    _run(hv, attn, w, cuda, kv="fp8")


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8), (8, 8)])
def test_decode_single_query(hv, attn, cuda, hq, hkv):
    w = hv.synthetic.attention_workload(batch=12, q_len=1, num_q_heads=hq, num_kv_heads=hkv,
                                        min_len=1, max_len=700, seed=2)
    _run(hv, attn, w, cuda)


def test_prefill_long_queries(hv, attn, cuda):
    w = hv.synthetic.attention_workload(batch=3, q_len=64, num_q_heads=32, num_kv_heads=8,
                                        min_len=64, max_len=400, seed=3)
    _run(hv, attn, w, cuda)


def test_ragged_query_lengths_and_strided_q(hv, attn, cuda):
    w = hv.synthetic.attention_workload(batch=6, q_len=5, num_q_heads=16, num_kv_heads=8,
                                        min_len=5, max_len=900, seed=4, lens=None)
    # make query lengths ragged: shrink some and rebuild the prefix sums
    ql = np.array([5, 1, 3, 5, 2, 4])
    keep = np.concatenate([np.arange(w["cu_seqlens_q"][b], w["cu_seqlens_q"][b] + ql[b])
                           for b in range(6)])
    w["q"] = np.ascontiguousarray(w["q"][keep])
    w["cu_seqlens_q"] = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    w["max_seqlen_q"] = int(ql.max())
    _run(hv, attn, w, cuda, q_strided=True)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_small_blocks_and_short_contexts(hv, attn, cuda, kv):
    w = hv.synthetic.attention_workload(batch=9, q_len=4, num_q_heads=32, num_kv_heads=8,
                                        block_size=32, lens=[4, 5, 31, 32, 33, 64, 65, 100, 257],
                                        seed=5)
    _run(hv, attn, w, cuda, kv=kv)


def test_balanced_launch_short_actual_contexts(hv, attn, cuda):
    """max_seqlen_k selects the one-workgroup-per-CU launch while the actual contexts are
    1..70 keys: most workgroups get an empty window range and tiles are cut between
    neighbouring workgroups after a window or two."""
    print("balanced launch, short contexts", flush=True)
    lens = np.random.default_rng(7).integers(1, 71, size=64)
    w = hv.synthetic.attention_workload(batch=64, q_len=4, lens=lens, seed=7)
    w["max_seqlen_k"] = 2048
    _run(hv, attn, w, cuda)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_balanced_launch_odd_group_and_small_blocks(hv, attn, cuda, kv):
    """24 Q / 8 KV heads (group of 3, the generic group path), 32-token blocks, 3 queries."""
    print(f"balanced launch, G=3, block 32, {kv}", flush=True)
    w = hv.synthetic.attention_workload(batch=24, q_len=3, num_q_heads=24, num_kv_heads=8,
                                        block_size=32, min_len=3, max_len=1500, seed=8)
    _run(hv, attn, w, cuda, kv=kv)


@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 2)])
def test_balanced_launch_kv_head_major(hv, attn, cuda, hq, hkv):
    """Fewer than 8 kv heads: the balanced launch's kv-head-major tiles (waves take
    alternate windows of one head and merge in LDS)."""
    print(f"balanced launch, kv-head-major, {hq}/{hkv} heads", flush=True)
    w = hv.synthetic.attention_workload(batch=48, q_len=4, num_q_heads=hq, num_kv_heads=hkv,
                                        min_len=4, max_len=1500, seed=9)
    _run(hv, attn, w, cuda)


def test_balanced_launch_prefill_tiles(hv, attn, cuda):
    """64 queries x 4 heads per kv head = 16 query tiles per sequence, each seeing a
    different causal key range, in the heads-in-waves balanced launch."""
    print("balanced launch, prefill tiles", flush=True)
    w = hv.synthetic.attention_workload(batch=8, q_len=64, num_q_heads=32, num_kv_heads=8,
                                        min_len=64, max_len=1024, seed=10)
    _run(hv, attn, w, cuda)


def test_batch1_verify_shape_of_8b_target(hv, attn, cuda):
    """B=1, gamma+1=4 queries, 32 Q / 8 KV heads: the verify shape of config 3."""
    w = hv.synthetic.attention_workload(batch=1, q_len=4, num_q_heads=32, num_kv_heads=8,
                                        lens=[324], seed=6)
    _run(hv, attn, w, cuda)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_batch1_decode_shape_of_draft(hv, attn, cuda, kv):
    """B=1, one query, 16 Q / 8 KV heads: the draft's decode shape in config 3. The block
    table is exactly two entries wide, so most threads of the prologue read the clamped
    last entry and discard it."""
    print(f"draft decode shape {kv}", flush=True)
    w = hv.synthetic.attention_workload(batch=1, q_len=1, num_q_heads=16, num_kv_heads=8,
                                        lens=[324], seed=12)
    assert w["block_tables"].shape == (1, 2)
    _run(hv, attn, w, cuda, kv=kv)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_store_kvcache(hv, attn, cuda, kv):
    rng = np.random.default_rng(7)
    nb, bs, H, D = 6, 32, 8, 128
    N = 40
    key = rng.standard_normal((N, H, D)).astype(np.float32) * 3
    val = rng.standard_normal((N, H, D)).astype(np.float32) * 3
    key = hv.synthetic.bf16_bits_to_f32(hv.synthetic.f32_to_bf16_bits(key))
    val = hv.synthetic.bf16_bits_to_f32(hv.synthetic.f32_to_bf16_bits(val))
    slots = rng.permutation(nb * bs)[:N].astype(np.int32)
    slots[[3, 17]] = -1
    if kv == "bf16":
        kc = torch.zeros((nb, bs, H, D), dtype=torch.bfloat16, device=cuda)
        vc = torch.zeros_like(kc)
        hv.ops.store_kvcache(_bf16(key, cuda), _bf16(val, cuda), kc, vc,
                             torch.from_numpy(slots).to(cuda))
        ek = np.zeros((nb, bs, H, D), np.float32)
        ev = np.zeros_like(ek)
        attn.store_kvcache(key, val, ek, ev, slots)
        np.testing.assert_array_equal(kc.float().cpu().numpy(), ek)
        np.testing.assert_array_equal(vc.float().cpu().numpy(), ev)
    else:
        ks, vs = 0.021, 0.017
        kc = torch.zeros((nb, bs, H, D), dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn)
        vc = torch.zeros_like(kc)
        hv.ops.store_kvcache(_bf16(key, cuda), _bf16(val, cuda), kc, vc,
                             torch.from_numpy(slots).to(cuda), k_scale=ks, v_scale=vs)
        ek = np.zeros((nb, bs, H, D), np.uint8)
        ev = np.zeros_like(ek)
        attn.store_kvcache(attn.e4m3fn_quantize(key, ks), attn.e4m3fn_quantize(val, vs), ek, ev,
                           slots)
        np.testing.assert_array_equal(kc.view(torch.uint8).cpu().numpy(), ek)
        np.testing.assert_array_equal(vc.view(torch.uint8).cpu().numpy(), ev)


# ---------------------------------------------------------------- unpaged prefill
@pytest.mark.parametrize("cache", ["none", "bf16", "fp8"])
def test_attention_forward_unpaged_prefill(hv, attn, cuda, cache):
    """Attention.forward under the reference's prefill context without block tables
    (model_runner.py:614-649: set_context(True, cu_seqlens_q, cu_seqlens_k,
    max_seqlen_q, max_seqlen_k, slot_mapping, None, None) for prompts with no
    cached prefix), ragged prompts of 1 to 1500 tokens: the output is
    flash_attn_varlen_func over the step's own k / v (attention.py:147-160), here
    the float64 oracle per sequence within 2e-2; with a bound cache the k / v rows
    land at slot_mapping first (bf16: bit-exact; fp8: the oracle codec), with
    none (the reference's warm-up) nothing is stored."""
    from importlib import import_module
    ctxm = import_module("hilda-vllm_amd.utils.context")
    layer_mod = import_module("hilda-vllm_amd.layers.attention")
    Hq, Hkv, D, bs = 16, 8, 128, 256
    lens = [1, 37, 300, 1500, 4]
    g = torch.Generator(device=cuda).manual_seed(11)
    N = sum(lens)
    q = torch.randn((N, Hq * D), generator=g, device=cuda).to(torch.bfloat16)
    k = torch.randn((N, Hkv * D), generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn((N, Hkv * D), generator=g, device=cuda).to(torch.bfloat16)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=cuda)
    layer = layer_mod.Attention(Hq, D, D ** -0.5, Hkv)
    nblk = [(n + bs - 1) // bs for n in lens]
    nb = sum(nblk) + 2
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(5)).tolist()
    slots, o = [], 0
    for n, m in zip(lens, nblk):
        blocks = perm[o:o + m]
        o += m
        slots += [blocks[i // bs] * bs + i % bs for i in range(n)]
    slots_t = torch.tensor(slots, dtype=torch.int32, device=cuda)
    ksc = vsc = 1.0
    if cache != "none":
        dt = torch.bfloat16 if cache == "bf16" else torch.float8_e4m3fn
        kc = torch.zeros((nb, bs, Hkv, D), dtype=dt, device=cuda)
        vc = torch.zeros_like(kc)
        layer.k_cache, layer.v_cache = kc, vc
        if cache == "fp8":
            ksc, vsc = 0.02, 0.015
            layer.k_scale, layer.v_scale = ksc, vsc
    print(f"unpaged prefill cache={cache} lens={lens}", flush=True)
    ctxm.set_context(True, cu, cu, max(lens), max(lens), slots_t, None, None)
    try:
        out = layer(q, k, v)
    finally:
        ctxm.reset_context()
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(N, Hq, D)
    qn = q.float().cpu().numpy().reshape(N, Hq, D)
    kn = k.float().cpu().numpy().reshape(N, Hkv, D)
    vn = v.float().cpu().numpy().reshape(N, Hkv, D)
    for b, n in enumerate(lens):
        s0 = int(cu[b])
        ref = attn.paged_attention(qn[s0:s0 + n], kn[None, s0:s0 + n], vn[None, s0:s0 + n],
                                   np.zeros((1, 1), np.int64), np.array([0, n]),
                                   np.array([0, n]), D ** -0.5)
        err = np.abs(got[s0:s0 + n] - ref).max()
        assert err <= TOL * max(1.0, np.abs(ref).max()), (b, n, err)
    if cache == "none":
        return
    kc_h = layer.k_cache.view(torch.uint8).cpu().numpy() if cache == "fp8" else \
        layer.k_cache.float().cpu().numpy()
    vc_h = layer.v_cache.view(torch.uint8).cpu().numpy() if cache == "fp8" else \
        layer.v_cache.float().cpu().numpy()
    sl = np.array(slots)
    if cache == "fp8":
        kexp, vexp = attn.e4m3fn_quantize(kn, ksc), attn.e4m3fn_quantize(vn, vsc)
    else:
        kexp, vexp = kn, vn
    np.testing.assert_array_equal(kc_h[sl // bs, sl % bs], kexp)
    np.testing.assert_array_equal(vc_h[sl // bs, sl % bs], vexp)


@pytest.mark.parametrize("qlens,klens", [([40, 200], [40, 200]), ([4], [2100])])
def test_verify_attention_unpaged_matches_paged(hv, cuda, qlens, klens):
    """The unpaged mode (no block table) and the paged kernel over a cache holding
    the same rows give the same bits: the same windows and arithmetic, only the
    row addresses differ. A ragged prefill, and 4 queries over 2100 keys (three
    key splits and their combine); both shapes run the per-tile grid."""
    Hq, Hkv, D, bs = 32, 8, 128, 256
    g = torch.Generator(device=cuda).manual_seed(12 + sum(klens))
    N, Nk = sum(qlens), sum(klens)
    q = torch.randn((N, Hq, D), generator=g, device=cuda).to(torch.bfloat16)
    k = torch.randn((Nk, Hkv, D), generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn((Nk, Hkv, D), generator=g, device=cuda).to(torch.bfloat16)
    cq = torch.tensor([0] + list(np.cumsum(qlens)), dtype=torch.int32, device=cuda)
    ck = torch.tensor([0] + list(np.cumsum(klens)), dtype=torch.int32, device=cuda)
    nblk = [(n + bs - 1) // bs for n in klens]
    kc = torch.zeros((sum(nblk), bs, Hkv, D), dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    B = len(klens)
    bt = torch.full((B, max(nblk)), -1, dtype=torch.int32, device=cuda)
    o = 0
    for b, (n, m) in enumerate(zip(klens, nblk)):
        bt[b, :m] = torch.arange(o, o + m, dtype=torch.int32)
        s0 = int(ck[b])
        for i in range(m):
            rows = min(bs, n - i * bs)
            kc[o + i, :rows] = k[s0 + i * bs:s0 + i * bs + rows]
            vc[o + i, :rows] = v[s0 + i * bs:s0 + i * bs + rows]
        o += m
    print(f"unpaged vs paged q={qlens} k={klens}", flush=True)
    a = hv.ops.verify_attention(q, k, v, None, cq, ck, max(qlens), max(klens), D ** -0.5)
    p = hv.ops.verify_attention(q, kc, vc, bt, cq, ck, max(qlens), max(klens), D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), p.view(torch.int16))
