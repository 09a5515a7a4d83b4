"""Pins the CPU oracle of the paged verify attention and the FP8 codec.

Independent checks:
  * torch's scaled_dot_product_attention (CPU, float64) on the de-paged keys
    with an explicit bottom-right causal mask;
  * invariance under a permutation of the physical blocks (paging must not
    change the result);
  * closed forms: one visible key returns its value row; equal keys give the
    mean of the values;
  * the e4m3fn codec against torch.float8_e4m3fn (exact decode of all 256
    codes; round-to-nearest-even encode for every representable range).
"""
import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def attn(orc):
    from oracle import attn as A
    return A


def _small_case(hv, **kw):
    args = dict(batch=5, q_len=4, num_q_heads=8, num_kv_heads=2, head_dim=128, block_size=32,
                min_len=4, max_len=150, seed=3)
    args.update(kw)
    return hv.synthetic.attention_workload(**args)


def test_matches_torch_sdpa_on_depaged_keys(hv, attn):
    w = _small_case(hv)
    got = attn.paged_attention(w["q"], w["k_cache"], w["v_cache"], w["block_tables"],
                               w["cu_seqlens_q"], w["cu_seqlens_k"], w["softmax_scale"])
    bs = w["block_size"]
    for b in range(len(w["lens"])):
        Lk, Lq = int(w["lens"][b]), int(w["q_lens"][b])
        pos = np.arange(Lk)
        blk = w["block_tables"][b][pos // bs]
        K = torch.from_numpy(w["k_cache"][blk, pos % bs].astype(np.float64))  # [Lk, Hkv, D]
        V = torch.from_numpy(w["v_cache"][blk, pos % bs].astype(np.float64))
        q0 = int(w["cu_seqlens_q"][b])
        Q = torch.from_numpy(w["q"][q0:q0 + Lq].astype(np.float64))  # [Lq, Hq, D]
        G = Q.shape[1] // K.shape[1]
        Kh = K.repeat_interleave(G, dim=1).permute(1, 0, 2)
        Vh = V.repeat_interleave(G, dim=1).permute(1, 0, 2)
        Qh = Q.permute(1, 0, 2)
        allowed = torch.arange(Lk)[None, :] <= (Lk - Lq + torch.arange(Lq))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            Qh, Kh, Vh, attn_mask=allowed, scale=w["softmax_scale"]).permute(1, 0, 2)
        np.testing.assert_allclose(got[q0:q0 + Lq], ref.numpy(), rtol=1e-10, atol=1e-10)


def test_block_permutation_invariance(hv, attn):
    w = _small_case(hv, seed=4)
    base = attn.paged_attention(w["q"], w["k_cache"], w["v_cache"], w["block_tables"],
                                w["cu_seqlens_q"], w["cu_seqlens_k"], w["softmax_scale"])
    perm = np.random.default_rng(0).permutation(w["num_blocks"])
    inv = np.argsort(perm)
    kc2, vc2 = w["k_cache"][perm], w["v_cache"][perm]
    bt2 = np.where(w["block_tables"] >= 0, inv[np.maximum(w["block_tables"], 0)], -1)
    moved = attn.paged_attention(w["q"], kc2, vc2, bt2, w["cu_seqlens_q"], w["cu_seqlens_k"],
                                 w["softmax_scale"])
    np.testing.assert_array_equal(base, moved)


def test_single_visible_key_returns_value(attn):
    D = 128
    rng = np.random.default_rng(1)
    kc = rng.standard_normal((2, 32, 1, D))
    vc = rng.standard_normal((2, 32, 1, D))
    q = rng.standard_normal((1, 2, D))
    out = attn.paged_attention(q, kc, vc, np.array([[1]]), np.array([0, 1]), np.array([0, 1]),
                               0.1)
    np.testing.assert_allclose(out[0, 0], vc[1, 0, 0])
    np.testing.assert_allclose(out[0, 1], vc[1, 0, 0])


def test_equal_keys_average_values(attn):
    D, L = 128, 20
    rng = np.random.default_rng(2)
    kc = np.broadcast_to(rng.standard_normal((1, 1, 1, D)), (1, 32, 1, D)).copy()
    vc = rng.standard_normal((1, 32, 1, D))
    q = rng.standard_normal((1, 1, D))
    out = attn.paged_attention(q, kc, vc, np.array([[0]]), np.array([0, 1]), np.array([0, L]),
                               0.3)
    np.testing.assert_allclose(out[0, 0], vc[0, :L, 0].mean(0), rtol=1e-12, atol=1e-12)


def test_e4m3fn_decode_matches_torch(attn):
    table = attn.e4m3fn_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(table), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(table[ok], ref[ok])
    assert table[0x7e] == 448.0 and table[0x01] == 2.0 ** -9


def test_e4m3fn_encode_matches_torch_in_range(attn):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-448, 448, 200000), rng.standard_normal(200000) * 1e-2,
                        rng.standard_normal(20000) * 1e-3,
                        attn.e4m3fn_table()[:0x7f].astype(np.float64)]).astype(np.float32)
    # exact midpoints between neighbouring codes exercise ties-to-even
    t = np.sort(attn.e4m3fn_table()[:0x7f].astype(np.float64))
    mids = ((t[1:] + t[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    got = attn.e4m3fn_quantize(x, 1.0)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, ref)


def test_e4m3fn_saturates(attn):
    x = np.array([448.0, 460.0, 1e6, -1e6, np.inf, -np.inf], np.float32)
    got = attn.e4m3fn_quantize(x, 1.0)
    assert got.tolist() == [0x7e, 0x7e, 0x7e, 0xfe, 0x7e, 0xfe]
    assert attn.e4m3fn_quantize(np.array([np.nan], np.float32), 1.0)[0] == 0x7f


def test_cpu_baseline_port_matches_oracle(hv, attn):
    """The torch-CPU fp32 restatement timed as bench.py's attention cpu_baseline computes the
    oracle's result (the NaN-filled slots past each length must stay unread)."""
    from oracle import torch_port
    w = _small_case(hv, seed=5, num_q_heads=16, num_kv_heads=8)
    ref = attn.paged_attention(w["q"], w["k_cache"], w["v_cache"], w["block_tables"],
                               w["cu_seqlens_q"], w["cu_seqlens_k"], w["softmax_scale"])
    got = torch_port.paged_attention(
        torch.from_numpy(w["q"]), torch.from_numpy(w["k_cache"]), torch.from_numpy(w["v_cache"]),
        torch.from_numpy(w["block_tables"]), w["cu_seqlens_q"], w["cu_seqlens_k"],
        w["softmax_scale"]).numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
