"""hs_verify_attention_noalloc against hs_verify_attention, through the C ABI.

The allocation-free entry point keeps the partial results of key splits and of
the balanced launch in the library's fixed per-GPU scratch instead of a
caller workspace. Its outputs must equal those of hs_verify_attention (same
kernels, same launch choice) bit for bit, over consecutive calls that share
the scratch, the later ones smaller; a call whose partials exceed the scratch
must be rejected before anything is launched.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bf16(hv, x, dev):
    bits = hv.synthetic.f32_to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)


def _inputs(hv, w, dev):
    return dict(q=_bf16(hv, w["q"], dev), kc=_bf16(hv, w["k_cache"], dev),
                vc=_bf16(hv, w["v_cache"], dev),
                bt=torch.from_numpy(w["block_tables"]).to(dev),
                cq=torch.from_numpy(w["cu_seqlens_q"]).to(dev),
                ck=torch.from_numpy(w["cu_seqlens_k"]).to(dev),
                max_q=w["max_seqlen_q"], max_k=w["max_seqlen_k"], scale=w["softmax_scale"])


def _noalloc(hv, t, out):
    q, kc, vc, bt = t["q"], t["kc"], t["vc"], t["bt"]
    nb, bs, Hkv, D = kc.shape
    N, Hq, _ = q.shape
    B = t["cq"].numel() - 1
    stream = torch.cuda.current_stream(q.device).cuda_stream
    return hv._lib.lib().hs_verify_attention_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), hv._lib.HS_BF16,
        kc.stride(0), kc.stride(1), kc.stride(2), 1.0, 1.0, bt.data_ptr(), bt.stride(0),
        bt.shape[1], nb, t["cq"].data_ptr(), t["ck"].data_ptr(), B, int(t["max_q"]),
        int(t["max_k"]), Hq, Hkv, D, bs, float(t["scale"]), out.data_ptr(), out.stride(0),
        out.stride(1), ctypes.c_void_p(stream))


def test_noalloc_matches_workspace_entry_point(hv, cuda):
    """Three calls in a row on the shared scratch, each smaller than the one before:
    config 2 (B = 64, the balanced launch, ~32 MiB of partials), two 8192/3000-key
    sequences (per-tile grid with key splits), and the batch-1 verify shape (no
    partials)."""
    lib = hv._lib.lib()
    assert lib.hs_verify_attention_noalloc_scratch_bytes() == 34 << 20
    cases = [
        ("config2 B=64", dict(seed=0)),
        ("B=2 long", dict(batch=2, q_len=4, num_q_heads=32, num_kv_heads=8, lens=[8192, 3000],
                          seed=1)),
        ("B=1 verify", dict(batch=1, q_len=4, num_q_heads=32, num_kv_heads=8, lens=[324],
                            seed=2)),
    ]
    for name, kw in cases:
        print(f"noalloc vs workspace entry point: {name}", flush=True)
        w = hv.synthetic.attention_workload(**kw)
        t = _inputs(hv, w, cuda)
        ref = hv.ops.verify_attention(t["q"], t["kc"], t["vc"], t["bt"], t["cq"], t["ck"],
                                      t["max_q"], t["max_k"], t["scale"])
        out = torch.full_like(ref, float("nan"))
        rc = _noalloc(hv, t, out)
        assert rc == 0, lib.hs_status_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), name
        assert torch.isfinite(out.float()).all()


def test_noalloc_rejects_calls_beyond_the_scratch(hv, cuda):
    """A long prefill (8192 queries over 8192 keys) needs ~272 MB of split partials:
    the entry point returns HS_ERR_SCRATCH_LIMIT and launches nothing (the output
    keeps its contents)."""
    lib = hv._lib.lib()
    Hq, Hkv, D, bs, L = 32, 8, 128, 256, 8192
    nb = L // bs
    t = dict(q=torch.zeros((L, Hq, D), dtype=torch.bfloat16, device=cuda),
             kc=torch.zeros((nb, bs, Hkv, D), dtype=torch.bfloat16, device=cuda),
             vc=torch.zeros((nb, bs, Hkv, D), dtype=torch.bfloat16, device=cuda),
             bt=torch.arange(nb, dtype=torch.int32, device=cuda).view(1, nb),
             cq=torch.tensor([0, L], dtype=torch.int32, device=cuda),
             ck=torch.tensor([0, L], dtype=torch.int32, device=cuda),
             max_q=L, max_k=L, scale=D ** -0.5)
    need = lib.hs_verify_attention_workspace_size(1, Hq, Hkv, L, L)
    assert need > lib.hs_verify_attention_noalloc_scratch_bytes()
    out = torch.full((L, Hq, D), 7.0, dtype=torch.bfloat16, device=cuda)
    rc = _noalloc(hv, t, out)
    torch.cuda.synchronize()
    assert rc == hv._lib.HS_ERR_SCRATCH_LIMIT, rc
    assert b"scratch" in lib.hs_status_string(rc)
    assert bool((out == 7.0).all())
    # the scratch is still usable afterwards
    w = hv.synthetic.attention_workload(batch=3, q_len=4, num_q_heads=16, num_kv_heads=8,
                                        lens=[100, 2000, 5000], seed=3)
    t = _inputs(hv, w, cuda)
    ref = hv.ops.verify_attention(t["q"], t["kc"], t["vc"], t["bt"], t["cq"], t["ck"],
                                  t["max_q"], t["max_k"], t["scale"])
    out = torch.empty_like(ref)
    assert _noalloc(hv, t, out) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
