"""CPU oracle of the paged verify attention and the KV-cache store (tests only).

TEST INFRASTRUCTURE: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg only.

paged_attention restates the verify branch of Attention.forward,
mini_vllm/layers/attention.py:145-160, i.e. flash_attn_varlen_func over a
paged cache with block_table and causal=True: keys of sequence b are gathered
page by page through block_tables[b], scores are q.k * softmax_scale, the mask
is bottom-right aligned (query i of Lq sees keys 0 .. Lk - Lq + i), softmax and
the value product are evaluated in float64 textbook form.
store_kvcache restates attention.py:59-90 (copy K/V row of token i to slot
slot_mapping[i], skip -1); the FP8 variant quantises with the e4m3fn codec of
attn_oracle.c.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import oracle as _o


def _lib():
    L = _o.lib()
    if not hasattr(L, "_attn_ready"):
        L.or_e4m3fn_decode.argtypes = [ctypes.c_uint8]
        L.or_e4m3fn_decode.restype = ctypes.c_float
        L.or_e4m3fn_encode_sat.argtypes = [ctypes.c_float]
        L.or_e4m3fn_encode_sat.restype = ctypes.c_uint8
        L.or_e4m3fn_quantize.argtypes = [
            np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS"), ctypes.c_int64,
            ctypes.c_float, np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")]
        L.or_e4m3fn_quantize.restype = None
        L._attn_ready = True
    return L


def e4m3fn_table() -> np.ndarray:
    """float32 value of every e4m3fn code (NaN for 0x7f / 0xff)."""
    L = _lib()
    return np.array([L.or_e4m3fn_decode(c) for c in range(256)], np.float32)


def e4m3fn_quantize(x: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    _lib().or_e4m3fn_quantize(x.reshape(-1), x.size, float(scale), out.reshape(-1))
    return out


def dequant(codes: np.ndarray, scale: float) -> np.ndarray:
    return e4m3fn_table()[codes].astype(np.float64) * scale


def paged_attention(q, k_cache, v_cache, block_tables, cu_seqlens_q, cu_seqlens_k,
                    softmax_scale, *, block_size=None):
    """q [N, Hq, D]; caches [nb, bs, Hkv, D] (float, already dequantised);
    block_tables [B, W] int; cu_seqlens_* [B+1]. Returns float64 [N, Hq, D]."""
    q = np.asarray(q, np.float64)
    kc = np.asarray(k_cache, np.float64)
    vc = np.asarray(v_cache, np.float64)
    nb, bs, Hkv, D = kc.shape
    N, Hq, _ = q.shape
    G = Hq // Hkv
    out = np.zeros((N, Hq, D), np.float64)
    B = len(cu_seqlens_q) - 1
    for b in range(B):
        q0, q1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        Lq, Lk = q1 - q0, int(cu_seqlens_k[b + 1] - cu_seqlens_k[b])
        if Lq == 0:
            continue
        pos = np.arange(Lk)
        blocks = np.asarray(block_tables[b])[pos // bs]
        K = kc[blocks, pos % bs]  # [Lk, Hkv, D]
        Vv = vc[blocks, pos % bs]
        qb = q[q0:q1]  # [Lq, Hq, D]
        Kh = np.repeat(K, G, axis=1)  # [Lk, Hq, D]
        Vh = np.repeat(Vv, G, axis=1)
        s = np.einsum("qhd,khd->hqk", qb, Kh) * softmax_scale
        lim = Lk - Lq + np.arange(Lq)
        mask = pos[None, :] > lim[:, None]  # [Lq, Lk]
        s = np.where(mask[None], -np.inf, s)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[q0:q1] = np.einsum("hqk,khd->qhd", p, Vh)
    return out


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """In-place numpy restatement (bf16/f32 caches as arrays of the same dtype)."""
    nb, bs = k_cache.shape[:2]
    for i, slot in enumerate(np.asarray(slot_mapping)):
        if slot < 0:
            continue
        k_cache[slot // bs, slot % bs] = key[i]
        v_cache[slot // bs, slot % bs] = value[i]
