"""Seeded synthetic workloads of the verify path (numpy, host side).

The shapes and distributions follow the benchmark configurations of the verify
path: config 0 (one sequence, fp32 logits), config 1 (batched bf16 logits with
per-sequence sampling settings) and config 2 (paged attention). Arrays come
from numpy's PCG64 generator so the same seed gives the same bytes on every
machine; `digest()` fingerprints a workload.
"""
from __future__ import annotations

import hashlib

import numpy as np

VOCAB = 151936


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even bf16 bit patterns of float32 values (NaN stays NaN).
    Works in place on a uint32 copy, 4M elements at a time."""
    u = np.array(x, dtype=np.float32, copy=True, order="C").view(np.uint32).reshape(-1)
    out = np.empty(u.shape, np.uint16)
    step = 1 << 22
    for a in range(0, u.size, step):
        c = u[a:a + step]
        nan = (c & 0x7FFFFFFF) > 0x7F800000
        r = c >> 16
        r &= 1
        r += 0x7FFF
        c += r  # finite values cannot carry past bit 31: |x| <= 0x7F7FFFFF
        c >>= 16
        c[nan] = 0x7FC0
        out[a:a + step] = c
    return out.reshape(np.shape(x))


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def softmax64(x: np.ndarray) -> np.ndarray:
    z = x.astype(np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=-1, keepdims=True)


def filtered_probs64(logits: np.ndarray, temperature: float, top_k: int, top_p: float):
    """float64 top-k / top-p distribution of one row (draft-side input only).

    Rank order is descending x = logit / T with ties broken by lower index; top-k
    keeps the first k ranks, top-p the ranks whose cumulative probability (over the
    top-k set) is below p, and rank 0. Only the candidates above a partition
    threshold are sorted, grown until they hold the top-p crossing."""
    x = logits.astype(np.float64) / temperature
    V = x.shape[-1]
    keep = np.ones(V, bool)
    if 0 < top_k < V:
        thr = np.partition(x, V - top_k)[V - top_k]  # k-th largest value
        above = np.flatnonzero(x > thr)
        ties = np.flatnonzero(x == thr)[:top_k - above.size]
        keep[:] = False
        keep[above] = True
        keep[ties] = True
    if top_p < 1.0:
        z = np.where(keep, x, -np.inf)
        e = np.exp(z - z.max())
        total = e.sum()
        nkeep = int(keep.sum())
        n = min(nkeep, 4096)
        while True:
            if n >= nkeep:
                cand = np.flatnonzero(keep)
            else:
                cand = np.flatnonzero(z > np.partition(z, V - n)[V - n])
            order = cand[np.lexsort((cand, -z[cand]))]
            ks = np.cumsum(e[order]) / total < top_p
            if not ks.all() or cand.size == nkeep:
                break
            n *= 4
        ks[0] = True
        keep[:] = False
        keep[order[ks]] = True
    z = np.where(keep, x, -np.inf)
    e = np.exp(z - z.max())
    return e / e.sum()


def _inv_cdf(p: np.ndarray, u: float) -> int:
    c = np.cumsum(p)
    return int(min(np.searchsorted(c, u * c[-1], side="right"), p.shape[0] - 1))


def accept_workload(batch: int, gamma: int, vocab: int = VOCAB, seed: int = 0,
                    dtype: str = "f32", temperature=1.0, top_k=0, top_p=1.0,
                    per_seq_settings: bool = False, mode: str = "reference") -> dict:
    """Inputs of one fused acceptance call.

    Target logits ~ N(0, 2^2) [B, gamma+1, V]; draft logits = target[:, :gamma]
    + N(0, 1). Draft probabilities are the draft distribution (filtered in
    filtered mode) and the draft tokens are drawn from it. Uniforms u_accept
    [B, gamma] and u_resample [B] come from the same seeded stream.
    With per_seq_settings, T ~ U[0.5, 1.2], top_k in {0, 20, 50} and
    top_p in {1.0, 0.9, 0.8} per sequence.
    dtype "bf16" rounds the logits to bf16 (logits_bits holds the patterns).
    """
    rng = _rng(seed)
    target = (rng.standard_normal((batch, gamma + 1, vocab), dtype=np.float32) * 2.0)
    noise = rng.standard_normal((batch, gamma, vocab), dtype=np.float32)
    draft = target[:, :gamma] + noise
    if dtype == "bf16":
        tb = f32_to_bf16_bits(target)
        target = bf16_bits_to_f32(tb)
        draft = bf16_bits_to_f32(f32_to_bf16_bits(draft))
    else:
        tb = None
    if per_seq_settings:
        temps = rng.uniform(0.5, 1.2, size=batch).astype(np.float32)
        top_ks = rng.choice(np.array([0, 20, 50], np.int32), size=batch)
        top_ps = rng.choice(np.array([1.0, 0.9, 0.8], np.float32), size=batch)
    else:
        temps = np.full(batch, temperature, np.float32)
        top_ks = np.full(batch, top_k, np.int32)
        top_ps = np.full(batch, top_p, np.float32)
    q = np.empty((batch, gamma, vocab), np.float32)
    dtok = np.empty((batch, gamma), np.int64)
    for b in range(batch):
        for j in range(gamma):
            if mode == "filtered":
                p = filtered_probs64(draft[b, j], float(temps[b]), int(top_ks[b]),
                                     float(top_ps[b]))
            else:
                p = softmax64(draft[b, j] / np.float64(temps[b]))
            q[b, j] = p.astype(np.float32)
            dtok[b, j] = _inv_cdf(p, rng.random())
    u_acc = rng.random((batch, gamma), dtype=np.float32)
    u_res = rng.random(batch, dtype=np.float32)
    return dict(logits=target.astype(np.float32), logits_bits=tb, draft_probs=q,
                draft_tokens=dtok, temperatures=temps, top_ks=top_ks.astype(np.int32),
                top_ps=top_ps.astype(np.float32), u_accept=u_acc, u_resample=u_res,
                dtype=dtype, mode=mode)


def digest(arrays: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(arrays):
        v = arrays[k]
        if isinstance(v, np.ndarray):
            h.update(k.encode())
            h.update(np.ascontiguousarray(v).tobytes())
    return h.hexdigest()


def attention_workload(batch: int = 64, q_len: int = 4, num_q_heads: int = 16,
                       num_kv_heads: int = 8, head_dim: int = 128, block_size: int = 256,
                       min_len: int = 64, max_len: int = 2048, seed: int = 0,
                       spare_blocks: int = 3, lens=None) -> dict:
    """Paged verify attention inputs (config 2 by default).

    Context lengths Lk ~ U[min_len, max_len] (or `lens`), q_len query tokens per
    sequence (the last q_len positions), blocks of block_size tokens assigned
    by a random permutation; Q, K, V ~ N(0, 1) rounded to bf16. Cache slots
    past each sequence's length hold NaN so reads beyond Lk are detectable.
    """
    rng = _rng(seed)
    if lens is None:
        lens = rng.integers(min_len, max_len + 1, size=batch)
    lens = np.asarray(lens, np.int64)
    q_lens = np.minimum(np.full(batch, q_len, np.int64), lens)
    nblk = (lens + block_size - 1) // block_size
    num_blocks = int(nblk.sum()) + spare_blocks
    perm = rng.permutation(num_blocks).astype(np.int32)
    W = int(nblk.max())
    bt = np.full((batch, W), -1, np.int32)
    off = 0
    for b in range(batch):
        bt[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += nblk[b]
    kc = rng.standard_normal((num_blocks, block_size, num_kv_heads, head_dim), dtype=np.float32)
    vc = rng.standard_normal((num_blocks, block_size, num_kv_heads, head_dim), dtype=np.float32)
    kc = bf16_bits_to_f32(f32_to_bf16_bits(kc))
    vc = bf16_bits_to_f32(f32_to_bf16_bits(vc))
    for b in range(batch):
        last = bt[b, nblk[b] - 1]
        used = lens[b] - (nblk[b] - 1) * block_size
        kc[last, used:] = np.nan
        vc[last, used:] = np.nan
    N = int(q_lens.sum())
    q = bf16_bits_to_f32(f32_to_bf16_bits(
        rng.standard_normal((N, num_q_heads, head_dim), dtype=np.float32)))
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return dict(q=q, k_cache=kc, v_cache=vc, block_tables=bt, cu_seqlens_q=cu_q,
                cu_seqlens_k=cu_k, max_seqlen_q=int(q_lens.max()), max_seqlen_k=int(lens.max()),
                softmax_scale=float(head_dim) ** -0.5, lens=lens, q_lens=q_lens,
                num_blocks=num_blocks, block_size=block_size)
