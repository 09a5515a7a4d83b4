"""torch-CPU restatement of the reference acceptance loop (CPU baseline only).

TEST INFRASTRUCTURE: used by bench.py's cpu_baseline leg and by tests that
compare it with the C oracle; never by the product path.

It follows ModelRunner.run_verify's per-sequence loop,
mini_vllm/engine/model_runner.py:391-428, operation by operation on torch
CPU tensors, with torch.rand (:407) and torch.multinomial (:412, :425)
replaced by the explicit uniforms u_accept / u_resample (inverse CDF over the
normalised weights, torch.searchsorted).
"""
from __future__ import annotations

import torch


def _draw(weights: torch.Tensor, u: float) -> tuple[int, float]:
    """Inverse-CDF draw standing in for torch.multinomial (model_runner.py:412,425):
    the first index whose float64 prefix sum exceeds u * total. Also returns the
    distance of u * total to the nearest prefix-sum boundary, relative to the
    total (how far the draw is from flipping to a neighbouring token)."""
    c = torch.cumsum(weights.double(), 0)
    tot = float(c[-1])
    t = u * tot
    i = int(torch.searchsorted(c, torch.tensor([t], dtype=torch.float64), right=True)[0])
    i = min(i, weights.shape[0] - 1)
    hi = float(c[i])
    lo = float(c[i - 1]) if i > 0 else 0.0
    margin = min(abs(hi - t), abs(t - lo)) / tot if tot > 0 else 0.0
    return i, margin


def apply_top_k(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Sampler._apply_top_k (sampler.py:27-37) for rows sharing one k: keep the k
    largest (k <= 0 or k >= V: all), the rest -inf. torch.sort's order among equal
    values is undefined (sampler.py:33); a stable sort keeps the lower index first,
    the tie rule of the C oracle."""
    V = logits.shape[-1]
    if top_k <= 0 or top_k >= V:
        return logits
    sl, si = torch.sort(logits, dim=-1, descending=True, stable=True)
    keep = torch.arange(V).unsqueeze(0) < top_k
    return torch.scatter(torch.empty_like(logits), 1, si, sl.masked_fill(~keep, float("-inf")))


def apply_top_p(logits: torch.Tensor, top_p: float) -> tuple[torch.Tensor, float]:
    """Sampler._apply_top_p (sampler.py:39-49) for rows sharing one p: keep the
    sorted prefix whose cumulative probability is strictly below p, plus rank 0.
    Also returns the smallest |cumsum - p| over the rows (how close the kept set is
    to gaining or losing its boundary element)."""
    if top_p >= 1.0:
        return logits, float("inf")
    sl, si = torch.sort(logits, dim=-1, descending=True, stable=True)
    cum = torch.cumsum(torch.softmax(sl, dim=-1), dim=-1)
    keep = cum < top_p
    keep[:, 0] = True
    margin = float((cum - top_p).abs().min())
    return (torch.scatter(torch.empty_like(logits), 1, si, sl.masked_fill(~keep, float("-inf"))),
            margin)


def run_verify_accept(logits: torch.Tensor, draft_probs: torch.Tensor,
                      draft_tokens: torch.Tensor, temperatures: torch.Tensor,
                      u_accept: torch.Tensor, u_resample: torch.Tensor, *,
                      mode: str = "reference", top_ks=None, top_ps=None, detail: bool = False):
    """logits [B, gamma+1, V], draft_probs [B, gamma, V] -> list[(tokens, n_acc)].

    mode "filtered" applies Sampler's top-k and top-p (sampler.py:20-49) to the
    target rows before the softmax (the draft probabilities are then the filtered
    draft distribution the caller drew the drafts from). With detail=True each
    result gets a third item, the decision margins of that sequence: "accept", the
    smallest |u_j - a_j| over the drafts the loop examined; "draw", the distance of
    the resample point to its nearest CDF boundary (relative); "top_p", the
    smallest |cumsum - p| of the target rows."""
    results = []
    B = logits.shape[0]
    for i in range(B):
        seq_logits = logits[i]
        num_draft = draft_tokens.shape[1]
        temperature = float(temperatures[i])
        x = seq_logits.float() / temperature
        m_top_p = float("inf")
        if mode == "filtered":
            x = apply_top_k(x, int(top_ks[i]))
            x, m_top_p = apply_top_p(x, float(top_ps[i]))
        target_probs = torch.softmax(x, dim=-1)
        draft_tok_ids = draft_tokens[i].to(torch.int64)
        draft_probs_stacked = draft_probs[i]
        p_target = target_probs[:num_draft].gather(1, draft_tok_ids.unsqueeze(1)).squeeze(1)
        p_draft = draft_probs_stacked.gather(1, draft_tok_ids.unsqueeze(1)).squeeze(1)
        accept_probs = torch.clamp(p_target / p_draft.clamp(min=1e-10), max=1.0)
        accepted_mask = u_accept[i] < accept_probs
        if bool(accepted_mask.all()):
            examined = num_draft
            accepted = draft_tok_ids.tolist()
            tok, m_draw = _draw(target_probs[num_draft], float(u_resample[i]))
            accepted.append(tok)
            n_acc = num_draft
        else:
            first_reject = int((~accepted_mask).nonzero(as_tuple=True)[0][0])
            examined = first_reject + 1
            accepted = draft_tok_ids[:first_reject].tolist()
            n_acc = first_reject
            adjusted = torch.clamp(target_probs[first_reject] - draft_probs_stacked[first_reject],
                                   min=0)
            s = adjusted.sum()
            if s > 1e-10:
                adjusted = adjusted / s
            else:
                adjusted = target_probs[first_reject]
            tok, m_draw = _draw(adjusted, float(u_resample[i]))
            accepted.append(tok)
        if detail:
            m_acc = float((u_accept[i][:examined] - accept_probs[:examined]).abs().min())
            results.append((accepted, n_acc, {"accept": m_acc, "draw": m_draw, "top_p": m_top_p}))
        else:
            results.append((accepted, n_acc))
    return results


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_tables: torch.Tensor, cu_seqlens_q, cu_seqlens_k,
                    softmax_scale: float) -> torch.Tensor:
    """torch-CPU fp32 restatement of the verify branch of Attention.forward
    (mini_vllm/layers/attention.py:147-160: flash_attn_varlen_func over the paged
    cache with block_table, causal=True): per sequence, gather its pages, expand
    the KV heads to their query heads and take softmax(Q K^T * scale) V with
    bottom-right causal alignment (query i of Lq sees keys 0 .. Lk - Lq + i).
    q [N, Hq, D]; caches [num_blocks, block_size, Hkv, D]; returns [N, Hq, D]."""
    out = torch.empty_like(q)
    Hq, Hkv = q.shape[1], k_cache.shape[2]
    G = Hq // Hkv
    bs = k_cache.shape[1]
    for b in range(len(cu_seqlens_q) - 1):
        qs, qe = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        Lk = int(cu_seqlens_k[b + 1]) - int(cu_seqlens_k[b])
        Lq = qe - qs
        nblk = (Lk + bs - 1) // bs
        blocks = block_tables[b, :nblk].long()
        k = k_cache[blocks].reshape(-1, Hkv, k_cache.shape[3])[:Lk].repeat_interleave(G, dim=1)
        v = v_cache[blocks].reshape(-1, Hkv, v_cache.shape[3])[:Lk].repeat_interleave(G, dim=1)
        s = torch.matmul(q[qs:qe].transpose(0, 1), k.permute(1, 2, 0).contiguous()) * softmax_scale
        keep = (torch.arange(Lk)[None, :] <= (Lk - Lq + torch.arange(Lq))[:, None])
        s = s.masked_fill(~keep[None], float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[qs:qe] = torch.matmul(p, v.transpose(0, 1).contiguous()).transpose(0, 1)
    return out
