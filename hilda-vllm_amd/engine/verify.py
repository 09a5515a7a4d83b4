"""Drop-in for ModelRunner.run_verify and ModelRunner.cleanup_rejected_kv_slots.

Same call shapes as mini_vllm/engine/model_runner.py:321-437 and :439-481:

    results = runner.run_verify(seqs, draft_tokens, draft_probs)
    # results[i] == (accepted_token_ids incl. the bonus token, num_accepted_drafts)
    runner.cleanup_rejected_kv_slots(seqs, results, gamma)

What changes underneath:
  * staging (model_runner.py:337-362) is vectorised per sequence into pinned
    host buffers and copied once;
  * the per-sequence softmax / gather / rejection loop with its D2H syncs
    (:387-428) becomes one hs_spec_accept launch chain over [B, gamma+1, V]
    target logits and [B, gamma, V] draft probabilities, followed by one D2H
    copy of the packed results;
  * torch.rand (:407) and torch.multinomial (:412, :425) are replaced by
    explicit uniforms, drawn on the device with torch.rand unless the caller
    passes them (uniforms=(u_accept [B, gamma], u_resample [B])).
Sequences with different draft counts are verified in groups of equal count.
A sequence without drafts samples its bonus token from P[0] (:410-414 with an
empty draft list).

cleanup_rejected_kv_slots zeroes whole token rows (all KV heads) of the slots
in the reference's position range [len, old_len + gamma + 1) in every bound
cache. The reference indexes a [tokens*heads, D] view with the slot id
(:471-481), which zeroes one head row of another token; the intent stated in
its docstring (zero the rejected tokens' KV) is what is implemented here.
"""
from __future__ import annotations

from time import perf_counter

import numpy as np
import torch

from .. import ops as _ops
from ..utils.context import reset_context, set_context


class VerifyRunner:
    """Holds the preallocated staging buffers of the verify step
    (model_runner.py:504-549) and the caches cleanup zeroes."""

    def __init__(self, model, *, block_size: int = 256, max_num_seqs: int = 256,
                 max_gamma: int = 8, mode: str = "reference", kv_caches=(),
                 device: torch.device | str = "cuda", record_breakdown: bool = True):
        if mode not in ("reference", "filtered"):
            raise ValueError("mode must be 'reference' or 'filtered' (temperature 0 selects greedy)")
        self.model = model
        self.block_size = int(block_size)
        self.mode = mode
        self.kv_caches = list(kv_caches)
        self.device = torch.device(device)
        self.record_breakdown = record_breakdown
        self.max_num_seqs = int(max_num_seqs)
        self.max_gamma = int(max_gamma)
        n = self.max_num_seqs * (self.max_gamma + 1)
        pin = torch.cuda.is_available()
        self.cpu = {
            "input_ids": torch.zeros(n, dtype=torch.int64, pin_memory=pin),
            "positions": torch.zeros(n, dtype=torch.int64, pin_memory=pin),
            "slot_mapping": torch.zeros(n, dtype=torch.int32, pin_memory=pin),
            "cu_seqlens_q": torch.zeros(self.max_num_seqs + 1, dtype=torch.int32, pin_memory=pin),
            "cu_seqlens_k": torch.zeros(self.max_num_seqs + 1, dtype=torch.int32, pin_memory=pin),
        }
        self.gpu = {k: torch.zeros_like(v, device=self.device) for k, v in self.cpu.items()}
        self.last_verify_breakdown: dict[str, float] = {}
        self.last_logits: torch.Tensor | None = None

    # -- staging (model_runner.py:337-362, :586-612) --------------------------------------
    def _stage(self, seqs, draft_tokens):
        cpu = self.cpu
        ids = cpu["input_ids"].numpy()
        pos = cpu["positions"].numpy()
        slots = cpu["slot_mapping"].numpy()
        cq = cpu["cu_seqlens_q"].numpy()
        ck = cpu["cu_seqlens_k"].numpy()
        bs = self.block_size
        total = 0
        max_q = max_k = 0
        cq[0] = ck[0] = 0
        verify_lens = []
        for i, seq in enumerate(seqs):
            toks = [seq.last_token] + list(draft_tokens[i])
            R = len(toks)
            start = len(seq) - 1
            p = np.arange(start, start + R, dtype=np.int64)
            bt = np.asarray(seq.block_table, dtype=np.int64)
            bi = p // bs
            ok = bi < bt.shape[0]
            s = np.full(R, -1, dtype=np.int64)
            s[ok] = bt[bi[ok]] * bs + p[ok] % bs
            ids[total:total + R] = toks
            pos[total:total + R] = p
            slots[total:total + R] = s
            total += R
            cq[i + 1] = total
            ck[i + 1] = ck[i] + start + R
            max_q = max(max_q, R)
            max_k = max(max_k, start + R)
            verify_lens.append(R)
        B = len(seqs)
        gpu = self.gpu
        for k, n in (("input_ids", total), ("positions", total), ("slot_mapping", total),
                     ("cu_seqlens_q", B + 1), ("cu_seqlens_k", B + 1)):
            gpu[k][:n].copy_(cpu[k][:n], non_blocking=True)
        width = max(len(s.block_table) for s in seqs)
        bt = torch.full((B, max(width, 1)), -1, dtype=torch.int32)
        for i, s in enumerate(seqs):
            if s.block_table:
                bt[i, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32)
        block_tables = bt.to(self.device, non_blocking=False)
        return total, max_q, max_k, verify_lens, block_tables

    def _sync(self):
        if self.record_breakdown:
            torch.cuda.synchronize(self.device)

    def _lm_head(self):
        w = getattr(self.model, "lm_head")
        return getattr(w, "weight", w)

    @torch.inference_mode()
    def run_verify(self, seqs, draft_tokens, draft_probs, uniforms=None):
        """model_runner.py:321-437. draft_probs: per sequence a list of gamma f32 [V]
        rows (the reference's layout) or one [B, gamma, V] f32 tensor."""
        B = len(seqs)
        if B == 0:
            return []
        if B > self.max_num_seqs:
            raise ValueError(f"{B} sequences exceed max_num_seqs={self.max_num_seqs}")
        if len(draft_tokens) != B:
            raise ValueError("one draft token list per sequence")
        gmax = max(len(d) for d in draft_tokens)
        if gmax > self.max_gamma:
            raise ValueError(f"{gmax} drafts exceed max_gamma={self.max_gamma}")
        t0 = perf_counter()
        total, max_q, max_k, verify_lens, block_tables = self._stage(seqs, draft_tokens)
        self._sync()
        prep = perf_counter() - t0

        t0 = perf_counter()
        gpu = self.gpu
        set_context(True, gpu["cu_seqlens_q"][:B + 1], gpu["cu_seqlens_k"][:B + 1], max_q, max_k,
                    gpu["slot_mapping"][:total], None, block_tables)
        try:
            hidden = self.model(gpu["input_ids"][:total], gpu["positions"][:total])
        finally:
            reset_context()
        self._sync()
        fwd = perf_counter() - t0

        t0 = perf_counter()
        # logits for every verify token (model_runner.py:380-383)
        logits = _ops.linear(hidden, self._lm_head())
        self._sync()
        lmh = perf_counter() - t0
        self.last_logits = logits

        t0 = perf_counter()
        results = self._accept(seqs, draft_tokens, draft_probs, logits, verify_lens, uniforms)
        samp = perf_counter() - t0
        self.last_verify_breakdown = {"prep_time_s": prep, "forward_time_s": fwd,
                                      "lmhead_time_s": lmh, "sampling_time_s": samp}
        return results

    # -- acceptance (model_runner.py:387-428) -----------------------------------------------
    def _accept(self, seqs, draft_tokens, draft_probs, logits, verify_lens, uniforms):
        dev = self.device
        B = len(seqs)
        V = logits.shape[-1]
        temps_l = [float(s.temperature) for s in seqs]
        greedy = all(t == 0.0 for t in temps_l)
        if not greedy and any(t <= 0.0 for t in temps_l):
            raise ValueError("temperature 0 (greedy) cannot be mixed with sampling in one batch")
        offsets = np.concatenate([[0], np.cumsum(verify_lens)])
        groups: dict[int, list[int]] = {}
        for i, d in enumerate(draft_tokens):
            groups.setdefault(len(d), []).append(i)
        temps = torch.tensor(temps_l, dtype=torch.float32).to(dev, non_blocking=True)
        topk_le64 = False
        if self.mode == "filtered":
            ks = [int(s.top_k) for s in seqs]
            tks = torch.tensor(ks, dtype=torch.int32).to(dev)
            tps = torch.tensor([float(s.top_p) for s in seqs], dtype=torch.float32).to(dev)
            topk_le64 = all(1 <= k <= 64 for k in ks)
        if uniforms is not None:
            u_acc_all, u_res_all = uniforms
            u_acc_all = torch.as_tensor(u_acc_all, dtype=torch.float32).to(dev)
            u_res_all = torch.as_tensor(u_res_all, dtype=torch.float32).to(dev).reshape(B)
        else:
            u_acc_all = torch.rand((B, max(max(groups), 1)), device=dev)
            u_res_all = torch.rand(B, device=dev)
        packed = torch.empty((B, self.max_gamma + 2), dtype=torch.int64, device=dev)
        packed.fill_(-1)
        for g, idx in groups.items():
            ix = torch.tensor(idx, dtype=torch.int64, device=dev)
            contiguous = idx == list(range(idx[0], idx[0] + len(idx)))
            if contiguous:
                lo, hi = int(offsets[idx[0]]), int(offsets[idx[-1] + 1])
                lg = logits[lo:hi].view(len(idx), g + 1, V)
            else:
                rows = np.concatenate([np.arange(offsets[i], offsets[i + 1]) for i in idx])
                lg = logits[torch.from_numpy(rows).to(dev)].view(len(idx), g + 1, V)
            if g == 0:
                r = _ops.sample_rows(lg[:, 0], temps[ix], mode="greedy" if greedy else "reference",
                                     uniforms=u_res_all[ix])
                packed[ix, 0] = r["tokens"]
                packed[ix, -1] = 0
                continue
            dt = torch.tensor([draft_tokens[i] for i in idx], dtype=torch.int64).to(dev)
            if greedy:
                q = None
            elif isinstance(draft_probs, torch.Tensor):
                q = draft_probs[ix, :g] if not contiguous or len(idx) != B else draft_probs[:, :g]
            else:
                q = torch.stack([torch.stack(list(draft_probs[i])) for i in idx])
            if q is not None:
                q = q.to(torch.float32)
            mode = "greedy" if greedy else self.mode
            nacc, out, _ = _ops.spec_accept(
                lg, q, dt, temps[ix], u_acc_all[ix, :g], u_res_all[ix], mode=mode,
                top_ks=tks[ix] if mode == "filtered" else None,
                top_ps=tps[ix] if mode == "filtered" else None,
                topk_le64=topk_le64 and mode == "filtered")
            packed[ix, :g + 1] = out
            packed[ix, -1] = nacc.to(torch.int64)
        host = packed.cpu().numpy()  # the one D2H copy (synchronises)
        # a negative count marks outputs the kernel could not produce (a bounded
        # wait ran out): committing them would silently drop the step's tokens
        _ops.check_accepted(torch.from_numpy(host[:, -1]), "run_verify")
        results = []
        for b in range(B):
            row = host[b]
            n = int(row[-1])
            results.append(([int(t) for t in row[:n + 1]], n))
        return results

    # -- dirty-slot zeroing (model_runner.py:439-481) ---------------------------------------
    @torch.inference_mode()
    def cleanup_rejected_kv_slots(self, seqs, verify_results, gamma: int) -> list[int]:
        """Zero the KV rows of positions [len(seq), old_len + gamma + 1) (old_len = length
        before the accepted tokens were appended) in every cache in self.kv_caches.
        Returns the slot ids it zeroed."""
        bs = self.block_size
        dirty: list[int] = []
        for seq, (accepted, _n) in zip(seqs, verify_results):
            kept = len(accepted)
            cur = len(seq)
            old = cur - kept
            for p in range(old + kept, old + gamma + 1):
                if p < 0:
                    continue
                bi = p // bs
                if bi < len(seq.block_table):
                    dirty.append(seq.block_table[bi] * bs + p % bs)
        if dirty:
            slots = torch.tensor(dirty, dtype=torch.int32).to(self.device)
            for cache in self.kv_caches:
                _ops.zero_kv_slots(cache, slots)
        return dirty
