"""Speculative-decoding runner on one MI355X.

Restates the spec path of mini_vllm/engine/model_runner.py (KV-cache
allocation and binding :141-247, run_draft_prefill :249-279, run_draft_decode
:281-319, run_verify :321-437) and of LLMEngine.step (llm_engine.py:104-208)
around the gfx950 kernels:
  * all per-step bookkeeping is device-resident (hs_spec_prealloc,
    hs_draft_prepare, hs_verify_prepare, hs_spec_commit), so a step needs no
    host staging loop and no host synchronisation;
  * the draft loop samples each draft token and writes the draft
    probabilities with one hs_sampler call per step;
  * verify runs the target over gamma+1 tokens, the LM head over all rows and
    the fused acceptance (hs_spec_accept) with explicit uniforms;
  * the draft phase and the verify phase can each be captured once into a HIP
    graph and replayed (one pair of graphs per gamma);
  * with adaptive=True gamma follows the acceptance-rate controller of
    llm_engine.py:197-208 (AdaptiveGamma); the step's accepted/proposed
    totals are read back after every step, as the reference does on the host.
Uniforms are drawn on the device from torch's generator (graph-safe).
"""
from __future__ import annotations

import math

import torch

from types import SimpleNamespace

from .. import ops
from ..layers.sampler import Sampler
from ..utils.context import reset_context, set_context
from .adaptive_gamma import AdaptiveGamma


class SpecRunner:

    def __init__(self, target, draft, *, batch: int, gamma: int, max_model_len: int = 4096,
                 block_size: int = 256, kv_cache_dtype: str = "auto", num_blocks: int | None = None,
                 temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
                 mode: str = "reference", eos: int = -1, k_scale: float | None = None,
                 v_scale: float | None = None, device="cuda", adaptive: bool = False,
                 max_gamma: int | None = None, chain_steps: bool | None = None):
        filters = 0 < top_k < target.g.vocab or top_p < 1.0
        # reference mode with top-k / top-p draws the draft tokens from the filtered
        # Sampler and keeps the unfiltered softmax as the draft probabilities
        # (model_runner.py:312-313): hs_sampler's output kind 2 gives both in one
        # call; the acceptance compares against the unfiltered target (:398)
        self.draft_out_kind = 2 if (mode == "reference" and filters) else 0
        self.draft_mode = "filtered" if (mode == "filtered" or self.draft_out_kind) else "reference"
        self.target, self.draft = target, draft
        self.B, self.gamma = batch, gamma
        self.max_gamma = max(gamma, max_gamma or (8 if adaptive else gamma))
        self.bs = block_size
        self.max_model_len = max_model_len
        self.W = math.ceil((max_model_len + self.max_gamma + 2) / block_size)
        self.num_blocks = num_blocks or batch * self.W + 2
        self.mode = mode
        # index-qualified ("cuda" -> "cuda:<current>"), so per-device lookups such
        # as ops.accept_error find the workspaces the kernels were given
        self.device = torch.device("cuda", ops._dev_index(device))
        self.V = target.g.vocab
        dev = self.device
        kv_dtype = torch.float8_e4m3fn if kv_cache_dtype == "fp8" else torch.bfloat16
        tg, dg = target.g, draft.g
        self.kv = torch.zeros((2, len(target.layers), self.num_blocks, block_size,
                               tg.num_kv_heads, tg.head_dim), dtype=kv_dtype, device=dev)
        self.dkv = torch.zeros((2, len(draft.layers), self.num_blocks, block_size,
                                dg.num_kv_heads, dg.head_dim), dtype=torch.bfloat16, device=dev)
        kmax = max_model_len + self.max_gamma + 2
        # FP8 per-tensor scales: given, or calibrated from the prompt by prefill()
        self.kv_calibrate = kv_cache_dtype == "fp8" and k_scale is None and v_scale is None
        for i, a in enumerate(target.attention_layers()):
            a.k_cache, a.v_cache = self.kv[0, i], self.kv[1, i]
            a.kv_cache_dtype = kv_cache_dtype
            a.k_scale = 1.0 if k_scale is None else float(k_scale)
            a.v_scale = 1.0 if v_scale is None else float(v_scale)
            a.max_model_len = kmax
        for i, a in enumerate(draft.attention_layers()):
            a.k_cache, a.v_cache = self.dkv[0, i], self.dkv[1, i]
            a.kv_cache_dtype = "auto"
            a.max_model_len = kmax
        self.state = ops.SpecStateTensors(batch, self.W, kmax + 1, self.num_blocks, block_size,
                                          eos, dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.temps = torch.full((batch,), float(temperature), **f32)
        self.top_ks = torch.full((batch,), int(top_k), dtype=torch.int32, device=dev)
        self.top_ps = torch.full((batch,), float(top_p), **f32)
        self.topk_le64 = mode == "filtered" and 1 <= int(top_k) <= 64
        self.tok_scratch = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.d_stage = self._stage_bufs(batch)
        self.d_stage0 = self._stage_bufs(2 * batch)
        self.sampler = Sampler()
        self._per_gamma: dict[int, SimpleNamespace] = {}
        self.controller = AdaptiveGamma(gamma, max_gamma=self.max_gamma) if adaptive else None
        # fixed gamma: each step's commit also pre-allocates the next step and stages its
        # first draft step (hs_spec_commit_next), so the next draft phase starts with
        # the draft forward; _staged says the state already holds that
        self.chain_steps = (not adaptive) if chain_steps is None else bool(chain_steps)
        if self.chain_steps and adaptive:
            raise ValueError("chained steps need a fixed gamma (the next step's gamma is "
                             "known when the commit runs)")
        self._staged = False
        # one sequence: the commit also stages the next verify step (all but the
        # draft tokens' ids, which the draft steps write straight into the verify
        # input ids), so the verify phase starts with the target forward
        self._stage_verify = self.chain_steps and batch == 1
        self.history: list[tuple[int, int, int]] = []  # (gamma, accepted, proposed) per step
        self.preempted: list[int] = []  # sequences out of the batch until readmit(), next first
        self.last = None

    def _g(self, gamma: int | None = None) -> SimpleNamespace:
        """Buffers (and graphs) of one gamma: draft tokens [B, g], draft probabilities
        [B, g, V], uniforms, eligibility and the last acceptance outputs."""
        g = self.gamma if gamma is None else gamma
        G = self._per_gamma.get(g)
        if G is None:
            dev, B = self.device, self.B
            # every uniform of a step in one buffer, drawn by one launch at the start
            # of the draft phase: the draft steps' draws [g, B], the acceptance
            # uniforms [B, g] and the resample uniforms [B]
            u_all = torch.zeros(2 * g * B + B, dtype=torch.float32, device=dev)
            v_stage = self._stage_bufs(B * (g + 1))
            # one sequence: the draft tokens are rows 1 .. g of the verify input ids
            draft_tokens = (v_stage[0].view(1, g + 1)[:, 1:] if B == 1 else
                            torch.zeros((B, g), dtype=torch.int64, device=dev))
            G = SimpleNamespace(
                gamma=g,
                v_stage=v_stage,
                draft_tokens=draft_tokens,
                draft_probs=torch.zeros((B, g, self.V), dtype=torch.float32, device=dev),
                u_all=u_all,
                u_draft=u_all[:g * B].view(g, B),
                u_acc=u_all[g * B:2 * g * B].view(B, g),
                u_res=u_all[2 * g * B:],
                elig=torch.zeros(B, dtype=torch.int32, device=dev),
                graphs=None, last=None, graph_last=None, logits=None, graph_logits=None)
            self._per_gamma[g] = G
        return G

    # buffers of the current gamma (the fixed-gamma interface)
    @property
    def u_res(self):
        return self._g().u_res

    @property
    def draft_tokens(self):
        return self._g().draft_tokens

    @property
    def draft_probs(self):
        return self._g().draft_probs

    @property
    def graphs(self):
        return self._g().graphs

    def _stage_bufs(self, rows):
        dev = self.device
        return (torch.zeros(rows, dtype=torch.int64, device=dev),
                torch.zeros(rows, dtype=torch.int64, device=dev),
                torch.zeros(rows, dtype=torch.int32, device=dev),
                torch.zeros(self.B + 1, dtype=torch.int32, device=dev),
                torch.zeros(self.B + 1, dtype=torch.int32, device=dev))

    # ------------------------------------------------------------------ setup
    def load_prompts(self, prompts: list[list[int]], max_tokens: int = 1 << 30,
                     ignore_eos: bool = True):
        """Allocates prompt blocks from the front of the free list (block_manager.py:59-82
        without prefix reuse: random prompts never share a full block)."""
        assert len(prompts) == self.B
        self._staged = False
        st = self.state
        free = list(range(self.num_blocks))
        tables, nblk = [], []
        for p in prompts:
            n = math.ceil(len(p) / self.bs)
            tables.append(free[:n])
            free = free[n:]
            nblk.append(n)
        dev = self.device
        bt = torch.full((self.B, self.W), -1, dtype=torch.int32)
        tok = torch.zeros((self.B, st.T), dtype=torch.int64)
        for i, (p, t) in enumerate(zip(prompts, tables)):
            bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
            tok[i, :len(p)] = torch.tensor(p, dtype=torch.int64)
        st.block_tables.copy_(bt)
        st.tokens.copy_(tok)
        st.num_seq_blocks.copy_(torch.tensor(nblk, dtype=torch.int32))
        st.context_lens.copy_(torch.tensor([len(p) for p in prompts], dtype=torch.int32))
        st.num_prompt.copy_(torch.tensor([len(p) for p in prompts], dtype=torch.int32))
        st.max_tokens.fill_(max_tokens)
        st.ignore_eos.fill_(int(ignore_eos))
        st.finished.zero_()
        ring = torch.zeros(self.num_blocks, dtype=torch.int32)
        ring[:len(free)] = torch.tensor(free, dtype=torch.int32)
        st.free_ring.copy_(ring)
        st.free_hdr.copy_(torch.tensor([0, len(free)], dtype=torch.int32))
        ref = torch.zeros(self.num_blocks, dtype=torch.int32)
        for t in tables:
            ref[t] = 1
        st.ref_count.copy_(ref)
        st.block_hash.fill_(-1)  # the first commit hashes the full prompt blocks
        self.prompts = prompts
        del dev

    @torch.inference_mode()
    def prefill(self):
        """Target prefill + first token, then draft prefill (model_runner.py:249-279)."""
        dev = self.device
        lens = [len(p) for p in self.prompts]
        ids = torch.tensor([t for p in self.prompts for t in p], dtype=torch.int64, device=dev)
        pos = torch.tensor([i for n in lens for i in range(n)], dtype=torch.int64, device=dev)
        bt = self.state.block_tables.cpu()
        slots = torch.tensor([int(bt[b, i // self.bs]) * self.bs + i % self.bs
                              for b, n in enumerate(lens) for i in range(n)],
                             dtype=torch.int32, device=dev)
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32,
                          device=dev)
        if self.kv_calibrate:
            self._calibrate_fp8(ids, pos, cu, max(lens), slots)
        set_context(True, cu, cu, max(lens), max(lens), slots, None, self.state.block_tables)
        h = self.target(ids, pos)
        last = h[cu[1:].long() - 1]
        logits = self.target.compute_logits(last)
        first = self.sampler(logits, self.temps, self.top_ks, self.top_ps)
        set_context(True, cu, cu, max(lens), max(lens), slots, None, self.state.block_tables)
        self.draft(ids, pos)
        reset_context()
        out = first.view(self.B, 1)
        ops.spec_commit(self.state, 0, out, torch.ones(self.B, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()

    # FP8 scales sit this factor above the prompt's amax, so later tokens have
    # headroom before they saturate at +-448 * scale
    FP8_HEADROOM = 2.0

    def _calibrate_fp8(self, ids, pos, cu, maxlen, slots):
        """Per-layer k/v scales of the FP8 target cache, headroom * amax / 448, from
        the K (after q/k-norm and RoPE) and V rows of the prompt: one extra target
        forward that attends over each layer's own bf16 K/V rows and stores nothing
        (so every layer's amax is measured on undistorted activations). Tokens past
        the prompt that exceed amax * headroom saturate at +-448 * scale:
        kv_saturation() measures how many codes did."""
        layers = self.target.attention_layers()
        for a in layers:
            a.calib = torch.zeros(2, dtype=torch.float32, device=self.device)
        set_context(True, cu, cu, maxlen, maxlen, slots, None, self.state.block_tables)
        try:
            self.target(ids, pos)
        finally:
            reset_context()
        amax = torch.stack([a.calib for a in layers]).cpu()
        for a, (ka, va) in zip(layers, amax.tolist()):
            a.k_scale = max(ka, 1e-6) * self.FP8_HEADROOM / 448.0
            a.v_scale = max(va, 1e-6) * self.FP8_HEADROOM / 448.0
            a.calib = None

    def kv_scales(self) -> list[tuple[float, float]]:
        return [(a.k_scale, a.v_scale) for a in self.target.attention_layers()]

    def kv_saturation(self) -> float:
        """Fraction of the FP8 target cache's codes in use (the blocks of the running
        sequences' tables) that sit at the e4m3fn saturation value +-448 (codes 0x7e,
        0xfe): values the per-tensor scales clipped. 0 for a bf16 cache. Reads the
        cache back (a diagnostic, synchronises)."""
        if self.kv.dtype != torch.float8_e4m3fn:
            return 0.0
        nb = self.state.num_seq_blocks.cpu().tolist()
        bt = self.state.block_tables.cpu()
        used = sorted({int(bt[b, i]) for b in range(self.B) for i in range(nb[b])})
        if not used:
            return 0.0
        codes = self.kv.view(torch.uint8)[:, :, torch.tensor(used, device=self.device)]
        sat = ((codes & 0x7F) == 0x7E).sum().item()
        return sat / codes.numel()

    # ------------------------------------------------------------------ preemption
    def preempt(self, b: int):
        """Scheduler.preempt (scheduler.py:313-320) of sequence b between steps: its
        blocks return to the tail of the free list in reverse table order
        (block_manager.py:84-92, deallocate) and it leaves the batch (finished = 1,
        so prealloc and commit skip it) until readmit() has recomputed its KV; its
        tokens and max_tokens stay. Like waiting.appendleft, the last one preempted
        comes back first."""
        if self._staged:
            raise RuntimeError("preempt between chained steps: build the runner with "
                               "adaptive=True or chain_steps=False")
        st = self.state
        n = int(st.num_seq_blocks[b])
        table = st.block_tables[b, :n].cpu().tolist()
        ref = st.ref_count.cpu()
        ring = st.free_ring.cpu()
        head, count = st.free_hdr.cpu().tolist()
        for blk in reversed(table):
            ref[blk] -= 1
            if int(ref[blk]) == 0:
                ring[(head + count) % self.num_blocks] = blk
                count += 1
        st.ref_count.copy_(ref)
        st.free_ring.copy_(ring)
        st.free_hdr.copy_(torch.tensor([head, count], dtype=torch.int32))
        st.block_tables[b].fill_(-1)
        st.num_seq_blocks[b] = 0
        st.finished[b] = 1
        self.preempted.insert(0, b)

    @torch.inference_mode()
    def readmit(self) -> int:
        """Brings preempted sequences back while the free list holds the blocks of
        their whole length (block_manager.py:59-82, allocate: from the front of the
        free list) and one more block for every running sequence, so that a sequence
        preempted for lack of blocks returns only once others have released some;
        the target and draft K/V of every token but the last, which the next step
        processes, are recomputed by prefill. Returns how many returned."""
        if self._staged:
            raise RuntimeError("readmit between chained steps: build the runner with "
                               "adaptive=True or chain_steps=False")
        st = self.state
        back = 0
        while self.preempted:
            b = self.preempted[0]
            n = int(st.context_lens[b])
            need = -(-n // self.bs)
            running = int((st.finished == 0).sum())
            head, count = st.free_hdr.cpu().tolist()
            if count < need + running:
                break
            ring = st.free_ring.cpu()
            blocks = [int(ring[(head + i) % self.num_blocks]) for i in range(need)]
            st.free_hdr.copy_(torch.tensor([(head + need) % self.num_blocks, count - need],
                                           dtype=torch.int32))
            idx = torch.tensor(blocks, dtype=torch.int64, device=self.device)
            st.ref_count.index_fill_(0, idx, 1)
            st.block_hash.index_fill_(0, idx, -1)  # Block.reset
            st.block_tables[b, :need] = idx.to(torch.int32)
            st.num_seq_blocks[b] = need
            self._prefill_rows(b, n - 1)
            st.finished[b] = 0
            self.preempted.pop(0)
            back += 1
        return back

    def _prefill_rows(self, b: int, n: int):
        """Target and draft K/V of tokens [0, n) of sequence b into its blocks."""
        if n <= 0:
            return
        dev = self.device
        st = self.state
        ids = st.tokens[b, :n].clone()
        pos = torch.arange(n, dtype=torch.int64, device=dev)
        bt = st.block_tables[b:b + 1]
        blk = bt[0, (pos // self.bs)].to(torch.int64)
        slots = (blk * self.bs + pos % self.bs).to(torch.int32)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        set_context(True, cu, cu, n, n, slots, None, bt)
        self.target(ids, pos)
        set_context(True, cu, cu, n, n, slots, None, bt)
        self.draft(ids, pos)
        reset_context()

    # ------------------------------------------------------------------ phases
    def draft_phase(self):
        """Pre-allocation (llm_engine.py:111-128) and gamma draft steps
        (model_runner.py:294-318)."""
        st = self.state
        G = self._g()
        if not self._staged:
            ops.spec_prealloc(st, G.gamma, out=G.elig)
        G.u_all.uniform_()  # this step's draft, acceptance and resample uniforms
        for j in range(G.gamma):
            if j == 0:
                # two queries: the previous token (fills the draft K/V the last step
                # left out when it accepted every draft) and the last token
                if self._staged:  # the previous commit staged them
                    ids, pos, slots, cq, ck = self.d_stage0
                else:
                    ids, pos, slots, cq, ck = ops.draft_prepare(st, None, 0, out=self.d_stage0,
                                                                lookback=True)
                set_context(True, cq, ck, 2, 0, slots, None, st.block_tables)
                h = self.draft(ids, pos)[1::2]
            else:
                ids, pos, slots, cq, ck = ops.draft_prepare(st, G.draft_tokens, j,
                                                            out=self.d_stage)
                set_context(False, cq, ck, 1, 0, slots, None, st.block_tables)
                h = self.draft(ids, pos)
            logits = self.draft.compute_logits(h)
            # one sequence: the token goes straight to its draft slot (a column of
            # several sequences is strided, so it goes through the scratch)
            tok = G.draft_tokens[:, j] if self.B == 1 else self.tok_scratch
            if self.mode == "greedy":
                ops.sample_rows(logits, mode="greedy", tokens_out=tok)
            else:
                ops.sample_rows(logits, self.temps, self.top_ks, self.top_ps,
                                mode=self.draft_mode, out_kind=self.draft_out_kind,
                                uniforms=G.u_draft[j], probs_out=G.draft_probs[:, j],
                                tokens_out=tok)
            if self.B != 1:
                G.draft_tokens[:, j].copy_(self.tok_scratch)
        reset_context()

    def verify_phase(self):
        """Verify forward + LM head over all gamma+1 rows + fused acceptance
        (model_runner.py:329-428) + commit/rollback (llm_engine.py:146-181)."""
        st = self.state
        G = self._g()
        g = G.gamma
        if self._staged and self._stage_verify:  # the previous commit staged it
            ids, pos, slots, cq, ck = G.v_stage
        else:
            ids, pos, slots, cq, ck = ops.verify_prepare(st, G.draft_tokens, g, out=G.v_stage)
        set_context(True, cq, ck, g + 1, 0, slots, None, st.block_tables)
        h = self.target(ids, pos)
        reset_context()
        logits = self.target.compute_logits(h).view(self.B, g + 1, self.V)
        # the uniforms were drawn at the start of the draft phase; chained steps
        # run this step's bookkeeping with the acceptance (one launch at batch 1)
        cn = None
        if self.chain_steps:
            cn = dict(state=st, eligible=G.elig, next_gamma=g, stage0=self.d_stage0,
                      lookback=True, stage_verify=G.v_stage if self._stage_verify else None)
        nacc, out, olen = ops.spec_accept(logits, G.draft_probs, G.draft_tokens, self.temps,
                                          G.u_acc, G.u_res, mode=self.mode,
                                          top_ks=self.top_ks, top_ps=self.top_ps,
                                          topk_le64=self.topk_le64, commit_next=cn)
        if self.chain_steps:
            self._staged = True
        else:
            ops.spec_commit(st, g, out, olen, eligible=G.elig)
        G.last = (nacc, out, olen)
        G.logits = logits  # the acceptance call's target rows (read by checks)
        self.last = G.last

    def step(self):
        """One eager speculative step (then the gamma update when adaptive)."""
        self.draft_phase()
        self.verify_phase()
        self._after_step()

    def step_graph(self):
        """One step through the HIP graphs of the current gamma; the first step at
        a new gamma runs eagerly and then captures that gamma's graphs."""
        G = self._g()
        if G.graphs is None:
            self.draft_phase()
            self.verify_phase()
            self.capture()
        else:
            self.replay()
        self._after_step()

    def _after_step(self):
        if self.controller is None:
            return
        G = self._g()
        nacc = G.last[0]
        # accepted drafts and proposals of the sequences that took part (llm_engine.py:150-151),
        # and the smallest count: -1 marks outputs the acceptance kernel could not produce
        tot = torch.stack([(nacc * G.elig).sum(), G.elig.sum(),
                           torch.where(G.elig != 0, nacc, 0).min()]).cpu().tolist()
        if int(tot[2]) < 0:
            raise RuntimeError("spec step: acceptance outputs invalid (a bounded wait inside "
                               "the single-launch kernel ran out); the step committed nothing "
                               "for those sequences")
        accepted, proposed = int(tot[0]), int(tot[1]) * G.gamma
        self.history.append((G.gamma, accepted, proposed))
        self.gamma = self.controller.update(accepted, proposed)

    def check(self):
        """Raises if any acceptance call since the last check produced invalid
        outputs (fixed-gamma runs read nothing back per step; the flag is sticky).
        Synchronises with the device."""
        if ops.accept_error(self.device, clear=True):
            raise RuntimeError("spec run: an acceptance or draft-sampler call produced invalid "
                               "outputs (a bounded wait inside a single-launch kernel ran out)")

    # ------------------------------------------------------------------ graphs
    def capture(self):
        """Records the draft phase and the verify phase of the current gamma into
        two HIP graphs (a memory pool of their own). The caller must have run at
        least one eager step at this gamma (workspaces and library handles exist)."""
        torch.cuda.synchronize()
        snap = self._snapshot()
        G = self._g()
        # the captured verify phase rebinds G.last to the graph's output tensors, which
        # hold nothing until the first replay: keep the eager step's outputs as the
        # last results and switch to the graph's on replay
        eager_last, eager_logits = G.last, G.logits
        gd, gv = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            with torch.cuda.graph(gd, stream=s):
                self.draft_phase()
            with torch.cuda.graph(gv, stream=s, pool=gd.pool()):
                self.verify_phase()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize()
        self._restore(snap)  # capture executed nothing, but keep the state exact
        G.graphs = (gd, gv)
        G.graph_last, G.graph_logits = G.last, G.logits
        G.last = self.last = eager_last
        G.logits = eager_logits

    def replay(self):
        G = self._g()
        gd, gv = G.graphs
        gd.replay()
        gv.replay()
        G.last = self.last = G.graph_last
        G.logits = G.graph_logits

    def _snapshot(self):
        st = self.state
        return {f: getattr(st, f).clone() for f in st.FIELDS}

    def _restore(self, snap):
        for f, t in snap.items():
            getattr(self.state, f).copy_(t)

    # ------------------------------------------------------------------ results
    def lengths(self) -> list[int]:
        return self.state.context_lens.cpu().tolist()

    def tokens(self, b: int) -> list[int]:
        n = int(self.state.context_lens[b])
        return self.state.tokens[b, :n].cpu().tolist()
