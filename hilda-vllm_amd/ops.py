"""torch-facing wrappers of the C ABI (device memory and streams come from torch).

Each wrapper validates shapes on the host, passes raw device pointers and the
current HIP stream to libhilda_spec.so and raises RuntimeError on any non-zero
status. Workspaces (intermediate partial results only, no initialisation
needed) are allocated once per (device, kind) and reused; calls on one device
are ordered by the current stream.
"""
from __future__ import annotations

import torch

from . import _lib as L

_MODES = {"reference": L.HS_ACCEPT_REFERENCE, "filtered": L.HS_ACCEPT_FILTERED,
          "greedy": L.HS_ACCEPT_GREEDY}
_WS: dict = {}
_RETIRED: list = []


def _dev_index(device) -> int:
    """Ordinal of a GPU device ("cuda", "cuda:1", torch.device or int): a device
    without an index means the current device, as torch resolves it for tensors."""
    if isinstance(device, int):
        return device
    d = torch.device(device)
    if d.index is not None:
        return d.index
    try:
        return torch.cuda.current_device()
    except (RuntimeError, AssertionError):  # no GPU here: the only ordinal is 0
        return 0


def workspace(device: torch.device, nbytes: int, kind: str) -> torch.Tensor:
    """Workspace of one kind on one device, grown on demand. A superseded buffer is
    kept alive (never freed) because HIP graphs captured earlier still point at it."""
    key = (_dev_index(device), kind)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _logit_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return L.HS_F32
    if t.dtype == torch.bfloat16:
        return L.HS_BF16
    raise TypeError(f"logits must be float32 or bfloat16, got {t.dtype}")


def _mode(mode) -> int:
    if isinstance(mode, str):
        if mode not in _MODES:
            raise ValueError(f"unknown mode {mode!r}")
        return _MODES[mode]
    return int(mode)


def _need_cuda(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("all tensors must live on the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must live on the same GPU")
    return dev


def _rows2d(t: torch.Tensor, rows: int, V: int) -> tuple[torch.Tensor, int]:
    """View t as `rows` rows of V contiguous elements with one row stride."""
    t2 = t.reshape(rows, V) if t.dim() != 2 else t
    if t2.stride(1) != 1 or t2.shape != (rows, V):
        t2 = t2.contiguous()
    return t2, t2.stride(0)


def spec_accept(target_logits: torch.Tensor, draft_probs: torch.Tensor | None,
                draft_tokens: torch.Tensor, temperatures: torch.Tensor | None,
                u_accept: torch.Tensor | None, u_resample: torch.Tensor | None, *,
                mode="reference", top_ks: torch.Tensor | None = None,
                top_ps: torch.Tensor | None = None, row_stats: bool = False,
                topk_le64: bool = False, chain_only: bool = False,
                commit_next: dict | None = None):
    """Fused acceptance sampler (drop-in for model_runner.py:387-428).

    commit_next: spec_commit_next's arguments after out_len, as a dict (state,
    eligible, next_gamma, stage0, and optionally lookback, stage_verify): the
    call then also runs that bookkeeping on this step's outputs
    (hs_spec_accept_commit_next). At batch 1 with the single-launch kernel it
    runs inside the acceptance launch; if that launch's bounded waits fail, the
    bookkeeping does not run (num_accepted -1 as below).

    topk_le64 (filtered mode): the caller knows every entry of top_ks is in
    [1, 64]; small batches then run as one launch. A sequence breaking that
    promise gets num_accepted -1.

    chain_only: run the launch chain even where a single-launch kernel would
    serve the call (same results; for tests and timing).

    target_logits [B, gamma+1, V] f32/bf16, draft_probs [B, gamma, V] f32,
    draft_tokens [B, gamma] int64, temperatures [B] f32, u_accept [B, gamma],
    u_resample [B]. Returns (num_accepted int32 [B], out_tokens int64
    [B, gamma+1], out_len int32 [B]) and, with row_stats=True, a 4th tensor
    [B*(gamma+1), 2] with the max and normaliser of every target row.

    The call does not synchronise, so a failure inside the single-launch
    kernel (a bounded wait for another workgroup's data that ran out) cannot
    raise here: that sequence's num_accepted is -1 and its out_len 0. The
    caller must check num_accepted >= 0 at its next synchronisation (or
    accept_error(device) at any later point: the flag is sticky).
    """
    m = _mode(mode)
    dev = _need_cuda(target_logits, draft_probs, draft_tokens, temperatures, u_accept,
                     u_resample, top_ks, top_ps)
    if target_logits.dim() != 3:
        raise ValueError("target_logits must be [B, gamma+1, V]")
    B, R, V = target_logits.shape
    gamma = R - 1
    if gamma < 1:
        raise ValueError("need at least one draft token")
    if tuple(draft_tokens.shape) != (B, gamma):
        raise ValueError(f"draft_tokens must be [{B}, {gamma}]")
    lg, lstride = _rows2d(target_logits, B * R, V)
    dt = draft_tokens.to(torch.int64).contiguous()
    q = None
    qstride = V
    if m != L.HS_ACCEPT_GREEDY:
        if draft_probs is None or tuple(draft_probs.shape) != (B, gamma, V):
            raise ValueError(f"draft_probs must be [{B}, {gamma}, {V}]")
        if draft_probs.dtype != torch.float32:
            raise TypeError("draft_probs must be float32")
        q, qstride = _rows2d(draft_probs, B * gamma, V)
        temperatures = temperatures.to(torch.float32).contiguous()
        u_accept = u_accept.to(torch.float32).reshape(B, gamma).contiguous()
        u_resample = u_resample.to(torch.float32).reshape(B).contiguous()
    if m == L.HS_ACCEPT_FILTERED:
        if top_ks is None or top_ps is None:
            raise ValueError("filtered mode needs top_ks and top_ps")
        top_ks = top_ks.to(torch.int32).contiguous()
        top_ps = top_ps.to(torch.float32).contiguous()
    elif topk_le64:
        raise ValueError("topk_le64 applies to filtered mode only")
    nacc = torch.empty(B, dtype=torch.int32, device=dev)
    out = torch.empty((B, R), dtype=torch.int64, device=dev)
    olen = torch.empty(B, dtype=torch.int32, device=dev)
    stats = torch.empty((B * R, 2), dtype=torch.float32, device=dev) if row_stats else None
    lib = L.lib()
    nbytes = lib.hs_spec_accept_workspace_size(B, gamma, V)
    ws = workspace(dev, nbytes, "spec_accept")

    def p(t):
        return None if t is None else t.data_ptr()

    args = (p(lg), _logit_dtype(lg), lstride, p(q), qstride, p(dt),
            p(temperatures) if m != L.HS_ACCEPT_GREEDY else None,
            p(top_ks) if m == L.HS_ACCEPT_FILTERED else None,
            p(top_ps) if m == L.HS_ACCEPT_FILTERED else None,
            p(u_accept) if m != L.HS_ACCEPT_GREEDY else None,
            p(u_resample) if m != L.HS_ACCEPT_GREEDY else None,
            B, gamma, V, m | (L.HS_ACCEPT_TOPK_LE64 if topk_le64 else 0)
            | (L.HS_ACCEPT_CHAIN if chain_only else 0),
            p(nacc), p(out), p(olen), p(stats), ws.data_ptr(), ws.numel())
    if commit_next is None:
        L.check(lib.hs_spec_accept(*args, _stream(dev)), "hs_spec_accept")
    else:
        cn = dict(commit_next)
        if cn["state"].B != B:
            raise ValueError("commit_next state does not match the batch")
        na, keep = _commit_next_args(gamma=gamma, **cn)
        L.check(lib.hs_spec_accept_commit_next(*args, ctypes_ref(na), _stream(dev)),
                "hs_spec_accept_commit_next")
        del keep
    if row_stats:
        return nacc, out, olen, stats
    return nacc, out, olen


def accept_error(device, clear: bool = False) -> bool:
    """True once a spec_accept call (num_accepted -1) or a sample_rows call (token
    -1) on this device's shared workspaces produced invalid outputs: the sticky
    32-bit word at byte 8 of either workspace (include/hilda_spec.h).
    Synchronises with the device."""
    bad = False
    for kind in ("spec_accept", "sampler"):
        ws = _WS.get((_dev_index(device), kind))
        if ws is None:
            continue
        word = ws[8:12]
        if bool(word.cpu().any()):
            bad = True
            if clear:
                word.zero_()
    return bad


def accept_wait_budget(device, polls: int | None, kind: str = "spec_accept") -> None:
    """Sets the wait budget of the single-launch kernels on this device's
    acceptance (kind "spec_accept") or row-sampler ("sampler") workspace (the
    32-bit word at byte 12, include/hilda_spec.h): `polls` polls per thread over
    all its waits of a launch, or the default with None. For tests of the
    failure path: a small budget makes the kernels give up their waits (every
    kernel still exits), and the calls report invalid outputs. Creates the
    workspace if needed; ordered on the current stream."""
    dev = torch.device("cuda", _dev_index(device))
    lib = L.lib()
    size = (lib.hs_spec_accept_workspace_size(1, 1, 8) if kind == "spec_accept"
            else lib.hs_sampler_workspace_size(1, 8))
    ws = workspace(dev, size, kind)
    word = ws[12:16].view(torch.int32)
    word.fill_(0 if polls is None else int(polls) + 1)


def check_accepted(num_accepted: torch.Tensor, what: str = "spec_accept") -> None:
    """Raises if any entry of num_accepted (already on the host, or copied here)
    is negative: the acceptance kernel marked that sequence's outputs invalid."""
    n = num_accepted.cpu() if num_accepted.is_cuda else num_accepted
    if n.numel() and int(n.min()) < 0:
        bad = torch.nonzero(n < 0).flatten().tolist()
        raise RuntimeError(f"{what}: acceptance outputs invalid for sequences {bad} "
                           "(a bounded wait inside the single-launch kernel ran out)")


def sample_rows(logits: torch.Tensor, temperatures: torch.Tensor | None = None,
                top_ks: torch.Tensor | None = None, top_ps: torch.Tensor | None = None, *,
                mode="reference", uniforms: torch.Tensor | None = None, want_probs: bool = False,
                out_kind: int = 0, row_stats: bool = False,
                probs_out: torch.Tensor | None = None, tokens_out: torch.Tensor | None = None,
                chain_only: bool = False):
    """Row sampler (Sampler.forward / draft probabilities).

    Returns dict(probs=[rows, V] f32 or None, tokens=[rows] int64 or None,
    row_stats=[rows, 2] or None). out_kind 1 returns the masked logits of the
    top-k/top-p filters instead of probabilities; out_kind 2 the unfiltered
    probabilities beside the filtered draw (model_runner.py:312-313). A few rows in reference mode
    run as one launch; chain_only runs the launch chain instead (same bits).
    A row whose single-launch draw could not complete (a bounded wait ran out)
    gets token -1 and sets the sticky flag accept_error reads.
    """
    m = _mode(mode)
    dev = _need_cuda(logits, temperatures, top_ks, top_ps, uniforms)
    if logits.dim() != 2:
        raise ValueError("logits must be [rows, V]")
    rows, V = logits.shape
    lg, lstride = _rows2d(logits, rows, V)
    if m != L.HS_ACCEPT_GREEDY:
        if temperatures is None:
            raise ValueError("temperatures required")
        temperatures = temperatures.to(torch.float32).reshape(rows).contiguous()
    if m == L.HS_ACCEPT_FILTERED:
        if top_ks is None or top_ps is None:
            raise ValueError("filtered mode needs top_ks and top_ps")
        top_ks = top_ks.to(torch.int32).reshape(rows).contiguous()
        top_ps = top_ps.to(torch.float32).reshape(rows).contiguous()
    probs = None
    if probs_out is not None:
        if probs_out.shape != (rows, V) or probs_out.stride(1) != 1 or \
                probs_out.dtype != torch.float32:
            raise ValueError("probs_out must be [rows, V] float32 with contiguous rows")
        probs = probs_out
    elif want_probs and m != L.HS_ACCEPT_GREEDY:
        probs = torch.empty((rows, V), dtype=torch.float32, device=dev)
    toks = None
    if m == L.HS_ACCEPT_GREEDY or uniforms is not None:
        if tokens_out is not None:
            if tokens_out.numel() != rows or not tokens_out.is_contiguous() or \
                    tokens_out.dtype != torch.int64:
                raise ValueError("tokens_out must be a contiguous int64 [rows] tensor")
            toks = tokens_out
        else:
            toks = torch.empty(rows, dtype=torch.int64, device=dev)
    if uniforms is not None:
        uniforms = uniforms.to(torch.float32).reshape(rows).contiguous()
    if m == L.HS_ACCEPT_GREEDY and uniforms is None:
        uniforms_ptr = None
    else:
        uniforms_ptr = None if uniforms is None else uniforms.data_ptr()
    stats = torch.empty((rows, 2), dtype=torch.float32, device=dev) if row_stats else None
    lib = L.lib()
    ws = workspace(dev, lib.hs_sampler_workspace_size(rows, V), "sampler")

    def p(t):
        return None if t is None else t.data_ptr()

    rc = lib.hs_sampler(p(lg), _logit_dtype(lg), lstride, rows, V, p(temperatures),
                        p(top_ks) if m == L.HS_ACCEPT_FILTERED else None,
                        p(top_ps) if m == L.HS_ACCEPT_FILTERED else None,
                        m | (L.HS_ACCEPT_CHAIN if chain_only else 0), p(probs),
                        probs.stride(0) if probs is not None else 0, int(out_kind),
                        uniforms_ptr if m != L.HS_ACCEPT_GREEDY else None,
                        p(toks), p(stats), ws.data_ptr(), ws.numel(), _stream(dev))
    L.check(rc, "hs_sampler")
    return dict(probs=probs, tokens=toks, row_stats=stats)


_KV_DTYPES = {torch.bfloat16: L.HS_BF16, torch.float8_e4m3fn: L.HS_FP8_E4M3}


def _kv_code(cache: torch.Tensor) -> int:
    if cache.dtype not in _KV_DTYPES:
        raise TypeError(f"KV cache must be bfloat16 or float8_e4m3fn, got {cache.dtype}")
    return _KV_DTYPES[cache.dtype]


def verify_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     block_tables: torch.Tensor | None, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int,
                     softmax_scale: float, *, k_scale: float = 1.0, v_scale: float = 1.0,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged causal attention over the KV cache (attention.py:145-160 semantics).

    q [tokens, Hq, 128] bf16; k_cache/v_cache [num_blocks, block_size, Hkv, 128]
    bf16 or float8_e4m3fn (dequantised as code * k_scale / v_scale);
    block_tables int32 [B, W]; cu_seqlens_q/k int32 [B+1].
    block_tables None: flash_attn_varlen_func without a block table
    (attention.py:147-160 for a prefill with no cached prefix): k_cache and
    v_cache are then the step's own k / v rows [tokens, Hkv, 128], sequence b's
    keys at rows cu_seqlens_k[b] .. cu_seqlens_k[b + 1] - 1.
    """
    dev = _need_cuda(q, k_cache, v_cache, block_tables, cu_seqlens_q, cu_seqlens_k, out)
    if q.dtype != torch.bfloat16 or q.dim() != 3 or q.stride(2) != 1:
        raise ValueError("q must be [tokens, heads, head_dim] bf16 with contiguous head_dim")
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must match")
    B = cu_seqlens_q.numel() - 1
    cq = cu_seqlens_q.to(torch.int32).contiguous()
    ck = cu_seqlens_k.to(torch.int32).contiguous()
    if block_tables is None:
        if k_cache.dim() != 3 or k_cache.stride() != v_cache.stride() or k_cache.stride(2) != 1:
            raise ValueError("unpaged k / v must be [tokens, kv_heads, head_dim] with identical "
                             "strides and contiguous head_dim")
        Nk, Hkv, D = k_cache.shape
        nb, bs, bt = 1, 32, None
        s_blk, s_tok, s_head = 0, k_cache.stride(0), k_cache.stride(1)
        bt_stride = bt_width = 1
    else:
        if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
            raise ValueError("k_cache and v_cache need identical strides with contiguous "
                             "head_dim")
        nb, bs, Hkv, D = k_cache.shape
        bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
        if bt.dim() != 2 or bt.shape[0] < B or bt.stride(1) != 1:
            bt = bt.contiguous()
        s_blk, s_tok, s_head = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
        bt_stride, bt_width = bt.stride(0), bt.shape[1]
    N, Hq, Dq = q.shape
    if Dq != D:
        raise ValueError("head_dim mismatch")
    if out is None:
        out = torch.empty((N, Hq, D), dtype=torch.bfloat16, device=dev)
    lib = L.lib()
    nbytes = lib.hs_verify_attention_workspace_size(B, Hq, Hkv, int(max_seqlen_q),
                                                    int(max_seqlen_k))
    ws = workspace(dev, nbytes, "attention")
    rc = lib.hs_verify_attention(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
        _kv_code(k_cache), s_blk, s_tok, s_head, float(k_scale), float(v_scale),
        None if bt is None else bt.data_ptr(), bt_stride, bt_width, nb, cq.data_ptr(),
        ck.data_ptr(), B, int(max_seqlen_q), int(max_seqlen_k), Hq, Hkv, D, bs,
        float(softmax_scale), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(),
        ws.numel(), _stream(dev))
    L.check(rc, "hs_verify_attention")
    return out


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor, *, k_scale: float = 1.0,
                  v_scale: float = 1.0) -> None:
    """Writes key/value [N, Hkv, 128] bf16 into the paged cache (attention.py:59-90)."""
    dev = _need_cuda(key, value, k_cache, v_cache, slot_mapping)
    if key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise TypeError("key/value must be bfloat16")
    N, Hkv, D = key.shape
    if slot_mapping.numel() != N:
        raise ValueError("slot_mapping must have one entry per token")
    if key.stride(2) != 1 or value.stride(2) != 1:
        raise ValueError("head_dim must be contiguous")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("k_cache and v_cache need identical strides with contiguous head_dim")
    nb, bs, Hc, Dc = k_cache.shape
    if (Hc, Dc) != (Hkv, D):
        raise ValueError("cache geometry mismatch")
    sm = slot_mapping.to(torch.int32).contiguous()
    rc = L.lib().hs_store_kvcache(
        key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
        value.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), _kv_code(k_cache),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), float(k_scale), float(v_scale),
        sm.data_ptr(), N, Hkv, D, bs, nb, _stream(dev))
    L.check(rc, "hs_store_kvcache")


class SpecStateTensors:
    """Device-resident bookkeeping state of a batch (layout of hs_spec_state).

    Fields mirror Sequence / BlockManager (sequence.py:14-132,
    block_manager.py:26-115): context_lens, num_prompt, max_tokens, ignore_eos,
    finished, block_tables [B, W] (-1 padded), num_seq_blocks, tokens [B, T],
    free_ring [num_blocks] + free_hdr (head, count), ref_count [num_blocks],
    block_hash [num_blocks] int64 (the blocks' prefix hashes, -1 for none).
    """

    FIELDS = ("context_lens", "num_prompt", "max_tokens", "ignore_eos", "finished",
              "block_tables", "num_seq_blocks", "tokens", "free_ring", "free_hdr", "ref_count",
              "block_hash")

    def __init__(self, B: int, W: int, T: int, num_blocks: int, block_size: int, eos: int,
                 device):
        i32 = dict(dtype=torch.int32, device=device)
        self.B, self.W, self.T = B, W, T
        self.num_blocks, self.block_size, self.eos = num_blocks, block_size, int(eos)
        self.context_lens = torch.zeros(B, **i32)
        self.num_prompt = torch.zeros(B, **i32)
        self.max_tokens = torch.zeros(B, **i32)
        self.ignore_eos = torch.zeros(B, **i32)
        self.finished = torch.zeros(B, **i32)
        self.block_tables = torch.full((B, W), -1, **i32)
        self.num_seq_blocks = torch.zeros(B, **i32)
        self.tokens = torch.zeros((B, T), dtype=torch.int64, device=device)
        self.free_ring = torch.arange(num_blocks, **i32)
        self.free_hdr = torch.tensor([0, num_blocks], **i32)
        self.ref_count = torch.zeros(num_blocks, **i32)
        self.block_hash = torch.full((num_blocks,), -1, dtype=torch.int64, device=device)
        self.commit_ws = torch.zeros(
            L.lib().hs_spec_commit_workspace_size(B, W, num_blocks), dtype=torch.uint8,
            device=device)

    def struct(self) -> "L.SpecState":
        st = L.SpecState()
        for f in self.FIELDS:
            setattr(st, f, getattr(self, f).data_ptr())
        st.B, st.W, st.T = self.B, self.W, self.T
        st.num_blocks, st.block_size, st.eos = self.num_blocks, self.block_size, self.eos
        return st


def spec_prealloc(state: SpecStateTensors, gamma: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """llm_engine.py:111-128 on the device; returns eligible int32 [B] (into `out`
    when given)."""
    dev = state.context_lens.device
    elig = out if out is not None else torch.empty(state.B, dtype=torch.int32, device=dev)
    if elig.dtype != torch.int32 or elig.numel() != state.B or not elig.is_contiguous():
        raise ValueError("out must be a contiguous int32 [B] tensor")
    st = state.struct()
    L.check(L.lib().hs_spec_prealloc(ctypes_ref(st), int(gamma), elig.data_ptr(), None,
                                     _stream(dev)), "hs_spec_prealloc")
    return elig


def verify_prepare(state: SpecStateTensors, draft_tokens: torch.Tensor, gamma: int,
                   out: tuple | None = None):
    """model_runner.py:339-362 on the device.

    Returns (input_ids, positions, slot_mapping, cu_seqlens_q, cu_seqlens_k); `out`
    may pass preallocated tensors of those shapes (the draft tokens may be a view
    into out's input_ids: each id is read before it is written)."""
    dev = state.context_lens.device
    B, R = state.B, gamma + 1
    if out is None:
        out = (torch.empty(B * R, dtype=torch.int64, device=dev),
               torch.empty(B * R, dtype=torch.int64, device=dev),
               torch.empty(B * R, dtype=torch.int32, device=dev),
               torch.empty(B + 1, dtype=torch.int32, device=dev),
               torch.empty(B + 1, dtype=torch.int32, device=dev))
    _check_verify_stage(state, gamma, out)
    ids, pos, slots, cq, ck = out
    dt = draft_tokens.to(torch.int64).contiguous() if gamma > 0 else None
    st = state.struct()
    L.check(L.lib().hs_verify_prepare(ctypes_ref(st), None if dt is None else dt.data_ptr(),
                                      int(gamma), ids.data_ptr(), pos.data_ptr(),
                                      slots.data_ptr(), cq.data_ptr(), ck.data_ptr(),
                                      _stream(dev)), "hs_verify_prepare")
    return out


def _check_verify_stage(state: SpecStateTensors, gamma: int, out: tuple) -> None:
    ids, pos, slots, cq, ck = out
    B, R = state.B, gamma + 1
    want = ((ids, B * R, torch.int64), (pos, B * R, torch.int64), (slots, B * R, torch.int32),
            (cq, B + 1, torch.int32), (ck, B + 1, torch.int32))
    for t, n, dt in want:
        if t.numel() != n or t.dtype != dt or not t.is_contiguous():
            raise ValueError("verify staging tensors do not match the batch and gamma")


def spec_commit(state: SpecStateTensors, gamma: int, out_tokens: torch.Tensor,
                out_len: torch.Tensor, *, dirty_mode: int | None = None,
                eligible: torch.Tensor | None = None):
    """llm_engine.py:146-195 on the device. Rows whose `eligible` entry is 0 (the
    status of spec_prealloc) take no tokens. Returns (appended, dirty_slots or None)."""
    dev = state.context_lens.device
    app = torch.empty(state.B, dtype=torch.int32, device=dev)
    dirty = None
    if dirty_mode is not None:
        dirty = torch.empty((state.B, gamma + 1), dtype=torch.int32, device=dev)
    ot = out_tokens.to(torch.int64).contiguous()
    ol = out_len.to(torch.int32).contiguous()
    el = None
    if eligible is not None:
        if eligible.dtype != torch.int32 or eligible.numel() != state.B:
            raise ValueError("eligible must be an int32 [B] tensor")
        el = eligible.contiguous()
    st = state.struct()
    L.check(L.lib().hs_spec_commit(ctypes_ref(st), int(gamma), None, ot.data_ptr(),
                                   ol.data_ptr(), None if el is None else el.data_ptr(),
                                   app.data_ptr(),
                                   None if dirty is None else dirty.data_ptr(),
                                   int(dirty_mode or 0), state.commit_ws.data_ptr(),
                                   state.commit_ws.numel(), _stream(dev)), "hs_spec_commit")
    return app, dirty


def spec_commit_next(state: SpecStateTensors, gamma: int, out_tokens: torch.Tensor,
                     out_len: torch.Tensor, eligible: torch.Tensor, next_gamma: int,
                     stage0: tuple, lookback: bool = True,
                     stage_verify: tuple | None = None) -> None:
    """spec_commit(eligible=eligible) then, in the same launch, the next step's
    spec_prealloc(next_gamma, out=eligible) and draft_prepare(step 0, lookback)
    into the staging tensors `stage0` (ids, positions, slots, cu_q, cu_k):
    llm_engine.py:146-195 and :111-128, model_runner.py:294-310. With
    `stage_verify` (verify_prepare's five outputs for next_gamma), also the next
    step's verify staging (model_runner.py:339-362) except the draft tokens' ids,
    which the draft steps write in place."""
    dev = state.context_lens.device
    na, keep = _commit_next_args(state, gamma, eligible, next_gamma, stage0, lookback,
                                 stage_verify)
    ot = out_tokens.to(torch.int64).contiguous()
    ol = out_len.to(torch.int32).contiguous()
    L.check(L.lib().hs_spec_commit_next(
        na.state, int(gamma), ot.data_ptr(), ol.data_ptr(), na.eligible, na.workspace,
        na.workspace_bytes, na.next_gamma, na.status, na.lookback, na.input_ids, na.positions,
        na.slot_mapping, na.cu_seqlens_q, na.cu_seqlens_k, na.v_input_ids, na.v_positions,
        na.v_slot_mapping, na.v_cu_seqlens_q, na.v_cu_seqlens_k, _stream(dev)),
        "hs_spec_commit_next")
    del keep


def _commit_next_args(state: SpecStateTensors, gamma: int, eligible: torch.Tensor,
                      next_gamma: int, stage0: tuple, lookback: bool = True,
                      stage_verify: tuple | None = None):
    """Checks spec_commit_next's arguments and packs them as hs_commit_next_args;
    returns it and the objects its pointers refer to (keep them alive for the call)."""
    import ctypes
    if eligible.dtype != torch.int32 or eligible.numel() != state.B or not eligible.is_contiguous():
        raise ValueError("eligible must be a contiguous int32 [B] tensor")
    R = 2 if lookback else 1
    ids, pos, slots, cq, ck = stage0
    if (ids.numel() != state.B * R or pos.numel() != state.B * R or slots.numel() != state.B * R
            or cq.numel() != state.B + 1 or ck.numel() != state.B + 1):
        raise ValueError("staging tensors do not match the batch")
    vp = (None,) * 5
    if stage_verify is not None:
        _check_verify_stage(state, next_gamma, stage_verify)
        vp = tuple(t.data_ptr() for t in stage_verify)
    st = state.struct()
    na = L.CommitNextArgs(ctypes.pointer(st), eligible.data_ptr(), state.commit_ws.data_ptr(),
                          state.commit_ws.numel(), int(next_gamma), int(R == 2), None,
                          ids.data_ptr(), pos.data_ptr(), slots.data_ptr(), cq.data_ptr(),
                          ck.data_ptr(), *vp)
    return na, (st,)


def zero_kv_slots(cache: torch.Tensor, slots: torch.Tensor) -> None:
    """Zero the rows of `slots` in every plane of a [P..., num_blocks, block_size, H, D] cache
    (cleanup_rejected_kv_slots, model_runner.py:467-481)."""
    dev = _need_cuda(cache, slots)
    nb, bs, H, D = cache.shape[-4:]
    planes = cache.numel() // (nb * bs * H * D)
    esz = cache.element_size()
    if not cache.is_contiguous():
        raise ValueError("cache must be contiguous")
    s = slots.to(torch.int32).reshape(-1).contiguous()
    L.check(L.lib().hs_zero_kv_slots(cache.data_ptr(), nb * bs * H * D * esz, planes,
                                     H * D * esz, H * D * esz, nb * bs, s.data_ptr(), s.numel(),
                                     _stream(dev)), "hs_zero_kv_slots")


def ctypes_ref(st):
    import ctypes
    return ctypes.byref(st)


def draft_prepare(state: SpecStateTensors, draft_tokens: torch.Tensor | None, step: int,
                  out: tuple | None = None, lookback: bool = False):
    """model_runner.py:294-310 on the device for draft step `step`.

    Returns (input_ids, positions, slot_mapping, cu_q [B+1], cu_k [B+1]) with R rows
    per sequence (R = 2 for step 0 with lookback, else 1); `out` may pass
    preallocated tensors of those shapes (graph capture)."""
    dev = state.context_lens.device
    B = state.B
    R = 2 if (step == 0 and lookback) else 1
    if out is None:
        out = (torch.empty(B * R, dtype=torch.int64, device=dev),
               torch.empty(B * R, dtype=torch.int64, device=dev),
               torch.empty(B * R, dtype=torch.int32, device=dev),
               torch.empty(B + 1, dtype=torch.int32, device=dev),
               torch.empty(B + 1, dtype=torch.int32, device=dev))
    ids, pos, slots, cq, ck = out
    st = state.struct()
    stride = draft_tokens.stride(0) if draft_tokens is not None else 0
    L.check(L.lib().hs_draft_prepare(
        ctypes_ref(st), None if draft_tokens is None else draft_tokens.data_ptr(), int(stride),
        int(step), int(R == 2), ids.data_ptr(), pos.data_ptr(), slots.data_ptr(), cq.data_ptr(),
        ck.data_ptr(), _stream(dev)), "hs_draft_prepare")
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """RMSNorm (layernorm.py:18-25) or fused add + RMSNorm (:27-36, residual updated
    in place). x [rows, H] bf16 with contiguous rows."""
    dev = _need_cuda(x, weight, residual, out)
    rows, H = x.shape
    if out is None:
        out = torch.empty((rows, H), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().hs_rmsnorm(x.data_ptr(), x.stride(0),
                               None if residual is None else residual.data_ptr(),
                               0 if residual is None else residual.stride(0), weight.data_ptr(),
                               out.data_ptr(), out.stride(0), rows, H, float(eps), _stream(dev)),
            "hs_rmsnorm")
    return out


def qk_norm_rope(qkv: torch.Tensor, num_q_heads: int, num_kv_heads: int, q_weight, k_weight,
                 cos_sin: torch.Tensor, positions: torch.Tensor, eps: float):
    """q/k RMSNorm + RoPE of a fused qkv projection [N, (Hq+2Hkv)*128] -> (q, k)."""
    dev = _need_cuda(qkv, q_weight, k_weight, cos_sin, positions)
    N = qkv.shape[0]
    q = torch.empty((N, num_q_heads, 128), dtype=torch.bfloat16, device=dev)
    k = torch.empty((N, num_kv_heads, 128), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().hs_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), num_q_heads, num_kv_heads,
                                    128, q_weight.data_ptr(), k_weight.data_ptr(),
                                    cos_sin.data_ptr(), positions.data_ptr(), float(eps),
                                    q.data_ptr(), k.data_ptr(), N, _stream(dev)),
            "hs_qk_norm_rope")
    return q, k


def qk_norm_rope_store(qkv: torch.Tensor, num_q_heads: int, num_kv_heads: int, q_weight,
                       k_weight, cos_sin: torch.Tensor, positions: torch.Tensor, eps: float,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       *, k_scale: float = 1.0, v_scale: float = 1.0) -> torch.Tensor:
    """qk_norm_rope plus the KV store of the same tokens in one launch: the normalised,
    rotated k heads and the v heads of qkv [N, (Hq+2Hkv)*128] go to their slot_mapping
    slots (store_kvcache semantics, slots < 0 skipped); returns q [N, Hq, 128]."""
    dev = _need_cuda(qkv, q_weight, k_weight, cos_sin, positions, k_cache, v_cache, slot_mapping)
    N = qkv.shape[0]
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be [tokens, (Hq + 2 Hkv) * 128] bf16 with contiguous rows")
    if qkv.shape[1] != (num_q_heads + 2 * num_kv_heads) * 128:
        raise ValueError("qkv width does not match the head counts")
    if slot_mapping.numel() != N or positions.numel() != N:
        raise ValueError("slot_mapping and positions need one entry per token")
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must match")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("k_cache and v_cache need identical strides with contiguous head_dim")
    nb, bs, Hc, Dc = k_cache.shape
    if (Hc, Dc) != (num_kv_heads, 128):
        raise ValueError("cache geometry mismatch")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.shape[1] != 128:
        raise ValueError("cos_sin must be a contiguous f32 [max_position, 128] table")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    sm = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
    pos, sm = pos.contiguous(), sm.contiguous()
    q = torch.empty((N, num_q_heads, 128), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().hs_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), num_q_heads, num_kv_heads, 128, q_weight.data_ptr(),
        k_weight.data_ptr(), cos_sin.data_ptr(), pos.data_ptr(), float(eps), q.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), _kv_code(k_cache), k_cache.stride(0),
        k_cache.stride(1), k_cache.stride(2), float(k_scale), float(v_scale), sm.data_ptr(), bs,
        nb, N, _stream(dev)), "hs_qk_norm_rope_store")
    return q


def qk_norm_rope_attend(qkv: torch.Tensor, num_q_heads: int, num_kv_heads: int, q_weight,
                        k_weight, cos_sin: torch.Tensor, positions: torch.Tensor, eps: float,
                        k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                        block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
                        cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int,
                        softmax_scale: float, *, k_scale: float = 1.0, v_scale: float = 1.0,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """qk_norm_rope_store then verify_attention on the stored cache
    (qwen3.py:83-86 with attention.py:59-90, :145-160), one launch for decode and
    verify steps (hs_qk_norm_rope_attend); returns the attention output
    [tokens, Hq, 128]. qkv holds the query tokens of the sequences in
    cu_seqlens_q order."""
    dev = _need_cuda(qkv, q_weight, k_weight, cos_sin, positions, k_cache, v_cache, slot_mapping,
                     block_tables, cu_seqlens_q, cu_seqlens_k, out)
    N = qkv.shape[0]
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be [tokens, (Hq + 2 Hkv) * 128] bf16 with contiguous rows")
    if qkv.shape[1] != (num_q_heads + 2 * num_kv_heads) * 128:
        raise ValueError("qkv width does not match the head counts")
    if slot_mapping.numel() != N or positions.numel() != N:
        raise ValueError("slot_mapping and positions need one entry per token")
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise ValueError("k_cache and v_cache must match")
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("k_cache and v_cache need identical strides with contiguous head_dim")
    nb, bs, Hc, Dc = k_cache.shape
    if (Hc, Dc) != (num_kv_heads, 128):
        raise ValueError("cache geometry mismatch")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.shape[1] != 128:
        raise ValueError("cos_sin must be a contiguous f32 [max_position, 128] table")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    sm = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
    pos, sm = pos.contiguous(), sm.contiguous()
    B = cu_seqlens_q.numel() - 1
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    if bt.dim() != 2 or bt.shape[0] < B or bt.stride(1) != 1:
        bt = bt.contiguous()
    cq = cu_seqlens_q.to(torch.int32).contiguous()
    ck = cu_seqlens_k.to(torch.int32).contiguous()
    q = torch.empty((N, num_q_heads, 128), dtype=torch.bfloat16, device=dev)
    if out is None:
        out = torch.empty((N, num_q_heads, 128), dtype=torch.bfloat16, device=dev)
    lib = L.lib()
    nbytes = lib.hs_verify_attention_workspace_size(B, num_q_heads, num_kv_heads,
                                                    int(max_seqlen_q), int(max_seqlen_k))
    ws = workspace(dev, nbytes, "attention")
    L.check(lib.hs_qk_norm_rope_attend(
        qkv.data_ptr(), qkv.stride(0), N, q_weight.data_ptr(), k_weight.data_ptr(),
        cos_sin.data_ptr(), cos_sin.shape[0], pos.data_ptr(), float(eps), sm.data_ptr(),
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), _kv_code(k_cache), k_cache.stride(0),
        k_cache.stride(1), k_cache.stride(2), float(k_scale), float(v_scale), bt.data_ptr(),
        bt.stride(0), bt.shape[1], nb, cq.data_ptr(), ck.data_ptr(), B, int(max_seqlen_q),
        int(max_seqlen_k), num_q_heads, num_kv_heads, 128, bs, float(softmax_scale),
        out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), _stream(dev)),
        "hs_qk_norm_rope_attend")
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """activation.py:8-16: silu(gate) * up of a fused [N, 2F] projection."""
    dev = _need_cuda(gate_up)
    N, F2 = gate_up.shape
    out = torch.empty((N, F2 // 2), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().hs_silu_mul(gate_up.data_ptr(), gate_up.stride(0), F2 // 2, out.data_ptr(),
                                out.stride(0), N, _stream(dev)), "hs_silu_mul")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, *, swiglu: bool = False,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight) for decode / verify rows (bf16). Rows <= 8 with
    in_features % 512 == 0 run the skinny HIP kernel (hs_linear); larger row
    counts are plain library GEMMs (hipBLASLt through torch). With swiglu=True
    the weight is [2F, K] (gate | up) and the result is silu(gate) * up [rows, F]."""
    if x.dim() != 2 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("linear expects a 2-D bf16 input and a bf16 weight")
    M, K = x.shape
    N = weight.shape[0] // 2 if swiglu else weight.shape[0]
    if weight.shape[1] != K:
        raise ValueError("in_features mismatch")
    fast = _skinny_ok(x, weight, N)
    if not fast:
        y = torch.nn.functional.linear(x, weight)
        return silu_mul(y) if swiglu else y
    dev = _need_cuda(x, weight, out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    elif out.shape != (M, N) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be [rows, out_features] bf16 with contiguous rows")
    L.check(L.lib().hs_linear(x.data_ptr(), x.stride(0), weight.data_ptr(), M, K, N,
                              1 if swiglu else 0, out.data_ptr(), out.stride(0), _stream(dev)),
            "hs_linear")
    return out


def _skinny_ok(x: torch.Tensor, weight: torch.Tensor, N: int) -> bool:
    M, K = x.shape
    return (M <= 8 and K % 512 == 0 and N % 4 == 0 and x.stride(1) == 1 and
            x.stride(0) % 8 == 0 and weight.is_contiguous() and x.data_ptr() % 16 == 0 and
            weight.data_ptr() % 16 == 0)


def linear_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: torch.Tensor,
                   *, residual: torch.Tensor | None = None, swiglu: bool = False):
    """linear(RMSNorm(x (+ residual)) * norm_weight, weight) for decode / verify rows, the
    norm computed inside the projection (hs_linear_rmsnorm). Returns (y, new_residual) with
    new_residual = bf16(x + residual) (layernorm.py:27-36), or x itself without a residual.
    Rows > 8 run hs_rmsnorm and a library GEMM; the residual is then updated in place."""
    if x.dim() != 2 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("linear_rmsnorm expects a 2-D bf16 input and a bf16 weight")
    M, K = x.shape
    N = weight.shape[0] // 2 if swiglu else weight.shape[0]
    if weight.shape[1] != K or norm_weight.numel() != K:
        raise ValueError("in_features mismatch")
    fast = _skinny_ok(x, weight, N) and norm_weight.is_contiguous() and \
        norm_weight.data_ptr() % 16 == 0
    if residual is not None:
        fast = fast and residual.shape == x.shape and residual.stride(1) == 1 and \
            residual.stride(0) % 8 == 0 and residual.data_ptr() % 16 == 0
    if not fast:
        xn = rmsnorm(x, norm_weight, eps, residual=residual)
        return linear(xn, weight, swiglu=swiglu), (x if residual is None else residual)
    dev = _need_cuda(x, weight, norm_weight, residual)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    res_out = None if residual is None else torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().hs_linear_rmsnorm(
        x.data_ptr(), x.stride(0), None if residual is None else residual.data_ptr(),
        0 if residual is None else residual.stride(0),
        None if res_out is None else res_out.data_ptr(), 0 if res_out is None else K,
        norm_weight.data_ptr(), float(eps), weight.data_ptr(), M, K, N, 1 if swiglu else 0,
        out.data_ptr(), N, _stream(dev)), "hs_linear_rmsnorm")
    return out, (x if residual is None else res_out)
