"""Attention layer and KV store backed by the gfx950 kernels.

Drop-in for mini_vllm/layers/attention.py: the same constructor
Attention(num_heads, head_dim, scale, num_kv_heads), the same module
attributes bound by the model runner (k_cache, v_cache, kv_cache_dtype) and
the same store_kvcache(key, value, k_cache, v_cache, slot_mapping) function.
forward(q, k, v) stores k/v at context.slot_mapping when a cache is bound
(attention.py:145) and then attends:
  * prefill / verify (context.is_prefill) with block tables: over the paged
    cache, cu_seqlens_q/k as given (attention.py:147-160, bottom-right causal);
  * prefill without block tables (no cached prefix): over the step's own k/v,
    cu_seqlens_q/k as given (attention.py:147-160 with block_table None; no
    cache needed, as in the reference's warm-up);
  * decode: one query per sequence with context.context_lens keys
    (attention.py:162-170); cu_seqlens_k is taken from context.cu_seqlens_k
    when the caller staged it on the device, else built from context_lens;
    the launch is sized by max_model_len when the runner set it, else by
    max_seqlen_k, else (the reference's decode context sets neither) by the
    block-table width times the block size.
kv_cache_dtype "fp8" means float8_e4m3fn caches with per-tensor scales
k_scale / v_scale, used by every phase (the reference keeps a separate BF16
prefill cache for verify, attention.py:114-131; one FP8 cache keeps the
accepted tokens' K/V in the cache decode reads).
"""
from __future__ import annotations


import torch
from torch import nn

from ..utils.context import get_context

from .. import ops as _ops


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor, k_scale: float = 1.0,
                  v_scale: float = 1.0) -> None:
    """attention.py:83-90: write K/V rows of N tokens to their cache slots (-1 skipped)."""
    N, num_heads, head_dim = key.shape
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert slot_mapping.numel() == N
    _ops.store_kvcache(key, value, k_cache, v_cache, slot_mapping, k_scale=k_scale,
                       v_scale=v_scale)


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = "auto"
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale = 1.0
        self.v_scale = 1.0
        # upper bound of keys per sequence used to size the launch (set by the runner
        # for graph capture; 0 means "use the context's max_seqlen_k")
        self.max_model_len = 0
        # FP8 scale calibration: when a [2] f32 tensor, the producer of this layer's
        # K/V raises it to the amax of the K and V rows it stores
        self.calib = None

    def _check_bound(self, ctx):
        if not (self.k_cache.numel() and self.v_cache.numel()):
            raise RuntimeError("Attention needs a bound KV cache (k_cache / v_cache)")
        if ctx.block_tables is None:
            raise RuntimeError("Attention over the cache needs context.block_tables")

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        k = k.view(-1, self.num_kv_heads, self.head_dim)
        v = v.view(-1, self.num_kv_heads, self.head_dim)
        if self.k_cache.numel() and self.v_cache.numel():
            store_kvcache(k, v, self.k_cache, self.v_cache, ctx.slot_mapping, self.k_scale,
                          self.v_scale)
        if ctx.is_prefill and ctx.block_tables is None:
            # attention.py:147-160 with block_table None: the step's own k / v
            q = q.view(-1, self.num_heads, self.head_dim)
            return _ops.verify_attention(q, k, v, None, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                         ctx.max_seqlen_q, ctx.max_seqlen_k, self.scale)
        return self.attend(q)

    def attend(self, q: torch.Tensor) -> torch.Tensor:
        """The attention half of forward: q against the cache, whose K/V for the
        current tokens a fused producer (ops.qk_norm_rope_store) has already stored."""
        ctx = get_context()
        self._check_bound(ctx)
        q = q.view(-1, self.num_heads, self.head_dim)
        cu_q, cu_k, max_q, max_k = self._bounds(ctx, q.shape[0], q.device)
        return _ops.verify_attention(q, self.k_cache, self.v_cache, ctx.block_tables, cu_q, cu_k,
                                     max_q, max_k, self.scale, k_scale=self.k_scale,
                                     v_scale=self.v_scale)

    def attend_qkv(self, qkv: torch.Tensor, q_norm, k_norm, cos_sin: torch.Tensor,
                   positions: torch.Tensor, eps: float) -> torch.Tensor:
        """q/k-norm + RoPE of the fused qkv rows, the K/V store of the current tokens
        and the attention, one launch for decode and verify steps
        (ops.qk_norm_rope_attend; qwen3.py:83-86 then forward)."""
        ctx = get_context()
        self._check_bound(ctx)
        cu_q, cu_k, max_q, max_k = self._bounds(ctx, qkv.shape[0], qkv.device)
        return _ops.qk_norm_rope_attend(qkv, self.num_heads, self.num_kv_heads, q_norm, k_norm,
                                        cos_sin, positions, eps, self.k_cache, self.v_cache,
                                        ctx.slot_mapping, ctx.block_tables, cu_q, cu_k, max_q,
                                        max_k, self.scale, k_scale=self.k_scale,
                                        v_scale=self.v_scale)

    def _bounds(self, ctx, num_tokens: int, device):
        """cu_seqlens_q / cu_seqlens_k and the maximum query and key lengths of the
        context (decode contexts carry context_lens instead of cu_seqlens_k)."""
        k_cache = self.k_cache
        if ctx.is_prefill:
            cu_q, cu_k = ctx.cu_seqlens_q, ctx.cu_seqlens_k
            max_q, max_k = ctx.max_seqlen_q, ctx.max_seqlen_k
        else:
            B = num_tokens
            cu_q = ctx.cu_seqlens_q
            if cu_q is None:
                cu_q = torch.arange(B + 1, dtype=torch.int32, device=device)
            if ctx.cu_seqlens_k is not None:
                cu_k = ctx.cu_seqlens_k
            else:
                cu_k = torch.zeros(B + 1, dtype=torch.int32, device=device)
                torch.cumsum(ctx.context_lens.to(torch.int32), 0, out=cu_k[1:])
            max_q, max_k = 1, ctx.max_seqlen_k
        if self.max_model_len:
            max_k = self.max_model_len
        elif not ctx.is_prefill and max_k <= 0:
            # the reference's decode context carries no max_seqlen_k
            # (model_runner.py:310 set_context(False, slot_mapping, context_lens,
            # block_tables)); the table width bounds every context without a sync
            max_k = ctx.block_tables.shape[1] * k_cache.shape[1]
        return cu_q, cu_k, max_q, max_k
