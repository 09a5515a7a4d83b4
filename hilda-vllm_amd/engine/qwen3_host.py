"""Random-initialised Qwen3 decoder stacks that drive the verify path.

The target (Qwen3-8B geometry) and draft (Qwen3-0.6B geometry) models of the
batch-1 speculative benchmark, restated after mini_vllm/models/qwen3.py:15-218
with the gfx950 kernels: skinny projections for decode / verify rows with the
layer's RMSNorm (and residual add) computed in their prologue and SwiGLU in the
gate_up epilogue, q/k-norm + RoPE fused with the KV-cache store, and the paged
attention; prefill-sized projections are hipBLASLt GEMMs through torch behind
the standalone RMSNorm kernel. Weights are N(0, 0.02^2) in bf16 (no checkpoint
is loaded).
"""
from __future__ import annotations

import copy
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .. import ops as _ops
from ..layers.attention import Attention
from ..utils.context import get_context


@dataclass(frozen=True)
class Qwen3Geometry:
    num_layers: int
    hidden: int
    num_heads: int
    num_kv_heads: int
    ffn: int
    head_dim: int = 128
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1000000.0
    tie_embeddings: bool = False
    max_position: int = 40960


QWEN3_8B = Qwen3Geometry(num_layers=36, hidden=4096, num_heads=32, num_kv_heads=8, ffn=12288)
QWEN3_0_6B = Qwen3Geometry(num_layers=28, hidden=1024, num_heads=16, num_kv_heads=8, ffn=3072,
                           tie_embeddings=True)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """layernorm.py:18-25: normalise in fp32, cast back, scale."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return xf.to(x.dtype) * w


def add_rms_norm(x, residual, w, eps):
    """layernorm.py:27-36: fused residual add; returns (normed, new residual)."""
    xf = x.float() + residual.float()
    res = xf.to(x.dtype)
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return xf.to(x.dtype) * w, res


class Rope(nn.Module):
    """rotary_embedding.py:8-50 (neox halves, fp32 cos/sin cache)."""

    def __init__(self, head_dim, max_position, base, device):
        super().__init__()
        inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device)
                              / head_dim))
        t = torch.arange(max_position, dtype=torch.float32, device=device)
        freqs = torch.outer(t, inv)
        self.register_buffer("cos_sin", torch.cat([freqs.cos(), freqs.sin()], -1),
                             persistent=False)

    def forward(self, positions, q, k):
        cs = self.cos_sin[positions].unsqueeze(1)
        cos, sin = cs.chunk(2, dim=-1)

        def rot(x):
            x1, x2 = x.float().chunk(2, dim=-1)
            return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1).to(x.dtype)

        return rot(q), rot(k)


class Qwen3Layer(nn.Module):
    def __init__(self, g: Qwen3Geometry, device, dtype, rope: Rope):
        super().__init__()
        D = g.head_dim
        self.g = g
        self.q_size = g.num_heads * D
        self.kv_size = g.num_kv_heads * D

        def w(*shape):
            return nn.Parameter(torch.randn(*shape, device=device, dtype=dtype) * 0.02,
                                requires_grad=False)

        def ones(n):
            return nn.Parameter(torch.ones(n, device=device, dtype=dtype), requires_grad=False)

        self.qkv = w(self.q_size + 2 * self.kv_size, g.hidden)
        self.o = w(g.hidden, self.q_size)
        self.gate_up = w(2 * g.ffn, g.hidden)
        self.down = w(g.hidden, g.ffn)
        self.q_norm, self.k_norm = ones(D), ones(D)
        self.ln1, self.ln2 = ones(g.hidden), ones(g.hidden)
        self.rope = rope
        self.attn = Attention(g.num_heads, D, D ** -0.5, g.num_kv_heads)

    def forward(self, positions, h, residual):
        """qwen3.py:148-161 in five fused launches: input RMSNorm (+ the residual add)
        inside the qkv projection; q/k-norm + RoPE + KV store + attention (one launch for
        decode and verify steps, two for prefill); o projection; post-attention RMSNorm
        inside the gate_up projection with SwiGLU; down projection."""
        g = self.g
        qkv, residual = _ops.linear_rmsnorm(h, self.ln1, g.rms_eps, self.qkv, residual=residual)
        attn = self.attn
        ctx = get_context()
        attn._check_bound(ctx)
        if attn.calib is not None:
            # FP8 calibration pass (a prefill with no cached prefix): amax of the K rows
            # (after q/k-norm and RoPE) and V rows, and the attention over those bf16
            # rows themselves (no cache store), so that later layers see the activations
            # of an exact cache rather than of one quantised with unknown scales
            qq, kk = _ops.qk_norm_rope(qkv, g.num_heads, g.num_kv_heads, self.q_norm, self.k_norm,
                                       self.rope.cos_sin, positions, g.rms_eps)
            vv = qkv[:, self.q_size + self.kv_size:]
            torch.maximum(attn.calib, torch.stack([kk.abs().amax(), vv.abs().amax()]).float(),
                          out=attn.calib)
            vr = vv.reshape(-1, g.num_kv_heads, g.head_dim).contiguous()  # k's strides
            o = _ops.verify_attention(qq, kk, vr, None, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                      ctx.max_seqlen_q, ctx.max_seqlen_k, attn.scale)
        else:
            # q/k-norm + RoPE + KV store + attention: one launch for decode and verify steps
            o = attn.attend_qkv(qkv, self.q_norm, self.k_norm, self.rope.cos_sin, positions,
                                g.rms_eps)
        h = _ops.linear(o.reshape(o.shape[0], -1), self.o)
        x, residual = _ops.linear_rmsnorm(h, self.ln2, g.rms_eps, self.gate_up, residual=residual,
                                          swiglu=True)
        h = _ops.linear(x, self.down)
        return h, residual

    def forward_reference(self, positions, h, residual):
        """Eager PyTorch restatement of the same layer (used by tests)."""
        g = self.g
        if residual is None:
            x, residual = rms_norm(h, self.ln1, g.rms_eps), h
        else:
            x, residual = add_rms_norm(h, residual, self.ln1, g.rms_eps)
        qkv = F.linear(x, self.qkv)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = rms_norm(q.reshape(-1, g.num_heads, g.head_dim), self.q_norm, g.rms_eps)
        k = rms_norm(k.reshape(-1, g.num_kv_heads, g.head_dim), self.k_norm, g.rms_eps)
        q, k = self.rope(positions, q, k)
        o = self.attn(q, k, v.reshape(-1, g.num_kv_heads, g.head_dim))
        h = F.linear(o.reshape(o.shape[0], -1), self.o)
        x, residual = add_rms_norm(h, residual, self.ln2, g.rms_eps)
        gu = F.linear(x, self.gate_up)
        gate, up = gu.chunk(2, dim=-1)
        h = F.linear(F.silu(gate) * up, self.down)
        return h, residual


class Qwen3Host(nn.Module):
    """Decoder stack + LM head. `layers`/`embed`/`norm`/`lm_head` may be shared
    with another instance (forced-acceptance draft = first layers of the target)."""

    def __init__(self, g: Qwen3Geometry, device="cuda", dtype=torch.bfloat16, seed=0,
                 share_from: "Qwen3Host | None" = None, num_layers: int | None = None):
        super().__init__()
        self.g = g
        if share_from is not None:
            # same weights, own Attention modules (each model binds its own KV cache)
            self.embed = share_from.embed
            layers = []
            for src in list(share_from.layers)[:num_layers or g.num_layers]:
                lyr = copy.copy(src)
                lyr._parameters = dict(src._parameters)
                lyr._buffers = dict(src._buffers)
                lyr._modules = dict(src._modules)
                lyr.attn = Attention(g.num_heads, g.head_dim, g.head_dim ** -0.5, g.num_kv_heads)
                layers.append(lyr)
            self.layers = nn.ModuleList(layers)
            self.norm = share_from.norm
            self.lm_head = share_from.lm_head
            self.rope = share_from.rope
            return
        gen_state = torch.cuda.get_rng_state(device)
        torch.cuda.manual_seed(seed)
        self.rope = Rope(g.head_dim, g.max_position, g.rope_theta, device)
        self.embed = nn.Parameter(torch.randn(g.vocab, g.hidden, device=device, dtype=dtype) * 0.02,
                                  requires_grad=False)
        self.layers = nn.ModuleList(Qwen3Layer(g, device, dtype, self.rope)
                                    for _ in range(num_layers or g.num_layers))
        self.norm = nn.Parameter(torch.ones(g.hidden, device=device, dtype=dtype),
                                 requires_grad=False)
        if g.tie_embeddings:
            self.lm_head = self.embed
        else:
            self.lm_head = nn.Parameter(
                torch.randn(g.vocab, g.hidden, device=device, dtype=dtype) * 0.02,
                requires_grad=False)
        torch.cuda.set_rng_state(gen_state, device)

    def attention_layers(self):
        return [layer.attn for layer in self.layers]

    def forward(self, input_ids, positions, reference: bool = False):
        h = F.embedding(input_ids, self.embed)
        residual = None
        for layer in self.layers:
            if reference:
                h, residual = layer.forward_reference(positions, h, residual)
            else:
                h, residual = layer(positions, h, residual)
        if reference:
            h, _ = add_rms_norm(h, residual, self.norm, self.g.rms_eps)
            return h
        return _ops.rmsnorm(h, self.norm, self.g.rms_eps, residual=residual)

    def compute_logits(self, h):
        return _ops.linear(h, self.lm_head)
