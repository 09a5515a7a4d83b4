"""Sampler backed by the gfx950 row sampler.

Drop-in for mini_vllm/layers/sampler.py: forward(logits, temperatures, top_ks,
top_ps) -> int64 token ids, with _apply_top_k / _apply_top_p returning the
masked logits (the reference tests call those directly, test_sampler.py:6-44).
Differences, by design: the random draw is an inverse-CDF draw driven by one
uniform per row (passed explicitly, or drawn with torch.rand on the device)
instead of the exponential race of sampler.py:24, so results are reproducible
from explicit inputs; a temperature of 0 selects greedy argmax.
"""
from __future__ import annotations


import torch
from torch import nn

from .. import ops as _ops


class Sampler(nn.Module):

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor, top_ks: torch.Tensor,
                top_ps: torch.Tensor, uniforms: torch.Tensor | None = None) -> torch.Tensor:
        rows = logits.shape[0]
        if bool((temperatures == 0).all()):
            return _ops.sample_rows(logits, mode="greedy")["tokens"]
        if uniforms is None:
            uniforms = torch.rand(rows, device=logits.device, dtype=torch.float32)
        r = _ops.sample_rows(logits, temperatures, top_ks.to(torch.int32), top_ps,
                             mode="filtered", uniforms=uniforms)
        return r["tokens"]

    @staticmethod
    def _apply_top_k(logits: torch.Tensor, top_ks: torch.Tensor) -> torch.Tensor:
        rows = logits.shape[0]
        one = torch.ones(rows, device=logits.device, dtype=torch.float32)
        return _ops.sample_rows(logits, one, top_ks.to(torch.int32), one, mode="filtered",
                                want_probs=True, out_kind=1)["probs"]

    @staticmethod
    def _apply_top_p(logits: torch.Tensor, top_ps: torch.Tensor) -> torch.Tensor:
        rows = logits.shape[0]
        one = torch.ones(rows, device=logits.device, dtype=torch.float32)
        zero = torch.zeros(rows, device=logits.device, dtype=torch.int32)
        return _ops.sample_rows(logits, one, zero, top_ps.to(torch.float32), mode="filtered",
                                want_probs=True, out_kind=1)["probs"]
