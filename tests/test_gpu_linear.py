"""Skinny projection kernel (hs_linear) vs an fp32 PyTorch reference.

Shapes are the decode / verify projections of the Qwen3-8B target and the
Qwen3-0.6B draft at 1..8 rows (qkv, o, gate_up + SwiGLU, down, lm_head).
Tolerance: outputs are bf16 (relative step 2^-8) of fp32 sums of K products,
accumulated in a different order than the reference: |err| <= 1e-2 * scale.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 6144), (4096, 4096), (12288, 4096), (1024, 4096), (2048, 1024),
          (3072, 1024), (1024, 151936), (4096, 512)]


def _ref(x, w):
    return x.float() @ w.float().t()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("K,N", SHAPES)
def test_linear_matches_fp32(hv, cuda, M, K, N):
    g = torch.Generator(device=cuda).manual_seed(K + N + M)
    x = torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    print(f"linear M={M} K={K} N={N}", flush=True)
    y = hv.ops.linear(x, w).float()
    ref = _ref(x, w)
    scale = ref.abs().max().item()
    err = (y - ref).abs().max().item()
    assert err <= 1e-2 * scale, (err, scale)


@pytest.mark.parametrize("M", [1, 4, 6])
@pytest.mark.parametrize("K,F", [(4096, 12288), (1024, 3072), (512, 4)])
def test_linear_swiglu(hv, cuda, M, K, F):
    g = torch.Generator(device=cuda).manual_seed(K + F + M)
    x = torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16)
    w = (torch.randn((2 * F, K), generator=g, device=cuda) * 0.05).to(torch.bfloat16)
    y = hv.ops.linear(x, w, swiglu=True).float()
    gu = _ref(x, w)
    gate, up = gu[:, :F], gu[:, F:]
    ref = torch.nn.functional.silu(gate) * up
    scale = ref.abs().max().item()
    assert (y - ref).abs().max().item() <= 2e-2 * scale


def test_linear_strided_rows_and_fallback(hv, cuda):
    g = torch.Generator(device=cuda).manual_seed(7)
    big = torch.randn((3, 2048 + 64), generator=g, device=cuda).to(torch.bfloat16)
    x = big[:, 64:]  # row stride 2112 (multiple of 8), offset 128 bytes
    w = (torch.randn((256, 2048), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    y = hv.ops.linear(x, w).float()
    ref = _ref(x, w)
    assert (y - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()
    # more than 8 rows: library GEMM
    x16 = torch.randn((16, 2048), generator=g, device=cuda).to(torch.bfloat16)
    y16 = hv.ops.linear(x16, w).float()
    assert torch.allclose(y16, _ref(x16, w), rtol=2e-2, atol=2e-2)
