"""Fused block kernels (fdl_rms_norm, fdl_silu_mul) against the unfused PyTorch code they
replace (modeling_llada.py:389-403 RMSLayerNorm; flash_cache_triton.py:618-633).

Both sides round to bf16 at the same points; the sum of squares is accumulated in a
different order, so an element may differ by one bf16 ulp. Bar: at least 99% of the
elements bit-identical and every element within one bf16 ulp (relative 2^-7)."""
import pytest
import torch

from fdl import ops
from fdl.model import RMSLayerNorm

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check(got: torch.Tensor, ref: torch.Tensor, what: str):
    g, r = got.float(), ref.float()
    same = (got.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert same >= 0.99, f"{what}: only {same:.4f} of the elements bit-identical"
    bound = r.abs() * 2.0 ** -7 + 1e-30
    assert bool(((g - r).abs() <= bound).all()), f"{what}: difference above one bf16 ulp"


@pytest.mark.parametrize("rows,d", [(1, 4096), (37, 4096), (512, 4096), (300, 512), (64, 8192)])
def test_rms_norm_matches_module(rows, d):
    gen = torch.Generator().manual_seed(rows * 7 + d)
    x = (torch.randn(rows, d, generator=gen) * 3.0).to(torch.bfloat16).to(DEV)
    norm = RMSLayerNorm(d, 1e-5, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((1.0 + 0.1 * torch.randn(d, generator=gen)).to(torch.bfloat16))
        ref = norm(x)
    got = ops.rms_norm(x, norm.weight.detach(), 1e-5)
    torch.cuda.synchronize()
    _check(got, ref, f"rms_norm {rows}x{d}")


@pytest.mark.parametrize("rows", [5, 512])
def test_add_rms_norm_matches_residual_then_module(rows):
    d = 4096
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, d, generator=gen).to(torch.bfloat16).to(DEV)
    att = (0.5 * torch.randn(rows, d, generator=gen)).to(torch.bfloat16).to(DEV)
    norm = RMSLayerNorm(d, 1e-5, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((1.0 + 0.1 * torch.randn(d, generator=gen)).to(torch.bfloat16))
        s_ref = x + att
        ref = norm(s_ref)
    s, got = ops.rms_norm(x, norm.weight.detach(), 1e-5, residual=att)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref), "residual sum must be bit-exact"
    _check(got, ref, "add+rms_norm")


@pytest.mark.parametrize("n", [8, 4096 * 3, 512 * 12288])
def test_silu_mul_matches_torch(n):
    gen = torch.Generator().manual_seed(n % 1000)
    g = (2.0 * torch.randn(n, generator=gen)).to(torch.bfloat16).to(DEV)
    u = torch.randn(n, generator=gen).to(torch.bfloat16).to(DEV)
    ref = torch.nn.functional.silu(g) * u
    got = ops.silu_mul(g, u)
    torch.cuda.synchronize()
    _check(got, ref, f"silu_mul n={n}")
