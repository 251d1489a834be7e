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


@pytest.mark.parametrize("rows,width", [(1, 8), (37, 4096), (512, 12288)])
def test_silu_mul_rows_on_gate_up_halves(rows, width):
    """fdl_silu_mul_rows on the two halves of one [rows, 2 * width] product (the fused
    ff_proj / up_proj GEMM) against silu(gate) * up on contiguous copies."""
    gen = torch.Generator().manual_seed(rows + width)
    gu = (2.0 * torch.randn(rows, 2 * width, generator=gen)).to(torch.bfloat16).to(DEV)
    gate, up = gu[:, :width], gu[:, width:]
    ref = torch.nn.functional.silu(gate.contiguous()) * up.contiguous()
    got = ops.silu_mul(gate, up)
    torch.cuda.synchronize()
    assert got.is_contiguous() and got.shape == (rows, width)
    _check(got, ref, f"silu_mul_rows {rows}x{width}")


def test_block_mlp_tail_fused_gate_up_matches_two_gemms():
    """The block epilogue with adjacent ff_proj / up_proj weights (one GEMM) against the
    same block with the weights in separate buffers (two GEMMs)."""
    import flash_cache_hip as fch
    from fdl.model import LLaDAConfig, LLaDALlamaBlock, random_init_
    cfg = LLaDAConfig.llada_8b()
    cfg.d_model, cfg.n_heads, cfg.mlp_hidden_size = 512, 4, 1536
    blk = LLaDALlamaBlock(cfg, 0, fch.flash_fused_elastic_cache, device=DEV, dtype=torch.bfloat16)
    gen = torch.Generator(device=DEV).manual_seed(0)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05, generator=gen)
    assert fch._adjacent_gate_up(blk) is not None
    x = torch.randn(40, 512, generator=gen, device=DEV).to(torch.bfloat16)
    att = torch.randn(40, 512, generator=gen, device=DEV).to(torch.bfloat16)
    fused = fch.block_mlp_tail(blk, x, att)
    blk.up_proj.weight = torch.nn.Parameter(blk.up_proj.weight.detach().clone())
    assert fch._adjacent_gate_up(blk) is None
    split = fch.block_mlp_tail(blk, x, att)
    torch.cuda.synchronize()
    # the GEMM library may order the reduction differently for the wider product
    torch.testing.assert_close(fused.float(), split.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("rows,width,chunks", [(5, 64, 2), (512, 12288, 4)])
def test_silu_mul_rows_chunked_output(rows, width, chunks):
    """out_chunks = S writes the same values as S column chunks [S, rows, width / S]."""
    gen = torch.Generator().manual_seed(rows)
    gu = (2.0 * torch.randn(rows, 2 * width, generator=gen)).to(torch.bfloat16).to(DEV)
    gate, up = gu[:, :width], gu[:, width:]
    plain = ops.silu_mul(gate, up)
    chunked = ops.silu_mul(gate, up, out_chunks=chunks)
    torch.cuda.synchronize()
    assert chunked.shape == (chunks, rows, width // chunks)
    assert torch.equal(chunked, plain.view(rows, chunks, width // chunks).transpose(0, 1))


@pytest.mark.parametrize("S,rows,cols", [(1, 3, 8), (4, 512, 4096), (3, 17, 72)])
def test_split_reduce_residual_bit_exact(S, rows, cols):
    """residual = bf16(residual + ((p0 + p1) + p2 ...)) in place, the same float32 order."""
    gen = torch.Generator().manual_seed(S * rows + cols)
    part = torch.randn(S, rows, cols, generator=gen).to(DEV)
    res = torch.randn(rows, cols, generator=gen).to(torch.bfloat16).to(DEV)
    acc = part[0].clone()
    for s in range(1, S):
        acc = acc + part[s]
    ref = (res.float() + acc).to(torch.bfloat16)
    out = ops.split_reduce_residual(part, res)
    torch.cuda.synchronize()
    assert out.data_ptr() == res.data_ptr() and torch.equal(out, ref)


def test_block_mlp_tail_split_k_ff_out_matches_single_product():
    """The epilogue with ff_out stored transposed (split-K: chunked SiLU output, batched
    float32-output product, partials + residual in one pass) against the same weights in
    the plain layout (one product accumulating into the residual), and against float32."""
    import flash_cache_hip as fch
    from fdl.model import LLaDAConfig, LLaDALlamaBlock
    cfg = LLaDAConfig.llada_8b()
    cfg.d_model, cfg.n_heads, cfg.mlp_hidden_size = 512, 4, 1536
    blk = LLaDALlamaBlock(cfg, 0, fch.flash_fused_elastic_cache, device=DEV, dtype=torch.bfloat16)
    gen = torch.Generator(device=DEV).manual_seed(1)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.05, generator=gen)
    x = torch.randn(96, 512, generator=gen, device=DEV).to(torch.bfloat16)
    att = torch.randn(96, 512, generator=gen, device=DEV).to(torch.bfloat16)
    assert fch._split_k_ff_out(blk, 96) is not None
    split = fch.block_mlp_tail(blk, x, att)
    blk.ff_out.weight = torch.nn.Parameter(blk.ff_out.weight.detach().contiguous())
    assert fch._split_k_ff_out(blk, 96) is None
    single = fch.block_mlp_tail(blk, x, att)
    # float32 reference of the same epilogue from the bf16 intermediates
    og = x + (att.float() @ blk.attn_out.weight.float().t()).to(torch.bfloat16)
    xn = blk.ff_norm(og)
    g = torch.nn.functional.silu(xn.float() @ blk.ff_proj.weight.float().t()).to(torch.bfloat16)
    u = (xn.float() @ blk.up_proj.weight.float().t()).to(torch.bfloat16)
    hidden = (g.float() * u.float()).to(torch.bfloat16)
    ref = og.float() + hidden.float() @ blk.ff_out.weight.float().t()
    torch.cuda.synchronize()
    torch.testing.assert_close(split.squeeze(0).float(), single.squeeze(0).float(), atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(split.squeeze(0).float(), ref, atol=5e-2, rtol=2e-2)
