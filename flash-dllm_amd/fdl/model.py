"""A minimal LLaDA-shaped masked-diffusion transformer with random weights.

The module tree and call signatures mirror the parts of the reference model that the
Flash-Cache path touches, so the decode scheduler and the attention driver see the same
objects:
  * LLaDAModelLM.forward(input_ids, use_cache, lengths=, positions=) -> .logits
    (llada/model/modeling_llada.py:1524-1561)
  * LLaDAModel: wte -> blocks -> ln_f -> ff_out (modeling_llada.py:1328-1488)
  * block.attention(x, block_idx, ..., positions, lengths) calls the attention driver
    `flash_fused_elastic_cache(self, x.squeeze(0), block_idx, positions, lengths)`
    (modeling_llada.py:748-773, :936-993); the driver also runs the block's MLP.
  * block fields read by the driver: attn_norm, q_proj, k_proj, v_proj, attn_out, ff_norm,
    ff_proj, up_proj, act, ff_out, dropout, _activation_checkpoint_fn, config, and the
    k_cache / v_cache the scheduler attaches (llada/generate.py:178-180).
The MLP activation is SiLU applied to ff_proj, multiplied by up_proj (the LLaDA-8B
gated MLP; flash_cache_triton.py:628-633). Weights are N(0, init_std), RMSNorm weights 1.
No checkpoint is loaded: there is none offline.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class LLaDAConfig:
    d_model: int = 4096
    n_heads: int = 32
    n_layers: int = 32
    mlp_hidden_size: int = 12288
    vocab_size: int = 126464
    rope_theta: float = 500000.0
    rms_norm_eps: float = 1e-5
    init_std: float = 0.02
    lm_head_std: float | None = None  # None: init_std
    mask_token_id: int = 126336
    eos_token_id: int = 126081

    @staticmethod
    def llada_8b() -> "LLaDAConfig":
        return LLaDAConfig()


class RMSLayerNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) in float32, cast back, times weight
    (modeling_llada.py:389-403)."""

    def __init__(self, size: int, eps: float, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(size, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        og = x.dtype
        x32 = x.to(torch.float32)
        var = x32.pow(2).mean(-1, keepdim=True)
        x = (x32 * torch.rsqrt(var + self.eps)).to(og)
        return self.weight * x


def _linear(i: int, o: int, device, dtype) -> nn.Linear:
    return nn.Linear(i, o, bias=False, device=device, dtype=dtype)


def _share_gate_up(block: nn.Module) -> None:
    """Puts ff_proj.weight and up_proj.weight (each [h, d]) into one [2h, d] buffer, up_proj's
    rows right after ff_proj's, keeping their values; the block's MLP can then run both
    projections as one GEMM."""
    wg, wu = block.ff_proj.weight, block.up_proj.weight
    buf = torch.cat([wg.detach(), wu.detach()], 0)
    h = wg.shape[0]
    block.ff_proj.weight = nn.Parameter(buf[:h], requires_grad=wg.requires_grad)
    block.up_proj.weight = nn.Parameter(buf[h:], requires_grad=wu.requires_grad)


def _transpose_ff_out(block: nn.Module) -> None:
    """Stores ff_out.weight ([d, h]) as the transposed view of a contiguous [h, d] buffer,
    keeping its values: K-chunks of W^T are then plain views, the right operands of a
    split-K ff_out product."""
    w = block.ff_out.weight
    block.ff_out.weight = nn.Parameter(w.detach().t().contiguous().t(),
                                       requires_grad=w.requires_grad)


@torch.no_grad()
def fuse_gate_up_(model: nn.Module) -> nn.Module:
    """Re-lays every block's ff_proj / up_proj weights out as one buffer (see _share_gate_up),
    for models whose parameters were created or loaded elsewhere."""
    for m in model.modules():
        if hasattr(m, "ff_proj") and hasattr(m, "up_proj"):
            _share_gate_up(m)
    return model


@torch.no_grad()
def transpose_ff_out_(model: nn.Module) -> nn.Module:
    """Re-lays every block's ff_out weight out transposed (see _transpose_ff_out), for
    models whose parameters were created or loaded elsewhere."""
    for m in model.modules():
        if hasattr(m, "ff_proj") and hasattr(m, "ff_out"):
            _transpose_ff_out(m)
    return model


class LLaDALlamaBlock(nn.Module):
    def __init__(self, cfg: LLaDAConfig, layer_id: int, attention_fn: Callable, device=None,
                 dtype=None):
        super().__init__()
        d, h = cfg.d_model, cfg.mlp_hidden_size
        self.config = cfg
        self.layer_id = layer_id
        self.attn_norm = RMSLayerNorm(d, cfg.rms_norm_eps, device, dtype)
        self.ff_norm = RMSLayerNorm(d, cfg.rms_norm_eps, device, dtype)
        self.q_proj = _linear(d, d, device, dtype)
        self.k_proj = _linear(d, d, device, dtype)
        self.v_proj = _linear(d, d, device, dtype)
        self.attn_out = _linear(d, d, device, dtype)
        self.ff_proj = _linear(d, h, device, dtype)
        self.up_proj = _linear(d, h, device, dtype)
        _share_gate_up(self)
        self.ff_out = _linear(h, d, device, dtype)
        _transpose_ff_out(self)
        self.act = nn.SiLU()
        self.dropout = nn.Identity()
        self._activation_checkpoint_fn = None
        self.attention_fn = attention_fn
        self.k_cache = None
        self.v_cache = None

    def attention(self, x, block_idx, mask=None, attention_bias=None, use_cache=False,
                  positions=None, lengths=None):
        return self.attention_fn(self, x.squeeze(0), block_idx, positions, lengths,
                                 softmax_scale=None)

    def forward(self, x, attention_bias=None, layer_past=None, use_cache=False,
                replace_position=None, positions=None, lengths=None, block_idx=0):
        return self.attention(x, block_idx, attention_bias, use_cache=use_cache,
                              positions=positions, lengths=lengths), None


class LLaDAModel(nn.Module):
    def __init__(self, cfg: LLaDAConfig, attention_fn: Callable, device=None, dtype=None):
        super().__init__()
        self.config = cfg
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(cfg.vocab_size, cfg.d_model, device=device, dtype=dtype),
            blocks=nn.ModuleList([LLaDALlamaBlock(cfg, i, attention_fn, device, dtype)
                                  for i in range(cfg.n_layers)]),
            ln_f=RMSLayerNorm(cfg.d_model, cfg.rms_norm_eps, device, dtype),
            ff_out=_linear(cfg.d_model, cfg.vocab_size, device, dtype),
        ))

    def forward(self, input_ids: torch.Tensor, positions=None, lengths=None,
                logit_rows: torch.Tensor | None = None) -> torch.Tensor:
        x = self.transformer.wte(input_ids)
        for block_idx, block in enumerate(self.transformer.blocks):
            x, _ = block(x, use_cache=True, positions=positions, lengths=lengths,
                         block_idx=block_idx)
        if logit_rows is not None:
            # only the rows the scheduler reads (same values, fewer vocab GEMM rows)
            x = x[:, logit_rows]
        x = self.transformer.ln_f(x)
        return self.transformer.ff_out(x)


class LLaDAOutput:
    def __init__(self, logits: torch.Tensor):
        self.logits = logits


class LLaDAModelLM(nn.Module):
    """HF-style wrapper: `model.model.transformer.blocks`, `model.config`, `model.device`."""

    def __init__(self, cfg: LLaDAConfig, attention_fn: Callable, device=None,
                 dtype=torch.bfloat16):
        super().__init__()
        self.config = cfg
        self.model = LLaDAModel(cfg, attention_fn, device, dtype)

    @property
    def device(self) -> torch.device:
        return self.model.transformer.wte.weight.device

    @property
    def dtype(self) -> torch.dtype:
        return self.model.transformer.wte.weight.dtype

    def set_attention(self, attention_fn: Callable) -> None:
        for blk in self.model.transformer.blocks:
            blk.attention_fn = attention_fn

    def forward(self, input_ids=None, use_cache=None, lengths=None, positions=None,
                logit_rows=None, **_unused) -> LLaDAOutput:
        return LLaDAOutput(self.model(input_ids, positions=positions, lengths=lengths,
                                      logit_rows=logit_rows))


@torch.no_grad()
def random_init_(model: LLaDAModelLM, seed: int = 0) -> LLaDAModelLM:
    """N(0, init_std) for every linear and the embedding, ones for the norms, drawn on
    the parameters' device with a seeded generator, in each parameter's logical element
    order (a weight stored transposed gets the values of the plain layout)."""
    cfg = model.config
    gen = torch.Generator(device=model.device).manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("norm.weight") or ".ln_f." in name:
            p.fill_(1.0)
        else:
            std = cfg.lm_head_std if (name.endswith("transformer.ff_out.weight")
                                      and cfg.lm_head_std is not None) else cfg.init_std
            if p.is_contiguous():
                p.normal_(0.0, std, generator=gen)
            else:
                p.copy_(torch.empty(p.shape, dtype=p.dtype, device=p.device).normal_(
                    0.0, std, generator=gen))
    return model


def build_model(cfg: LLaDAConfig, attention_fn: Callable, device, dtype=torch.bfloat16,
                seed: int = 0) -> LLaDAModelLM:
    with torch.device(device):
        model = LLaDAModelLM(cfg, attention_fn, device=device, dtype=dtype)
    model.eval()
    model.requires_grad_(False)  # inference only
    return random_init_(model, seed)
