"""A small trained LLaDA-shaped model for greedy-decoding checks.

Random weights give near-tied logits, where any bf16 arithmetic flips argmaxes, so a
comparison of greedy decodes needs a model whose decisions are not near ties. This module
trains one in seconds on a GPU: 2 layers, d_model 256 (two heads of 128), SiLU-gated MLP
512, vocabulary 64, on a copy task under LLaDA's masked-diffusion objective: a prompt of
PROMPT_LEN tokens, the response is the prompt twice (GEN_LEN tokens), then EOS up to the
decode's key count (llada/generate.py seqlen_k), every position past the prompt masked with
probability t ~ U(0.05, 1) and predicted with cross-entropy.

The training forward is the model's own computation on a whole sequence (RMSNorm, Q/K/V
projections, rotate-half RoPE from the decode's tables, bidirectional attention over the
sequence and its trailing slots up to the key count, SiLU-gated MLP, residuals, final norm,
LM head), so the weights mean the same to the Flash-Cache decode.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .generate import get_rotary_embedding
from .model import LLaDAConfig, LLaDAModelLM, build_model

CONFIG = dict(d_model=256, n_heads=2, n_layers=2, mlp_hidden_size=512, vocab_size=64,
              rope_theta=10000.0, mask_token_id=63, eos_token_id=62)
PROMPT_LEN, GEN_LEN = 32, 64
KEY_LEN = (PROMPT_LEN + GEN_LEN) // 128 * 128 + 128  # seqlen_k of the decode
N_TOKENS = 60  # prompt tokens 0 .. 59
EOS, MASK = 62, 63


def expected_response(prompt: list[int], n: int) -> list[int]:
    """The task's answer for the first n decoded positions: the prompt twice, then EOS."""
    return (list(prompt) * 2 + [EOS] * max(0, n - GEN_LEN))[:n]


def train_copy_model(device, attention_fn, steps: int = 400, seed: int = 0,
                     batch: int = 64) -> tuple[LLaDAModelLM, float, float]:
    """A float32 model (running `attention_fn` at inference) trained on the copy task.
    Returns (model, masked-token accuracy, smallest top-2 logit gap), the last two on a
    held-out batch of 256 sequences."""
    torch.manual_seed(seed)
    cfg = LLaDAConfig(**CONFIG)
    m = build_model(cfg, attention_fn, device, torch.float32, seed=seed)
    m.requires_grad_(True)
    m.train()
    T, P, G = KEY_LEN, PROMPT_LEN, GEN_LEN
    sin, cos = get_rotary_embedding(T, 128, cfg.rope_theta, device)
    H = cfg.n_heads

    def rope(t):
        return t * cos + torch.cat((-t[..., 64:], t[..., :64]), -1) * sin

    def forward(ids):
        tr = m.model.transformer
        B = ids.shape[0]
        x = tr.wte(ids)
        for blk in tr.blocks:
            h = blk.attn_norm(x)
            q, k, v = (F.linear(h, w).view(B, T, H, 128).transpose(1, 2)
                       for w in (blk.q_proj.weight, blk.k_proj.weight, blk.v_proj.weight))
            a = F.scaled_dot_product_attention(rope(q), rope(k), v)
            x = x + F.linear(a.transpose(1, 2).reshape(B, T, -1), blk.attn_out.weight)
            h = blk.ff_norm(x)
            x = x + F.linear(F.silu(F.linear(h, blk.ff_proj.weight)) *
                             F.linear(h, blk.up_proj.weight), blk.ff_out.weight)
        return F.linear(tr.ln_f(x), tr.ff_out.weight)

    gen = torch.Generator(device=device).manual_seed(seed)

    def sample(B):
        pr = torch.randint(0, N_TOKENS, (B, P), device=device, generator=gen)
        full = torch.cat([pr, pr, pr, torch.full((B, T - P - G), EOS, device=device)], 1)
        t = torch.rand(B, 1, device=device, generator=gen) * 0.95 + 0.05
        mk = torch.rand(B, T - P, device=device, generator=gen) < t
        mk[:, 0] |= ~mk.any(1)
        inp = full.clone()
        inp[:, P:][mk] = MASK
        return inp, full, mk

    opt = torch.optim.AdamW(m.parameters(), lr=2e-3, weight_decay=0.0, foreach=False)
    for _ in range(steps):
        inp, full, mk = sample(batch)
        loss = F.cross_entropy(forward(inp)[:, P:][mk], full[:, P:][mk])
        opt.zero_grad()
        loss.backward()
        opt.step()
    with torch.no_grad():
        inp, full, mk = sample(256)
        lg = forward(inp)[:, P:]
        acc = (lg.argmax(-1)[mk] == full[:, P:][mk]).float().mean().item()
        top2 = lg.topk(2, -1).values
        gap = (top2[..., 0] - top2[..., 1])[mk].min().item()
    m.eval()
    m.requires_grad_(False)
    return m, acc, gap


def compare_decodes(prompts, resp_a, resp_b) -> dict:
    """Position-by-position agreement of two decodes of the same prompts: each response up
    to its first EOS must have the same length (`content_mismatch` counts those that do
    not); positions both decodes filled are compared (past the first EOS a decode may accept
    a few EOS-region tokens, as the reference loop does, and how many depends on which of
    equally confident rows each step takes); `right` counts decode a's tokens equal to the
    task's answer."""
    pos = same = right = tails = content_mismatch = 0
    for i, p in enumerate(prompts):
        a, b = list(resp_a[i]), list(resp_b[i])  # lists, or dicts by prompt index
        ea = a.index(EOS) if EOS in a else len(a)
        eb = b.index(EOS) if EOS in b else len(b)
        content_mismatch += int(ea != eb)
        tails += int(len(a) != len(b))
        n = min(len(a), len(b))
        want = expected_response(p.tolist() if hasattr(p, "tolist") else p, n)
        pos += n
        same += sum(int(x == y) for x, y in zip(a[:n], b[:n]))
        right += sum(int(x == y) for x, y in zip(a[:n], want))
    return dict(positions=pos, agreement=same / max(pos, 1), right=right / max(pos, 1),
                content_mismatch=content_mismatch, eos_tails_differing=tails)
