"""The attention driver restated with unfused PyTorch ops: the baseline the HIP kernels are
measured against on the same GPU (and a second implementation for end-to-end cross-checks).

Same contract as flash_cache_hip.flash_fused_elastic_cache (flash_cache_triton.py:462-638):
F.linear Q/K/V, rotate-half RoPE on gathered sin/cos rows, index_copy_ into the caches,
per-block softmax attention in float32 (probabilities cast to bf16 before PV, like
flash_cache_triton.py:168), the raw-logit importance `attn_scores += S.mean((0, 1))`, the
verify attention over gathered cache keys plus in-block keys under the mask, and the
block's norm/MLP tail with the model's own modules. Every op is a PyTorch op: no kernel of
libfdl.so runs here. It is selected explicitly (model.set_attention); nothing falls
back to it.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .schedule import AttnPlan, page_slots


def _rotate(t: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor, n_heads: int) -> torch.Tensor:
    """Rotate-half RoPE per head in float32 (flash_cache_triton.py:90-93, :433-441)."""
    rows, d = t.shape
    hd = d // n_heads
    half = hd // 2
    t = t.float().view(rows, n_heads, hd)
    s = sin[:, None, :]
    c = cos[:, None, :]
    t1, t2 = t[..., :half], t[..., half:]
    o1 = t1 * c[..., :half] - t2 * s[..., :half]
    o2 = t2 * c[..., half:] + t1 * s[..., half:]
    return torch.cat([o1, o2], dim=-1).view(rows, d)


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_heads: int, scale: float,
            allow: torch.Tensor | None = None, want_logits: bool = False):
    """Per-head softmax attention, float32 logits; returns (out bf16, raw logits or None)."""
    rows, d = q.shape
    hd = d // n_heads
    qh = q.float().view(rows, n_heads, hd).transpose(0, 1).contiguous()
    kh = k.float().view(-1, n_heads, hd).transpose(0, 1).contiguous()
    vh = v.float().view(-1, n_heads, hd).transpose(0, 1).contiguous()
    s = torch.matmul(qh, kh.transpose(1, 2).contiguous())  # [H, rows, keys]
    raw = s if want_logits else None
    s = s * scale
    if allow is not None:
        s = s.masked_fill(~allow[None], float("-inf"))
    p = torch.softmax(s, dim=-1).to(q.dtype).float()
    o = torch.matmul(p, vh)  # [H, rows, hd]
    return o.transpose(0, 1).reshape(rows, d).to(q.dtype), raw


def _mlp_tail(self, x: torch.Tensor, att: torch.Tensor) -> torch.Tensor:
    """attn_out + residual + gated MLP + residual with plain modules, each step as the
    reference writes it (flash_cache_triton.py:618-638)."""
    ck = self._activation_checkpoint_fn
    att = self.attn_out(att)
    x = x + self.dropout(att)
    og_x = x
    x = ck(self.ff_norm, x) if ck is not None else self.ff_norm(x)
    x, x_up = self.ff_proj(x), self.up_proj(x)
    x = ck(self.act, x) if ck is not None else self.act(x)
    x = x * x_up
    x = self.ff_out(x)
    x = self.dropout(x)
    x = og_x + x
    return x.unsqueeze(0)


def flash_fused_elastic_cache_torch(self, x: torch.Tensor, block_idx, positions, lengths,
                                    softmax_scale: float = None):
    query_pos_flat, key_pos_flat, rotary_emb_pos, info, attn_scores, attn_mask = positions
    (start_layer, query_verify_blocks, query_masked_blocks, query_tracked_blocks, query_blocks,
     active_batch, num_active, max_length, block_m, block_n, elastic_cache, verify) = lengths
    d_model = self.config.d_model
    n_heads = self.config.n_heads
    softmax_scale = softmax_scale or (1.0 / math.sqrt(d_model // n_heads))
    batch_size = len(active_batch)

    x_normed = self.attn_norm(x)
    pos = query_pos_flat
    sin = rotary_emb_pos[0][pos]
    cos = rotary_emb_pos[1][pos]
    q = _rotate(F.linear(x_normed, self.q_proj.weight), sin, cos, n_heads).to(x.dtype)
    k = _rotate(F.linear(x_normed, self.k_proj.weight), sin, cos, n_heads).to(x.dtype)
    v = F.linear(x_normed, self.v_proj.weight)
    att = torch.zeros_like(x)

    if verify:
        blocks = query_verify_blocks.tolist() if query_verify_blocks is not None else []
        rows = 2 * block_m
        for vi, (k0, k1, q0, q1) in enumerate(blocks):
            cache = key_pos_flat[k0:k1]
            keys = torch.cat([self.k_cache[cache].to(k.dtype), k[q0:q1]], dim=0)
            vals = torch.cat([self.v_cache[cache].to(v.dtype), v[q0:q1]], dim=0)
            nr = q1 - q0
            allow = torch.ones((nr, k1 - k0 + nr), dtype=torch.bool, device=x.device)
            allow[:, k1 - k0:] = attn_mask[vi * rows: vi * rows + nr, :nr].bool()
            att[q0:q1], _ = _attend(q[q0:q1], keys, vals, n_heads, softmax_scale, allow)
    else:
        # a plan over a paged pool: the query rows' cache slots, and each sequence's keys
        # through its page-table row (contiguous slots b * max_length + n otherwise)
        paged = isinstance(info, AttnPlan) and info.kv_slot is not None
        slot = info.kv_slot if paged else pos
        if x.shape[0] > 0:
            self.k_cache.index_copy_(0, slot, k.to(self.k_cache.dtype))
            self.v_cache.index_copy_(0, slot, v.to(self.v_cache.dtype))
        importance = block_idx > 1
        S_mean = None
        if importance:
            n = self.k_cache.shape[0] if paged else batch_size * max_length
            S_mean = torch.zeros(n, dtype=torch.float32, device=x.device)
        for table, is_masked in ((query_masked_blocks, True), (query_tracked_blocks, False)):
            if table is None or len(table) == 0:
                continue
            for b, k_end, q0, q1 in table.tolist():
                if paged:
                    keys = torch.from_numpy(page_slots(info.page_table[b], k_end,
                                                       info.page_log2)).to(x.device)
                else:
                    keys = torch.arange(b * max_length, b * max_length + k_end, device=x.device)
                out, raw = _attend(q[q0:q1], self.k_cache[keys], self.v_cache[keys], n_heads,
                                   softmax_scale, want_logits=importance and is_masked)
                att[q0:q1] = out
                if raw is not None:
                    # S.mean((0, 1)) over [block_m, n_heads] (flash_cache_triton.py:538, :615)
                    S_mean[keys] += raw.sum(dim=(0, 1)) / (block_m * n_heads)
        if importance:
            attn_scores += S_mean

    return _mlp_tail(self, x, att)
