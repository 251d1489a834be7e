"""Drop-in replacement of `flash_cache_triton.flash_fused_elastic_cache` for MI355X.

    from flash_cache_hip import flash_fused_elastic_cache

has the signature and the side effects of the reference driver
(llada/flash_cache_triton.py:462-638): it runs one transformer block for the packed query
rows of a denoising step and returns the block output [1, Q, d_model]. The attention
half runs on the hand-written gfx950 kernels behind the C ABI (include/fdl.h):

  non-verify pass (flash_cache_triton.py:536-615)
    fdl_qkv_rope_cache       Q packed by row; K/V written to self.k_cache/self.v_cache at
                             query_pos_flat (replaces _flash_qkv_proj_cache_fwd)
    fdl_block_attention      masked and tracked rows of a sequence in one tile (replaces
                             _flash_masked_attention_fwd + _flash_tracked_attention_fwd)
    fdl_importance_accumulate  attn_scores += mean over (block_m rows, heads) of the raw
                             logits of the masked rows, for block_idx > 1 (replaces the
                             S buffer and `attn_scores += S.mean((0, 1))`)
  verify pass (flash_cache_triton.py:499-535)
    fdl_qkv_rope_cache       kv_packed: Q/K/V of the verify rows, cache untouched
    fdl_verify_attention     cache keys through key_pos_flat + in-block keys under attn_mask

The RMSLayerNorms and the SiLU gate run on fused HIP kernels (fdl_rms_norm, with the
attention residual add folded into ff_norm's pass, and fdl_silu_mul); the projections of
the MLP half (attn_out, ff_proj, up_proj, ff_out; :618-636) are plain library GEMMs through
torch, as in the reference. Norm or activation modules of other kinds run as the modules
themselves.

positions = [query_pos_flat, key_pos_flat, [sin, cos], info, attn_scores, attn_mask]
lengths   = [start_layer, query_verify_blocks, query_masked_blocks, query_tracked_blocks,
             query_blocks, active_batch, num_active, max_length, block_m, block_n,
             elastic_cache, verify]
Where the results differ from the reference's (same arithmetic, different roundings):
  * x = og_x + ff_out(x) is rounded to bf16 once (the residual rides in the product, or in
    the split-K reduction), where the reference rounds ff_out(x) and then the sum: the block
    output can differ in the last bf16 bit;
  * the verify attention's softmax is exact over both key sets (the reference adds the
    in-block terms without raising its running maximum, flash_cache_triton.py:416).

`info` (unused by the reference kernels) may carry a precomputed fdl.schedule.AttnPlan;
otherwise the plan is derived from the masked/tracked block tables once per forward
(the same table objects are passed to every layer) and reused by all layers: on the GPU
(fdl_work_from_blocks, no host copy) when the tables are GPU tensors. A plan over a
paged K/V pool carries `kv_slot`, the cache slots of the query rows; query_pos_flat then
indexes only the RoPE tables, and key_pos_flat (verify) and attn_scores use pool slots.
"""
from __future__ import annotations

import math
import weakref

import numpy as np
import torch
import torch.nn.functional as F

from fdl import lib as _lib
from fdl import ops
from fdl.schedule import (DEFAULT_PAGE_LOG2, AttnPlan, contiguous_page_table, make_plan,
                          seqs_from_reference_blocks)

_plan_cache: dict = {}
_workspace: dict = {}


def _as_np_table(t) -> np.ndarray:
    if t is None or (isinstance(t, (list, tuple)) and len(t) == 0):
        return np.zeros((0, 4), dtype=np.int64)
    return t.detach().to("cpu").numpy().astype(np.int64).reshape(-1, 4)


def _on_device(t, device) -> bool:
    return isinstance(t, torch.Tensor) and t.device == torch.device(device)


def _plan_from_tables(masked, tracked, n_seq: int, max_length: int, n_rows: int,
                      device) -> AttnPlan:
    """AttnPlan for the reference's block tables, cached on the identity of the tables (every
    layer of a forward gets the same table objects). Tables on the GPU are turned into the
    work list there (fdl_work_from_blocks: no host copy, no synchronisation); host tables
    through fdl.schedule."""
    key = (id(masked), id(tracked), n_seq, max_length, n_rows, str(device))
    hit = _plan_cache.get("entry")
    if hit is not None and hit[0] == key and hit[1]() is masked and hit[2]() is tracked:
        return hit[3]
    empty = lambda t: t is None or (isinstance(t, (list, tuple)) and len(t) == 0)  # noqa: E731
    on_dev = all(empty(t) or _on_device(t, device) for t in (masked, tracked)) and not (
        empty(masked) and empty(tracked))
    table = contiguous_page_table(n_seq, max_length)
    if on_dev:
        key_t = ("page_table", n_seq, max_length, str(device))
        table_d = _plan_cache.get(key_t)
        if table_d is None:
            table_d = torch.from_numpy(table).to(device)
            _plan_cache[key_t] = table_d
        as_i64 = lambda t: None if empty(t) else t.reshape(-1, 4).to(torch.int64)  # noqa: E731
        plan = ops.work_from_blocks(as_i64(masked), as_i64(tracked), n_seq, n_rows, table,
                                    table_d, DEFAULT_PAGE_LOG2)
    else:
        seqs = seqs_from_reference_blocks(_as_np_table(masked), _as_np_table(tracked),
                                          importance=True)
        plan = make_plan(seqs, table, device=device)
    ref = lambda t: weakref.ref(t) if isinstance(t, torch.Tensor) else (lambda: t)  # noqa: E731
    _plan_cache["entry"] = (key, ref(masked), ref(tracked), plan)
    return plan


def _imp_workspace(n_heads: int, n_slots: int, device) -> torch.Tensor:
    key = (n_heads, n_slots, str(device))
    ws = _workspace.get(key)
    if ws is None:
        ws = torch.empty((n_heads, n_slots), dtype=torch.float32, device=device)
        _workspace.clear()
        _workspace[key] = ws
    return ws


def _rms_params(norm):
    """(weight, eps) when `norm` is a plain RMSLayerNorm with a bf16 weight and no bias
    (modeling_llada.py:375-403), else None."""
    if "RMS" not in type(norm).__name__ or "Gemma" in type(norm).__name__:
        return None
    w = getattr(norm, "weight", None)
    if not isinstance(w, torch.Tensor) or w.dtype != torch.bfloat16 or w.dim() != 1:
        return None
    if getattr(norm, "bias", None) is not None or not hasattr(norm, "eps"):
        return None
    return w, float(norm.eps)


def _identity_dropout(m) -> bool:
    return isinstance(m, torch.nn.Identity) or (
        isinstance(m, torch.nn.Dropout) and (m.p == 0.0 or not m.training))


def _norm(norm, x: torch.Tensor, checkpoint_fn) -> torch.Tensor:
    p = _rms_params(norm) if checkpoint_fn is None else None
    if p is None or x.dtype != torch.bfloat16:
        return checkpoint_fn(norm, x) if checkpoint_fn is not None else norm(x)
    return ops.rms_norm(x.contiguous(), p[0], p[1])


def _adjacent_gate_up(block) -> torch.Tensor | None:
    """[2h, d] view over ff_proj.weight and up_proj.weight when up_proj's rows directly
    follow ff_proj's in one buffer (as LLaDABlock parameters are laid out by
    fdl.model.fuse_gate_up_), else None. Neither projection may have a bias."""
    fp, up = block.ff_proj, block.up_proj
    wg, wu = fp.weight, up.weight
    if getattr(fp, "bias", None) is not None or getattr(up, "bias", None) is not None:
        return None
    if (wg.dim() != 2 or wg.shape != wu.shape or wg.dtype != wu.dtype or wg.device != wu.device
            or not wg.is_contiguous() or not wu.is_contiguous()):
        return None
    if wu.data_ptr() != wg.data_ptr() + wg.numel() * wg.element_size():
        return None
    if wu.untyped_storage().data_ptr() != wg.untyped_storage().data_ptr():
        return None
    h, d = wg.shape
    return torch.as_strided(wg, (2 * h, d), (d, 1))


# ff_out (K = mlp width, N = d_model) as a split-K product at up to SPLIT_K_MAX_ROWS rows:
# at 512 rows its N = 4096 outputs give too few tiles for the CUs; four K-chunks as one
# batched product with float32 partials, then one pass that adds them and the residual,
# take 57 + 7 us against 78-82 us for the single product (LLaDA-8B shape, MI355X).
SPLIT_K = 4
SPLIT_K_MAX_ROWS = 1024
_BMM_FP32_OUT = hasattr(torch.ops.aten.bmm, "dtype")  # torch.bmm(..., out_dtype=float32)


def _split_k_ff_out(block, rows: int) -> torch.Tensor | None:
    """ff_out.weight^T as [SPLIT_K, K / SPLIT_K, N] views when the split-K product applies
    (bf16 GPU weight stored transposed, see fdl.model.transpose_ff_out_; no bias; identity
    dropout; 1 .. SPLIT_K_MAX_ROWS rows), else None."""
    lin = block.ff_out
    w = lin.weight
    if (not _BMM_FP32_OUT or getattr(lin, "bias", None) is not None
            or not _identity_dropout(block.dropout) or w.dtype != torch.bfloat16
            or not w.is_cuda or w.dim() != 2 or not 0 < rows <= SPLIT_K_MAX_ROWS):
        return None
    n, k = w.shape
    wt = w.t()
    if not wt.is_contiguous() or k % (8 * SPLIT_K) or n % 8:
        return None
    return wt.view(SPLIT_K, k // SPLIT_K, n)


def _ff_out_residual(block, x: torch.Tensor, og_x: torch.Tensor) -> torch.Tensor:
    """og_x + dropout(ff_out(x)) (flash_cache_triton.py:634-636); with an identity dropout
    and no bias the residual add rides in the GEMM (beta = 1) and the GEMM accumulates into
    og_x in place (og_x is the block's own residual-stream tensor), saving a pass over the
    rows and a copy."""
    w = block.ff_out.weight
    if (_identity_dropout(block.dropout) and getattr(block.ff_out, "bias", None) is None
            and x.dim() == 2 and og_x.dim() == 2 and x.dtype == og_x.dtype == w.dtype
            and og_x.is_contiguous()):
        return og_x.addmm_(x, w.t())
    return og_x + block.dropout(block.ff_out(x))


def block_mlp_tail(self, x: torch.Tensor, att: torch.Tensor) -> torch.Tensor:
    """attn_out + residual + SiLU-gated MLP + residual (flash_cache_triton.py:618-638)."""
    att = self.attn_out(att)
    ck = self._activation_checkpoint_fn
    p = _rms_params(self.ff_norm) if ck is None else None
    if (p is not None and _identity_dropout(self.dropout) and x.dtype == torch.bfloat16
            and att.dtype == torch.bfloat16):
        # x + dropout(att) and ff_norm in one pass
        og_x, x = ops.rms_norm(x.contiguous(), p[0], p[1], residual=att.contiguous())
    else:
        x = x + self.dropout(att)
        og_x = x
        x = ck(self.ff_norm, x) if ck is not None else self.ff_norm(x)
    w_gu = _adjacent_gate_up(self)
    if w_gu is not None and ck is None and isinstance(self.act, torch.nn.SiLU) \
            and x.dtype == torch.bfloat16:
        # one GEMM over the concatenated ff_proj / up_proj weights, then SiLU(gate) * up
        # over the two halves of each output row
        h = self.ff_proj.weight.shape[0]
        gu = F.linear(x, w_gu)
        ws = _split_k_ff_out(self, gu.shape[0])
        if ws is not None and og_x.is_contiguous() and og_x.dtype == torch.bfloat16:
            # SiLU(gate) * up written as the K-chunks [S, rows, K / S]; the batched product's
            # right operands are contiguous chunks of W^T; partials + residual in one pass
            xs = ops.silu_mul(gu[:, :h], gu[:, h:], out_chunks=ws.shape[0])
            part = torch.bmm(xs, ws, out_dtype=torch.float32)
            return ops.split_reduce_residual(part, og_x).unsqueeze(0)
        x = ops.silu_mul(gu[:, :h], gu[:, h:])
        return _ff_out_residual(self, x, og_x).unsqueeze(0)
    x, x_up = self.ff_proj(x), self.up_proj(x)
    if ck is None and isinstance(self.act, torch.nn.SiLU) and x.dtype == torch.bfloat16:
        x = ops.silu_mul(x, x_up)
    else:
        x = ck(self.act, x) if ck is not None else self.act(x)
        x = x * x_up
    return _ff_out_residual(self, x, og_x).unsqueeze(0)


def flash_fused_elastic_cache(self, x: torch.Tensor, block_idx, positions, lengths,
                              softmax_scale: float = None):
    """One transformer block over the packed query rows (see the module docstring)."""
    query_pos_flat, key_pos_flat, rotary_emb_pos, info, attn_scores, attn_mask = positions
    (start_layer, query_verify_blocks, query_masked_blocks, query_tracked_blocks, query_blocks,
     active_batch, num_active, max_length, block_m, block_n, elastic_cache, verify) = lengths

    d_model = self.config.d_model
    n_heads = self.config.n_heads
    head_dim = d_model // n_heads
    batch_size = len(active_batch)
    softmax_scale = softmax_scale or (1.0 / math.sqrt(head_dim))

    x_normed = _norm(self.attn_norm, x, None)
    att = torch.empty_like(x)
    q = torch.empty_like(x)
    sin, cos = rotary_emb_pos[0], rotary_emb_pos[1]

    if verify:
        k = torch.empty_like(x)
        v = torch.empty_like(x)
        if query_verify_blocks is not None and query_verify_blocks.shape[0] > 0:
            ops.qkv_rope_cache(x_normed, self.q_proj.weight, self.k_proj.weight,
                               self.v_proj.weight, sin, cos, query_pos_flat, q, k, v, n_heads,
                               kv_packed=True)
            keys = key_pos_flat
            if not isinstance(keys, torch.Tensor) or keys.dtype != torch.int64:
                keys = torch.as_tensor(keys, dtype=torch.int64, device=x.device)
            ops.verify_attention(q, k, v, self.k_cache, self.v_cache, keys,
                                 query_verify_blocks, attn_mask, 2 * block_m, att, n_heads,
                                 softmax_scale)
    else:
        n_rows = x.shape[0]
        if n_rows > 0:
            plan = info if isinstance(info, AttnPlan) else _plan_from_tables(
                query_masked_blocks, query_tracked_blocks, batch_size, max_length, n_rows,
                x.device)
            if plan.kv_slot is not None:
                # paged pool: positions pick the RoPE rows, the plan's slots the cache rows
                ops.qkv_rope_cache(x_normed, self.q_proj.weight, self.k_proj.weight,
                                   self.v_proj.weight, sin, cos, plan.kv_slot, q, self.k_cache,
                                   self.v_cache, n_heads, rope_row=query_pos_flat)
            else:
                ops.qkv_rope_cache(x_normed, self.q_proj.weight, self.k_proj.weight,
                                   self.v_proj.weight, sin, cos, query_pos_flat, q,
                                   self.k_cache, self.v_cache, n_heads)
            importance = block_idx > 1 and plan.has_importance
            ws = _imp_workspace(n_heads, self.k_cache.shape[0], x.device) if importance else None
            ops.block_attention(q, self.k_cache, self.v_cache, plan, att, n_heads, softmax_scale,
                                _lib.IMP_RAW_LOGIT if importance else _lib.IMP_NONE, ws)
            if importance:
                # S.mean((0, 1)) divides by block_m * n_heads (flash_cache_triton.py:538, :615)
                scale = 1.0 / (block_m * n_heads)
                if plan.defer_last_importance and block_idx == self.config.n_layers - 1:
                    plan.deferred_importance = (ws, scale)  # reduced by the caller's ranking
                else:
                    ops.importance_accumulate(ws, plan, scale, attn_scores)

    return block_mlp_tail(self, x, att)
