"""torch-facing wrappers of the C-ABI entry points (include/fdl.h).

Each wrapper checks devices, dtypes, shapes and contiguity, then calls the library on
torch's current HIP stream of the tensors' device. The calls are asynchronous, like the
reference's Triton launches. There is no CPU or PyTorch fallback: a tensor that is not on
a GPU is an error.
"""
from __future__ import annotations

import weakref

import numpy as np
import torch

from . import lib as _lib
from .schedule import LONG_TILE_ROWS, MAX_TILE_ROWS, MID_TILE_ROWS, AttnPlan, DeviceAttnPlan

BF16 = torch.bfloat16


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    """torch's current stream on t's device, as the raw handle the C ABI takes (the same
    value as torch.cuda.current_stream(t.device).cuda_stream, without building the Python
    stream object on every launch)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, ndim: int | None = None,
          device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise _lib.FdlError(_lib.FDL_ERR_UNSUPPORTED,
                            f"{name} is on {t.device}; the HIP path needs GPU tensors")
    if device is not None and t.device != device:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} has dtype {t.dtype}, expected {dtype}")
    if ndim is not None and t.dim() != ndim:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} has {t.dim()} dims, expected {ndim}")
    if not t.is_contiguous():
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} must be contiguous")


_halves_seen: dict = {}


def tables_repeat_halves(rope_sin: torch.Tensor, rope_cos: torch.Tensor) -> bool:
    """Whether every row of both RoPE tables repeats its first half (sin[r, c + hd/2] ==
    sin[r, c], the same for cos), as tables built like the reference's cat(freqs, freqs)
    (llada/generate.py:44-50) do. Compared on the device once per pair of table tensors (one
    synchronisation) and remembered while both tensors live unmodified; under graph capture
    an unseen pair counts as not repeating (nothing is compared)."""
    key = (id(rope_sin), id(rope_cos))
    hit = _halves_seen.get(key)
    if (hit is not None and hit[0]() is rope_sin and hit[1]() is rope_cos
            and hit[2] == (rope_sin._version, rope_cos._version)):
        return hit[3]
    if rope_sin.is_cuda and torch.cuda.is_current_stream_capturing():
        return False
    h = rope_sin.shape[1] // 2
    same = bool(rope_sin.shape[1] % 2 == 0
                and torch.equal(rope_sin[:, :h], rope_sin[:, h:])
                and torch.equal(rope_cos[:, :h], rope_cos[:, h:]))
    if len(_halves_seen) >= 64:
        for k in [k for k, v in _halves_seen.items() if v[0]() is None or v[1]() is None]:
            del _halves_seen[k]
        if len(_halves_seen) >= 64:
            _halves_seen.clear()
    _halves_seen[key] = (weakref.ref(rope_sin), weakref.ref(rope_cos),
                         (rope_sin._version, rope_cos._version), same)
    return same


def qkv_rope_cache(x: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
                   rope_sin: torch.Tensor, rope_cos: torch.Tensor, slot: torch.Tensor,
                   q_out: torch.Tensor, k_out: torch.Tensor, v_out: torch.Tensor, n_heads: int,
                   rope_row: torch.Tensor | None = None, kv_packed: bool = False,
                   rope_halves_equal: bool | None = None) -> None:
    """Fused QKV projection + RoPE + K/V write (fdl_qkv_rope_cache).

    x [Q, D] bf16; w* [D, D] bf16; rope tables fp32 [R, hd]; slot int64 [Q];
    q_out [Q, D]; k_out/v_out the cache [n_slots, D] (or [Q, D] with kv_packed).
    rope_halves_equal: whether every table row repeats its first half (then only that half
    is read); None checks the tables once (see rope_halves_equal()).
    """
    dev = x.device
    _need(x, "x", BF16, 2)
    n_rows, d_model = x.shape
    for n, t in (("wq", wq), ("wk", wk), ("wv", wv)):
        _need(t, n, BF16, 2, dev)
        if tuple(t.shape) != (d_model, d_model):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{n} has shape {tuple(t.shape)}, expected ({d_model}, {d_model})")
    _need(rope_sin, "rope_sin", torch.float32, 2, dev)
    _need(rope_cos, "rope_cos", torch.float32, 2, dev)
    if rope_sin.shape != rope_cos.shape:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "rope_sin and rope_cos differ in shape")
    head_dim = d_model // n_heads
    if rope_sin.shape[1] != head_dim:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"rope tables have {rope_sin.shape[1]} columns, expected {head_dim}")
    _need(slot, "slot", torch.int64, 1, dev)
    if slot.shape[0] != n_rows:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"slot has {slot.shape[0]} entries for {n_rows} rows")
    if rope_row is not None:
        _need(rope_row, "rope_row", torch.int64, 1, dev)
        if rope_row.shape[0] != n_rows:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "rope_row length differs from the row count")
    _need(q_out, "q_out", BF16, 2, dev)
    if tuple(q_out.shape) != (n_rows, d_model):
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "q_out shape differs from x")
    _need(k_out, "k_out", BF16, 2, dev)
    _need(v_out, "v_out", BF16, 2, dev)
    if k_out.shape != v_out.shape or k_out.shape[1] != d_model:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "k_out/v_out must both be [n, d_model]")
    if rope_halves_equal is None:
        rope_halves_equal = tables_repeat_halves(rope_sin, rope_cos)
    flags = (_lib.QKV_KV_PACKED if kv_packed else 0) | \
        (_lib.QKV_ROPE_HALVES_EQUAL if rope_halves_equal else 0)
    _lib.call("fdl_qkv_rope_cache", x.data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(),
              rope_sin.data_ptr(), rope_cos.data_ptr(), rope_sin.shape[0],
              slot.data_ptr(), _ptr(rope_row), n_rows, d_model, n_heads, head_dim,
              q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), k_out.shape[0],
              flags, _stream(x))


def _class_ranges(plan: AttnPlan):
    """(first, count, tile_rows) of the plan's long, mid and short tiles."""
    n_short = plan.n_work - plan.n_long - plan.n_mid
    return ((0, plan.n_long, LONG_TILE_ROWS), (plan.n_long, plan.n_mid, MID_TILE_ROWS),
            (plan.n_long + plan.n_mid, n_short, MAX_TILE_ROWS))


def attention_workspace_floats(plan: AttnPlan, n_heads: int) -> int:
    """fp32 workspace that lets every importance tile of the plan's 64-row class keep its
    softmax-importance probabilities for one pass (fdl_block_attention's workspace; the
    launches of one call reuse it). Only 64-row tiles keep them: the 128-row and 256-row
    kernels take a second pass over K instead. Tiles of at most ATTN_ONCHIP_BLOCKS key blocks
    keep them on chip: a plan without longer 64-row importance tiles needs none."""
    first, count, _ = _class_ranges(plan)[2]
    w = plan.work[first:first + count]
    if count == 0 or w.shape[0] != count or not (w[:, 5] > 0).any():
        return 0
    blocks = int(((w[:, 2].astype(np.int64) - w[:, 1] + 63) // 64).max())
    if blocks <= _lib.ATTN_ONCHIP_BLOCKS:
        return 0
    return count * n_heads * blocks * _lib.ATTN_WS_FLOATS_PER_BLOCK


_cu_count: dict = {}


def _cus(dev: torch.device) -> int:
    n = _cu_count.get(dev.index)
    if n is None:
        n = _cu_count[dev.index] = torch.cuda.get_device_properties(dev).multi_processor_count
    return n


def _split_parts(plan: AttnPlan, first: int, count: int, tile_rows: int, n_heads: int,
                 cus: int) -> int:
    """Key-split parts of one tile class (0: none): a class of 64- or 128-row tiles whose
    count * n_heads workgroups fill at most a quarter of the `cus` compute units (so that at
    least four parts fit; two parts on a half-filled device cost more than they save)
    spreads each tile's key blocks over min(ATTN_MAX_KV_PARTS, cus // (count * n_heads))
    workgroups, capped at its largest tile's block count (more parts would stay empty).

    The cap changes no result bit: part z of p takes blocks [z nb / p, (z + 1) nb / p), so
    with p >= nb every non-empty part holds one block, in the same order, and empty parts
    add exact zeros in the merge; one part is the unsplit launch. A plan built on the device
    has no host copy of its tiles, so it runs uncapped with the same results."""
    if count == 0 or tile_rows == LONG_TILE_ROWS or 4 * count * n_heads > cus:
        return 0
    parts = min(_lib.ATTN_MAX_KV_PARTS, cus // (count * n_heads))
    w = plan.work[first:first + count]
    if w.shape[0] == count:
        parts = min(parts, int(((w[:, 2].astype(np.int64) - w[:, 1] + 63) // 64).max()))
    return parts if parts >= 2 else 0


def attention_split_floats(plan: AttnPlan, n_heads: int, cus: int) -> int:
    """fp32 workspace for fdl_block_attention's key split (no or raw importance): the largest
    class need of _split_parts workgroups per tile, each writing ATTN_PART_FLOATS floats per
    row-index entry and head. fdl_block_attention takes its part count from the room it is
    given, so block_attention hands each class only its own parts' room."""
    n_row_idx = max(int(plan.row_idx.size), 1)
    need = 0
    for first, count, tile_rows in _class_ranges(plan):
        parts = _split_parts(plan, first, count, tile_rows, n_heads, cus)
        need = max(need, parts * n_row_idx * n_heads * _lib.ATTN_PART_FLOATS)
    return need


def block_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    plan: AttnPlan, out: torch.Tensor, n_heads: int, softmax_scale: float,
                    imp_mode: int = _lib.IMP_NONE, imp_part: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None, key_split: bool = True) -> None:
    """Block-table attention with the importance side output (fdl_block_attention). With
    softmax-colsum importance a float32 `workspace` of attention_workspace_floats(plan,
    n_heads) elements keeps the importance rows' probabilities; without, one of
    attention_split_floats(plan, n_heads, CUs) elements holds the partial rows of a key split
    (a launch that would fill at most a quarter of the device). Allocated from torch's caching
    allocator when not given; key_split=False runs every tile in one workgroup per head."""
    dev = q.device
    _need(q, "q", BF16, 2)
    _need(k_cache, "k_cache", BF16, 2, dev)
    _need(v_cache, "v_cache", BF16, 2, dev)
    _need(out, "out", BF16, 2, dev)
    if k_cache.shape != v_cache.shape or k_cache.shape[1] != q.shape[1] or out.shape != q.shape:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "q/out/k_cache/v_cache shapes disagree")
    if plan.work_d is None:
        plan.to(dev)
    if imp_mode != _lib.IMP_NONE:
        if imp_part is None:
            raise _lib.FdlError(_lib.FDL_ERR_NULL, "imp_part is required with an importance mode")
        _need(imp_part, "imp_part", torch.float32, 2, dev)
        if tuple(imp_part.shape) != (n_heads, k_cache.shape[0]):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "imp_part must be [n_heads, n_slots]")
    d_model = q.shape[1]
    stream = _stream(q)
    n_row_idx = max(int(plan.row_idx.size), 1)
    if (imp_mode == _lib.IMP_SOFTMAX_COLSUM and plan.n_long and plan.work.shape[0] >= plan.n_long
            and int(plan.work[:plan.n_long, 5].max()) > MID_TILE_ROWS):
        raise _lib.FdlError(_lib.FDL_ERR_UNSUPPORTED,
                            f"softmax-colsum importance needs at most {MID_TILE_ROWS} importance rows per sequence")
    if imp_mode == _lib.IMP_SOFTMAX_COLSUM and workspace is None:
        workspace = torch.empty(max(attention_workspace_floats(plan, n_heads), 4),
                                dtype=torch.float32, device=dev)
    elif imp_mode != _lib.IMP_SOFTMAX_COLSUM and workspace is None and key_split:
        n = attention_split_floats(plan, n_heads, _cus(dev))
        if n:
            workspace = torch.empty(n, dtype=torch.float32, device=dev)
    if workspace is not None:
        _need(workspace, "workspace", torch.float32, 1, dev)
    # long tiles (the first n_long work items), mid tiles (the next n_mid), short tiles
    cus = _cus(dev)
    for first, count, tile_rows in _class_ranges(plan):
        if count == 0:
            continue
        ws_n = 0 if workspace is None else workspace.numel()
        if imp_mode != _lib.IMP_SOFTMAX_COLSUM and key_split:
            # the room of this class's own parts (the launcher splits as far as the room allows)
            ws_n = min(ws_n, _split_parts(plan, first, count, tile_rows, n_heads, cus) *
                       n_row_idx * n_heads * _lib.ATTN_PART_FLOATS)
        elif imp_mode != _lib.IMP_SOFTMAX_COLSUM:
            ws_n = 0
        _lib.call("fdl_block_attention", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                  q.shape[0], k_cache.shape[0], d_model, n_heads, d_model // n_heads,
                  plan.page_table_d.data_ptr(), plan.page_table.shape[0], plan.page_table.shape[1],
                  plan.page_log2, plan.work_d[first:].data_ptr(), count, plan.row_idx_d.data_ptr(),
                  n_row_idx, tile_rows, float(softmax_scale), out.data_ptr(), int(imp_mode),
                  _ptr(imp_part), _ptr(workspace) if ws_n else None, ws_n, stream)


def work_from_blocks(masked: torch.Tensor, tracked: torch.Tensor, n_seq: int, n_q_rows: int,
                     page_table: np.ndarray, page_table_d: torch.Tensor, page_log2: int,
                     status: torch.Tensor | None = None) -> DeviceAttnPlan:
    """An attention plan built on the device from the reference's block tables (int64
    [n, 4] device tensors, rows (batch, k_end, q0, q1); fdl_work_from_blocks): no host
    copy of the tables. Regions: n_q_rows // 128 long, n_seq mid and n_seq short items."""
    dev = page_table_d.device
    tabs = []
    for name, t in (("masked", masked), ("tracked", tracked)):
        if t is None or t.numel() == 0:
            tabs.append(None)
            continue
        _need(t, name, torch.int64, 2, dev)
        if t.shape[1] != 4:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} must be [n, 4]")
        tabs.append(t.contiguous())
    n_m = 0 if tabs[0] is None else tabs[0].shape[0]
    n_t = 0 if tabs[1] is None else tabs[1].shape[0]
    # every 256-row tile belongs to a group of more than 128 rows: at most n_q_rows // 128
    cap_long, cap_mid, cap_short = n_q_rows // MID_TILE_ROWS, n_seq, n_seq
    work = torch.empty((max(cap_long + cap_mid + cap_short, 1), 8), dtype=torch.int32, device=dev)
    row_idx = torch.empty(max(n_q_rows, 1), dtype=torch.int32, device=dev)
    if status is not None:
        _need(status, "status", torch.int32, 1, dev)
    max_k = int(page_table.shape[1]) << page_log2
    _lib.call("fdl_work_from_blocks", _ptr(tabs[0]), n_m, _ptr(tabs[1]), n_t, n_seq, n_q_rows,
              max_k, work.data_ptr(), cap_long, cap_mid, cap_short, row_idx.data_ptr(),
              _ptr(status), _stream(page_table_d))
    return DeviceAttnPlan(work, row_idx, n_q_rows, page_table, page_table_d, page_log2, cap_long,
                          cap_mid, cap_long + cap_mid + cap_short, n_m > 0)


def importance_accumulate(imp_part: torch.Tensor, plan: AttnPlan, scale: float,
                          scores: torch.Tensor) -> None:
    """scores[slot] += scale * sum_h imp_part[h][slot] (fdl_importance_accumulate)."""
    dev = imp_part.device
    _need(imp_part, "imp_part", torch.float32, 2)
    _need(scores, "scores", torch.float32, 1, dev)
    if scores.shape[0] != imp_part.shape[1]:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "scores length differs from imp_part columns")
    if plan.work_d is None:
        plan.to(dev)
    _lib.call("fdl_importance_accumulate", imp_part.data_ptr(), imp_part.shape[0], imp_part.shape[1],
              plan.page_table_d.data_ptr(), plan.page_table.shape[0], plan.page_table.shape[1],
              plan.page_log2, plan.work_d.data_ptr(), plan.n_work, float(scale), scores.data_ptr(),
              _stream(imp_part))


def importance_rank(scores: torch.Tensor, slots: torch.Tensor, seg: torch.Tensor, max_len: int,
                    topk_out: torch.Tensor | None = None, k: int = 0,
                    imp_part: torch.Tensor | None = None, scale: float = 1.0,
                    plan: AttnPlan | None = None, seg_keys: torch.Tensor | None = None) -> None:
    """Sorts each segment (start, len) of `slots` in place by importance and gathers the
    top-k (fdl_importance_rank). With `imp_part` [n_heads, n_scores], `plan` (its page
    table) and `seg_keys` int32 [n_seg, 2] = (page-table row, key count) per segment, first
    reduces imp_part into the scores of each segment's sequence keys, as
    importance_accumulate does (fdl_importance_accumulate_rank)."""
    dev = scores.device
    if imp_part is not None:
        _need(imp_part, "imp_part", torch.float32, 2, dev)
        if imp_part.shape[1] != scores.shape[0]:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "imp_part must be [n_heads, len(scores)]")
        if plan is None or seg_keys is None:
            raise _lib.FdlError(_lib.FDL_ERR_NULL, "imp_part needs plan and seg_keys")
        _need(seg_keys, "seg_keys", torch.int32, 2, dev)
        if tuple(seg_keys.shape) != (seg.shape[0], 2):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "seg_keys must be [n_seg, 2]")
        if plan.page_table_d is None:
            plan.to(dev)
    _need(scores, "scores", torch.float32, 1)
    _need(slots, "slots", torch.int64, None, dev)
    _need(seg, "seg", torch.int32, 2, dev)
    if seg.shape[1] != 2:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "seg must be [n_seg, 2]")
    if topk_out is not None:
        _need(topk_out, "topk_out", torch.int64, 2, dev)
        if tuple(topk_out.shape) != (seg.shape[0], k):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "topk_out must be [n_seg, k]")
    kk = int(k if topk_out is not None else 0)
    if imp_part is not None:
        _lib.call("fdl_importance_accumulate_rank", imp_part.data_ptr(), imp_part.shape[0],
                  float(scale), plan.page_table_d.data_ptr(), plan.page_table.shape[0],
                  plan.page_table.shape[1], plan.page_log2, seg_keys.data_ptr(),
                  scores.data_ptr(), scores.shape[0], slots.data_ptr(),
                  slots.numel(), seg.data_ptr(), seg.shape[0], int(max_len), _ptr(topk_out), kk,
                  _stream(scores))
        return
    _lib.call("fdl_importance_rank", scores.data_ptr(), scores.shape[0], slots.data_ptr(),
              slots.numel(), seg.data_ptr(), seg.shape[0], int(max_len), _ptr(topk_out), kk,
              _stream(scores))


def verify_attention(q: torch.Tensor, k_blk: torch.Tensor, v_blk: torch.Tensor,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, key_slots: torch.Tensor,
                     vblocks: torch.Tensor, mask: torch.Tensor, block_rows: int,
                     out: torch.Tensor, n_heads: int, softmax_scale: float) -> None:
    """Flash-Verify attention (fdl_verify_attention). `mask` is the reference's boolean
    [n_blocks * block_rows, block_rows] mask, or int32 [n_blocks, 2] = (T, S) per block for
    the closed-form mask (no mask read from memory)."""
    dev = q.device
    _need(q, "q", BF16, 2)
    for n, t in (("k_blk", k_blk), ("v_blk", v_blk), ("out", out)):
        _need(t, n, BF16, 2, dev)
        if t.shape != q.shape:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{n} shape differs from q")
    _need(k_cache, "k_cache", BF16, 2, dev)
    _need(v_cache, "v_cache", BF16, 2, dev)
    _need(key_slots, "key_slots", torch.int64, 1, dev)
    _need(vblocks, "vblocks", torch.int32, 2, dev)
    nv = vblocks.shape[0]
    vmeta = None
    if mask.dtype == torch.int32:
        vmeta, mask = mask, None
        _need(vmeta, "vmeta", torch.int32, 2, dev)
        if tuple(vmeta.shape) != (nv, 2):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"vmeta must be [{nv}, 2]")
    else:
        if mask.dtype == torch.bool:
            mask = mask.view(torch.uint8)
        _need(mask, "mask", torch.uint8, 2, dev)
        if tuple(mask.shape) != (nv * block_rows, block_rows):
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"mask must be [{nv * block_rows}, {block_rows}]")
    d_model = q.shape[1]
    _lib.call("fdl_verify_attention", q.data_ptr(), k_blk.data_ptr(), v_blk.data_ptr(),
              k_cache.data_ptr(), v_cache.data_ptr(), q.shape[0], k_cache.shape[0], d_model,
              n_heads, d_model // n_heads, key_slots.data_ptr() if key_slots.numel() else None,
              key_slots.numel(), vblocks.data_ptr(), nv, _ptr(mask), _ptr(vmeta),
              int(block_rows), float(softmax_scale), out.data_ptr(), _stream(q))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
             sum_out: torch.Tensor | None = None):
    """RMSLayerNorm of x (or of bf16(x + residual)) times weight (fdl_rms_norm).

    Returns out, or (sum_out, out) when a residual is given."""
    dev = x.device
    _need(x, "x", BF16, 2)
    n_rows, d = x.shape
    _need(weight, "weight", BF16, 1, dev)
    if weight.shape[0] != d:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"weight has {weight.shape[0]} entries, expected {d}")
    if out is None:
        out = torch.empty_like(x)
    _need(out, "out", BF16, 2, dev)
    if residual is not None:
        _need(residual, "residual", BF16, 2, dev)
        if residual.shape != x.shape:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "residual shape differs from x")
        if sum_out is None:
            sum_out = torch.empty_like(x)
        _need(sum_out, "sum_out", BF16, 2, dev)
    _lib.call("fdl_rms_norm", x.data_ptr(), _ptr(residual), weight.data_ptr(), n_rows, d,
              float(eps), _ptr(sum_out), out.data_ptr(), _stream(x))
    return out if residual is None else (sum_out, out)


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None,
             out_chunks: int = 1) -> torch.Tensor:
    """bf16(bf16(silu(gate)) * up) (fdl_silu_mul). gate and up may also be [rows, width]
    views with one common row stride and unit column stride, such as the two halves of a
    [rows, 2 * width] product (fdl_silu_mul_rows); out is then a new contiguous tensor,
    [rows, width], or with out_chunks = S > 1 the column chunks [S, rows, width / S]."""
    if up.shape != gate.shape:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "up shape differs from gate")
    if out_chunks != 1 and gate.dim() != 2:
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "out_chunks needs [rows, width] operands")
    if (gate.dim() == 2 and (out_chunks != 1 or not gate.is_contiguous()) and gate.stride(1) == 1
            and up.stride() == gate.stride()):
        for t, name in ((gate, "gate"), (up, "up")):
            if t.device.type != "cuda" or t.dtype != BF16:
                raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"{name} must be a bf16 GPU tensor")
        if up.device != gate.device:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "up is on another device than gate")
        rows, width = gate.shape
        if out_chunks < 1 or width % out_chunks:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"out_chunks {out_chunks} does not divide {width}")
        shape = (rows, width) if out_chunks == 1 else (out_chunks, rows, width // out_chunks)
        if out is None:
            out = torch.empty(shape, dtype=BF16, device=gate.device)
        _need(out, "out", BF16, len(shape), gate.device)
        if tuple(out.shape) != shape:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, f"out must be {list(shape)}")
        _lib.call("fdl_silu_mul_rows", gate.data_ptr(), up.data_ptr(), rows, width,
                  gate.stride(0), out_chunks, out.data_ptr(), _stream(gate))
        return out
    _need(gate, "gate", BF16)
    _need(up, "up", BF16, None, gate.device)
    if out is None:
        out = torch.empty_like(gate)
    _need(out, "out", BF16, None, gate.device)
    _lib.call("fdl_silu_mul", gate.data_ptr(), up.data_ptr(), gate.numel(), out.data_ptr(),
              _stream(gate))
    return out


def split_reduce_residual(part: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual = bf16(residual + sum_s part[s]) in place (fdl_split_reduce_residual):
    part fp32 [S, rows, cols], residual bf16 [rows, cols]."""
    _need(residual, "residual", BF16, 2)
    _need(part, "part", torch.float32, 3, residual.device)
    if tuple(part.shape[1:]) != tuple(residual.shape):
        raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "part must be [S, rows, cols] of the residual")
    _lib.call("fdl_split_reduce_residual", part.data_ptr(), part.shape[0], residual.shape[0],
              residual.shape[1], residual.data_ptr(), _stream(residual))
    return residual


def softmax_confidence(logits: torch.Tensor, token: torch.Tensor | None = None
                       ) -> tuple[torch.Tensor, torch.Tensor]:
    """(prob float64 [rows], arg int64 [rows]) of bf16 logits [rows, vocab]
    (fdl_softmax_confidence): without `token`, the float64 softmax maximum of each row and
    the first index of its maximum (torch.max(softmax(logits.double(), -1), -1)); with
    `token` [rows] int64, the float64 softmax probability of that token."""
    _need(logits, "logits", BF16, 2)
    dev = logits.device
    n, vocab = logits.shape
    if token is not None:
        _need(token, "token", torch.int64, 1, dev)
        if token.shape[0] != n:
            raise _lib.FdlError(_lib.FDL_ERR_SHAPE, "token must have one entry per row")
    prob = torch.empty(n, dtype=torch.float64, device=dev)
    arg = torch.empty(n, dtype=torch.int64, device=dev)
    _lib.call("fdl_softmax_confidence", logits.data_ptr(), n, vocab, _ptr(token),
              prob.data_ptr(), arg.data_ptr(), _stream(logits))
    return prob, arg
