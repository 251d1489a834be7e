"""Decode scheduler of Flash-dLLM (Flash-Cache + Flash-Verify), restated over the HIP kernels.

`generate_with_Flash_dLLM` keeps the reference's signature and decisions
(llada/generate.py:61-472):
  * slot layout: sequence j owns cache rows [j*L, (j+1)*L) with
    L = ((max prompt + gen + block_m) // 128 + 1) * 128 (:76-79), k_end = seqlen_k (:122);
  * step 0 recomputes every slot (masked block + all other slots tracked, :125-134);
  * each step: forward over the packed rows (masked rows of all sequences, then tracked
    rows, :146-167, :439-467); confidence = max of the float64 softmax of the masked rows'
    logits; accept the rows with confidence >= threshold, at least one (:335-350);
  * Flash-Verify (:210-303, :312-333): the not-accepted masked rows, by confidence, become
    S = min(len - keep, block_m / 2) candidates; a second forward over
    [T fill rows, S draft rows, S mask rows] (T = 2 block_m - 2S) against all other cache
    slots under the verify mask; the candidates' draft tokens are accepted as the prefix
    whose cumulative probability stays >= gamma;
  * refresh (:364-381): the previously decoded slots are re-ordered by attention
    importance (ascending) and the tracked set for the next step is the last
    track_num * block_m decoded entries plus the look-ahead window;
  * finished sequences are replaced by the next prompt (:405-427).

With `kv_pages`, the K/V caches are a paged pool (fdl.schedule.PagePool) instead of the
fixed stride: host arrays keep the logical layout (slot j*L + p), the caches, attn_scores
and the kernels' slot arguments use pool slots through the page table, and a finished
sequence's pages go back to the pool.

What differs from the reference, on purpose:
  * bookkeeping (token ids, full_pos, per-sequence counters) lives in host numpy arrays,
    so a step synchronises with the GPU twice (pass-1 confidences, verify probabilities;
    the importance ranking is read back after one of them) instead of at every `.item()`;
  * the logits are computed only for the rows the step reads (the masked rows, the verify
    mask-view rows); the LM head is row-wise, so the values are the same;
  * the importance ranking runs on the GPU (fdl_importance_rank) with ties broken toward
    the lower slot; the reference's torch.sort leaves ties unordered;
  * sorting the confidences uses a stable order (ties keep row order);
  * a masked block cut short by the end of the slot row is handled (the reference's
    verify pass fails on it with a shape mismatch, generate.py:215/:235);
  * without a tokenizer, responses[i] holds the generated token ids.
"""
from __future__ import annotations

import inspect
import math
import time
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

from . import ops
from .schedule import (DEFAULT_PAGE_LOG2, PagedRows, PagePool, SeqRows, contiguous_page_table,
                       make_plan, pages_reserved)


def get_rotary_embedding(seq_len: int, dim: int, rope_theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """sin, cos float32 [seq_len, dim] (llada/generate.py:44-50).

    The reference's float32 steps (inv_freq = 1 / theta^(arange(0, dim, 2) / dim), freqs =
    p * inv_freq, cat(freqs, freqs) -> sin, cos), each correctly rounded: every step is
    evaluated in float64 and rounded to float32 once, so the table does not depend on the
    device's float32 pow and sin (which may be an ulp or two off; an ulp of inv_freq moves
    the angle at position 900 by ~5e-5)."""
    f64 = torch.float64
    e = torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim
    inv_freq = (1.0 / (rope_theta ** e.to(f64)).float().to(f64)).float()
    seq = torch.arange(seq_len, device=device, dtype=f64)
    freqs = torch.outer(seq, inv_freq.to(f64)).float()
    positions = torch.cat((freqs, freqs), dim=-1).to(f64)
    return positions.sin().float(), positions.cos().float()


def conf_order(conf: np.ndarray) -> np.ndarray:
    """Row order of `x0_p.sort(descending=True)` (generate.py:230, :343): descending, NaN
    before every number (torch sorts NaN as the largest value), ties in row order (the
    reference's sort is not declared stable; this fixes its tie order)."""
    conf = np.asarray(conf, dtype=np.float64)
    nan = np.isnan(conf)
    return np.lexsort((-np.where(nan, 0.0, conf), ~nan))


def make_blocks(j: int, seqlen_k, start_m: int, end_m: int, block_m: int) -> np.ndarray:
    """(batch, k_end, q_start, q_end) rows over [start_m, end_m) (llada/generate.py:52-58)."""
    starts = np.arange(start_m, end_m, block_m, dtype=np.int64)
    ends = np.minimum(starts + block_m, end_m)
    return np.stack([np.full_like(starts, j), np.full_like(starts, seqlen_k[j]), starts, ends], axis=1)


def verify_mask(T: int, S: int, block_m: int) -> np.ndarray:
    """The [2 block_m, 2 block_m] verify mask in closed form (llada/generate.py:262-269):
    fill rows never see the drafts; draft i sees drafts j <= i and masks j > i; mask i sees
    drafts j < i and masks j >= i; every other entry is True."""
    n = 2 * block_m
    m = np.ones((n, n), dtype=bool)
    m[:T, T:T + S] = False
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    m[T:T + S, T:T + S] = i >= j
    m[T:T + S, T + S:T + 2 * S] = i < j
    m[T + S:T + 2 * S, T:T + S] = i > j
    m[T + S:T + 2 * S, T + S:T + 2 * S] = i <= j
    return m


@dataclass
class DecodeStats:
    steps: int = 0
    forwards: int = 0
    rows: int = 0
    verify_accepted: int = 0  # tokens accepted by the verify pass
    decoded: int = 0          # tokens decoded (both passes), finished or not
    host_syncs: int = 0        # host waits for the GPU (device-scheduled decode)
    fused_rank_steps: int = 0  # steps whose ranking folded in the last layer's reduction
    split_rank_steps: int = 0  # steps that reduced first (a ranked row without importance)
    wall_s: float = 0.0
    per_step_s: list = field(default_factory=list)
    per_step_decoded: list = field(default_factory=list)  # tokens decoded in each step
    # host schedule: the token ids x[b * L + p] when the loop returned (a bounded decode
    # stopped by max_steps included; [MASK] where nothing was decoded)
    x_final: np.ndarray = field(default=None, repr=False)


class _Seq:
    __slots__ = ("prompt", "nd", "seqlen_k", "masked", "tracked", "predicted_length",
                 "decoded_eos", "keep_rows", "verify_pos")

    def __init__(self):
        # an idle row: no prompt, no rows
        self.prompt, self.nd, self.seqlen_k, self.predicted_length = -1, 0, 0, 0
        self.decoded_eos, self.keep_rows = -1, 0
        self.masked = self.tracked = self.verify_pos = np.zeros(0, np.int64)


def _to_dev(a: np.ndarray, device, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


def _to_dev_many(arrays: list, device) -> list:
    """Uploads several host arrays through one pinned buffer and one copy (16-byte aligned
    slices; dtypes and shapes kept). The step's table uploads sit between two GPU
    synchronisations, so each separate copy is GPU idle time."""
    arrays = [np.ascontiguousarray(a) for a in arrays]
    if torch.device(device).type != "cuda":
        return [torch.from_numpy(a.copy()).to(device) for a in arrays]
    offs, total = [], 0
    for a in arrays:
        offs.append(total)
        total += (a.nbytes + 15) // 16 * 16
    host = torch.empty(max(total, 16), dtype=torch.uint8, pin_memory=True)
    hv = host.numpy()
    for a, o in zip(arrays, offs):
        hv[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
    buf = host.to(device, non_blocking=True)
    return [buf[o:o + a.nbytes].view(torch.from_numpy(np.empty(0, a.dtype)).dtype).view(a.shape)
            for a, o in zip(arrays, offs)]


def _accepts_logit_rows(model) -> bool:
    """True if model.forward takes a `logit_rows` argument (fdl.model's LLaDAModelLM does; the
    reference's does not)."""
    try:
        params = inspect.signature(model.forward).parameters
    except (TypeError, ValueError):
        return False
    return "logit_rows" in params or any(p.kind == p.VAR_KEYWORD for p in params.values())


@torch.no_grad()
def generate_with_Flash_dLLM(model, prompts, prompt_lengths, batch_size, responses, n_steps, steps=128,
                             gen_length=128, block_length=128, temperature=0., remasking='low_confidence',
                             mask_id=126336, threshold=0.9, gamma=0.9, track_num=4, mask_num=4, eos_id=126081,
                             verify=False, sliding_window=True, is_instruct=True, tokenizer=None,
                             stop_tokens=None, stats: DecodeStats | None = None, use_gpu_rank: bool = True,
                             rows_only: bool = True, max_steps: int | None = None,
                             kv_pages: int | None = None, device_schedule: bool = False):
    """Returns (responses, num_tokens, max_num_tokens) like llada/generate.py:472.

    use_gpu_rank: rank the decoded slots with fdl_importance_rank (else numpy, same order).
    rows_only: run the LM head only on the rows the step reads (else on every row).
    max_steps: stop after this many denoising steps (benchmarking a bounded sample;
        stats.decoded then counts the tokens decoded so far).
    device_schedule: keep the decode's bookkeeping on the device (fdl.device_decode; one
        host synchronisation per step). Needs the HIP driver on a GPU, the device ranking and
        no tokenizer; the decisions are the same, with or without kv_pages.
    kv_pages: K/V caches as a pool of this many 32-slot pages (None: the fixed stride of L
        slots per sequence). A sequence starts with the pages of its seqlen_k key slots and
        gets more when its masked block reaches past them; admission reserves pages up to
        max(seqlen_k, prompt + gen + block_m - 1) positions, the reach of a decode that
        does not accept tokens past prompt + gen ahead of earlier ones (beyond the
        reservation a sequence grows from the free pages, MemoryError if there are none).
        A finished sequence's pages return to the pool; prompts are admitted in order into
        idle rows while their reservation fits (MemoryError if a prompt does not fit an
        empty pool). With pages for every row the decode is the fixed-stride decode, token
        for token.
    """
    dev = model.device
    cfg = model.config
    stats = stats if stats is not None else DecodeStats()
    if device_schedule:
        if (torch.device(dev).type != "cuda" or tokenizer is not None
                or not use_gpu_rank or not rows_only or not _accepts_logit_rows(model)):
            raise ValueError("device_schedule needs a GPU model with logit rows, the device "
                             "ranking and no tokenizer")
        from .device_decode import generate_device_scheduled
        return generate_device_scheduled(model, prompts, prompt_lengths, batch_size, responses,
                                         n_steps, gen_length, block_length, mask_id, threshold,
                                         gamma, track_num, mask_num, eos_id, verify, stats,
                                         max_steps, kv_pages)
    bm = block_length
    bn = 128
    B = batch_size
    L = ((max(prompt_lengths) + gen_length + bm) // bn + 1) * bn
    d_model, n_layers, n_heads = cfg.d_model, cfg.n_layers, cfg.n_heads
    rows_only = rows_only and _accepts_logit_rows(model)
    row_kw = (lambda rows: {"logit_rows": rows}) if rows_only else (lambda rows: {})
    t_start = time.perf_counter()

    x = np.full(B * L, mask_id, dtype=np.int64)
    x_draft = np.full(B * L, mask_id, dtype=np.int64)
    full_pos = np.arange(B * L, dtype=np.int64).reshape(B, L)
    paged = kv_pages is not None
    PL = DEFAULT_PAGE_LOG2
    if paged:
        pool = PagePool(kv_pages, PL)
        rows_p = PagedRows(pool, B, L)
        page_table = rows_p.page_table
        n_slots = pool.n_slots
    else:
        page_table = contiguous_page_table(B, L)
        n_slots = B * L
    attn_scores = torch.zeros(n_slots, dtype=torch.float32, device=dev)
    num_tokens = 0
    max_num_tokens = 0
    active = [-1] * B
    seqs = [_Seq() for _ in range(B)]
    start_layer = [-1] * B
    count = 0

    def seqlen_k_of(i: int) -> int:
        return (int(prompt_lengths[i]) + gen_length) // bn * bn + bn

    def pages_needed(i: int) -> int:
        """Pages reserved at admission (positions a decode normally reaches)."""
        return pages_reserved(pool, L, seqlen_k_of(i), int(prompt_lengths[i]), gen_length, bm)

    def phys(a: np.ndarray) -> np.ndarray:
        """Cache slots of logical slots j * L + p."""
        return rows_p.phys(a) if paged else a

    def idle(j: int) -> None:
        s = seqs[j]
        active[j] = -1
        s.masked = np.zeros(0, np.int64)
        s.tracked = np.zeros(0, np.int64)
        s.verify_pos = np.zeros(0, np.int64)

    def release(j: int) -> None:
        if paged:
            rows_p.release(j)

    def admit(j: int) -> bool:
        """Loads the next prompt into row j if there is one and its pages fit."""
        nonlocal count
        if count >= len(prompts):
            return False
        if paged:
            need = pages_needed(count)
            if not rows_p.fits(need):
                return False
            rows_p.admit(j, need, seqlen_k_of(count))
        load_prompt(j, count)
        count += 1
        return True

    def load_prompt(j: int, i: int) -> None:
        pl = int(prompt_lengths[i])
        s = seqs[j]
        x[j * L:(j + 1) * L] = mask_id
        x[j * L:j * L + pl] = np.asarray(prompts[i], dtype=np.int64)[:pl]
        x[j * L + pl + gen_length:(j + 1) * L] = eos_id
        x_draft[j * L:(j + 1) * L] = mask_id
        x_draft[j * L:j * L + pl] = x[j * L:j * L + pl]
        full_pos[j] = np.arange(j * L, (j + 1) * L)
        s.prompt = i
        s.nd = pl
        s.seqlen_k = (pl + gen_length) // bn * bn + bn
        s.masked = full_pos[j, s.nd:s.nd + bm].copy()
        s.tracked = np.concatenate([full_pos[j, :s.nd], full_pos[j, s.nd + bm:s.seqlen_k]])
        s.predicted_length = s.nd + gen_length + j * L
        s.decoded_eos = -1
        s.keep_rows = 0
        s.verify_pos = np.zeros(0, np.int64)
        active[j] = i
        start_layer[j] = -1

    for j in range(B):
        if not admit(j):
            idle(j)

    sin, cos = get_rotary_embedding(L, d_model // n_heads, cfg.rope_theta, dev)
    rope = [sin.repeat(B, 1).contiguous(), cos.repeat(B, 1).contiguous()]
    for blk in model.model.transformer.blocks:
        blk.k_cache = torch.empty((n_slots, d_model), dtype=model.dtype, device=dev)
        blk.v_cache = torch.empty((n_slots, d_model), dtype=model.dtype, device=dev)
    empty_i32 = torch.zeros(0, dtype=torch.int32, device=dev)
    # Device ranking (use_gpu_rank): the ranked segment of sequence j is full_pos[j, :n_j],
    # with n_j the decoded count before the step's last acceptance stage (the pass-1 count
    # with Flash-Verify, the pre-step count without). Both that segment and attn_scores are
    # final once that stage is known, so the rank kernel is enqueued then, through pinned
    # buffers, and read back after the synchronization that follows anyway (the verify
    # probabilities, or the pass-1 confidences).
    gpu_rank = use_gpu_rank
    if gpu_rank:
        if torch.device(dev).type != "cuda":
            raise ValueError("use_gpu_rank ranks on the GPU; the model is on " + str(dev))
        full_pos_d = torch.empty(B * L, dtype=torch.int64, device=dev)
        fp_up = torch.empty(B * L, dtype=torch.int64, pin_memory=True)
        fp_back = torch.empty(B * L, dtype=torch.int64, pin_memory=True)
        seg_up = torch.empty((2, B, 2), dtype=torch.int32, pin_memory=True)
        seg_d = torch.empty((2, B, 2), dtype=torch.int32, device=dev)
        rank_done = torch.cuda.Event()
    rank_len = [0] * B

    def enqueue_rank() -> None:
        """Ranks full_pos[j, :seqs[j].nd] of every active sequence on the device."""
        act = [j for j in range(B) if active[j] != -1]
        if not act:
            return
        rank_done.synchronize()  # the previous step's copies through fp_up / fp_back are done
        fp_up.numpy()[:] = phys(full_pos.reshape(-1))
        seg = seg_up.numpy()  # [0]: (start, len) of each segment, [1]: (row, seqlen_k)
        for i, j in enumerate(act):
            seg[0, i] = (j * L, seqs[j].nd)
            seg[1, i] = (j, seqs[j].seqlen_k)
            rank_len[j] = seqs[j].nd
        full_pos_d.copy_(fp_up, non_blocking=True)
        seg_d.copy_(seg_up, non_blocking=True)
        # The last layer's head reduction, when the driver deferred it, rides in the ranking:
        # it covers the keys [0, seqlen_k) of the ranked rows, which are the rows with
        # importance rows (every active row has a masked block); otherwise it runs first.
        part, scale = plan.deferred_importance or (None, 1.0)
        if part is not None and not all(j in imp_rows for j in act):
            ops.importance_accumulate(part, plan, scale, attn_scores)
            part = None
            stats.split_rank_steps += 1
        elif part is not None:
            stats.fused_rank_steps += 1
        n = len(act)
        ops.importance_rank(attn_scores, full_pos_d, seg_d[0, :n], int(seg[0, :n, 1].max()),
                            imp_part=part, scale=scale, plan=plan, seg_keys=seg_d[1, :n])
        fp_back.copy_(full_pos_d, non_blocking=True)
        rank_done.record()

    while True:
        t_step = time.perf_counter()
        if paged:
            for j in range(B):
                if active[j] == -1 and not admit(j):
                    break
        if all(a == -1 for a in active):
            if count >= len(prompts):
                break
            raise MemoryError(f"prompt {count} needs {pages_needed(count)} pages; the pool has "
                              f"{kv_pages}")
        if paged:
            # pages for every position this step touches (queries and cache writes)
            for j in range(B):
                if active[j] != -1:
                    s = seqs[j]
                    hi = max(int(s.masked.max()) if len(s.masked) else -1,
                             int(s.tracked.max()) if len(s.tracked) else -1)
                    if hi >= 0:
                        rows_p.grow(j, hi - j * L + 1)
        # ---- pack the step's query rows: masked rows, then tracked rows (:439-467)
        masked_blocks, tracked_blocks, seq_rows = [], [], []
        acc = 0
        rows_of = {}
        for j in range(B):
            if active[j] != -1 and len(seqs[j].masked):
                n = len(seqs[j].masked)
                masked_blocks.append(make_blocks(j, [s.seqlen_k for s in seqs], acc, acc + n, bm))
                rows_of[j] = [np.arange(acc, acc + n)]
                acc += n
        n_masked_rows = acc
        for j in range(B):
            if active[j] != -1 and len(seqs[j].tracked):
                n = len(seqs[j].tracked)
                tracked_blocks.append(make_blocks(j, [s.seqlen_k for s in seqs], acc, acc + n, bm))
                rows_of.setdefault(j, [np.zeros(0, np.int64)]).append(np.arange(acc, acc + n))
                acc += n
        order_j = [j for j in range(B) if active[j] != -1 and (len(seqs[j].masked) or len(seqs[j].tracked))]
        qpos = np.concatenate([seqs[j].masked for j in range(B) if active[j] != -1 and len(seqs[j].masked)] +
                              [seqs[j].tracked for j in range(B) if active[j] != -1 and len(seqs[j].tracked)])
        for j in order_j:
            r = rows_of[j]
            rows = np.concatenate(r)
            seq_rows.append(SeqRows(batch=j, k_end=seqs[j].seqlen_k, rows=rows,
                                    n_imp=len(r[0]) if len(seqs[j].masked) else 0))
        plan = make_plan(seq_rows, page_table, device=dev)
        plan.defer_last_importance = gpu_rank
        imp_rows = {sr.batch for sr in seq_rows if sr.n_imp > 0}
        mb = np.concatenate(masked_blocks) if masked_blocks else np.zeros((0, 4), np.int64)
        tb = np.concatenate(tracked_blocks) if tracked_blocks else np.zeros((0, 4), np.int64)
        mb_t, tb_t = torch.from_numpy(mb), torch.from_numpy(tb)
        if paged:
            qpos_d, x_query, plan.kv_slot = _to_dev_many([qpos, x[qpos], phys(qpos)], dev)
        else:
            qpos_d, x_query = _to_dev_many([qpos, x[qpos]], dev)
        x_query = x_query[None]
        positions = [qpos_d, empty_i32, rope, plan, attn_scores, []]
        lengths = [start_layer, None, mb_t, tb_t, torch.cat([mb_t, tb_t]), active, len(mb), L, bm, bn, None,
                   False]
        logits = model(x_query, use_cache=True, lengths=lengths, positions=positions,
                       **row_kw(torch.arange(n_masked_rows, device=dev))).logits.squeeze(0)
        logits = logits[:n_masked_rows]
        stats.forwards += 1
        stats.rows += len(qpos)
        if logits.dtype == torch.bfloat16 and logits.is_cuda and logits.shape[0] > 0:
            x0_p_all, x0_all = ops.softmax_confidence(logits.contiguous())
        else:
            x0_p_all, x0_all = torch.max(F.softmax(logits.to(torch.float64), dim=-1), dim=-1)
        if gpu_rank and not verify:
            enqueue_rank()
        x0_p_all = x0_p_all.cpu().numpy()
        x0_all = x0_all.cpu().numpy()
        if len(x0_all) and (x0_all.min() < 0 or x0_all.max() >= logits.shape[-1]):
            raise RuntimeError(f"token ids outside [0, {logits.shape[-1]}) from the LM head")
        del logits

        keep_num = [0] * B
        acc_masked = 0
        if verify:
            x_verify, key_pos, masks, vblocks, vq_pos = [], [], [], [], []
            acc_q = acc_k = 0
            verify_meta = {}
            for j in range(B):
                if active[j] == -1:
                    continue
                s = seqs[j]
                nm = len(s.masked)
                # The reference reads block_m rows here (generate.py:215); a masked block
                # that reached the end of the slot row is shorter, and the reference then
                # fails on a shape mismatch (:235). Reading the block's own rows is the
                # same whenever the reference is defined.
                rows = slice(acc_masked, acc_masked + min(nm, bm))
                acc_masked += nm
                s.masked = s.masked[:bm]
                conf = x0_p_all[rows].copy()
                toks = x0_all[rows]
                if s.decoded_eos != -1:
                    lmask = s.masked >= s.predicted_length
                    conf[lmask] = 0
                    length_num = len(s.masked) - int(lmask.sum())
                else:
                    length_num = len(s.masked)
                order = conf_order(conf)
                keep = max(int((conf >= threshold).sum()), 1)
                x_draft[s.masked] = toks
                full_pos[j, s.nd:s.nd + len(s.masked)] = s.masked[order]
                new_pos = full_pos[j, s.nd:s.nd + keep].copy()
                new_tok = toks[order][:keep]
                x[new_pos] = new_tok
                s.nd += keep
                stats.decoded += keep
                if s.decoded_eos == -1:
                    eos_pos = new_pos[new_tok == eos_id]
                    if len(eos_pos):
                        s.decoded_eos = int(eos_pos.max())
                        s.predicted_length = s.decoded_eos + 1
                S = min(max(length_num - keep, 0), bm // 2)
                T = 2 * bm - 2 * S
                if s.nd < T:
                    raise NotImplementedError(
                        f"verify needs at least {T} decoded slots before the block (have {s.nd}); "
                        "use prompts of at least 2 * block_length tokens")
                s.keep_rows = T
                cand = full_pos[j, s.nd:s.nd + S].copy()
                fill = full_pos[j, s.nd - T:s.nd].copy()
                x_verify.append(np.concatenate([x[fill], x_draft[cand], x[cand]]))
                s.verify_pos = np.concatenate([fill, cand, cand])
                keys = np.concatenate([full_pos[j, :s.nd - T], full_pos[j, s.nd + S:s.seqlen_k]])
                key_pos.append(keys)
                m = verify_mask(T, S, bm)
                masks.append(m)
                vblocks.append((acc_k, acc_k + len(keys), acc_q, acc_q + len(s.verify_pos)))
                verify_meta[j] = (acc_q, T, S)
                acc_q += len(s.verify_pos)
                acc_k += len(keys)
            if gpu_rank:
                enqueue_rank()
            vq = np.concatenate([seqs[j].verify_pos for j in range(B) if active[j] != -1])
            # the mask-view rows [T+S, T+2S) of each block are read (:318); the LM head runs on
            # the block's last block_m // 2 rows, which hold them (the last S), so every block
            # gives the product the same number of rows whatever its S
            tail = bm // 2
            lr = np.concatenate([np.arange(a + 2 * bm - tail, a + 2 * bm) for (a, T, S) in verify_meta.values()])
            xv = np.concatenate(x_verify)
            tail_tok = np.concatenate([np.where(np.arange(tail) >= tail - S,
                                                xv[np.clip(a + T + np.arange(tail) - (tail - S), a, None)], -1)
                                       for (a, T, S) in verify_meta.values()])
            vblocks_d, key_pos_d, mask_d, vq_d, xq, lr_d, draft_tok = _to_dev_many(
                [np.asarray(vblocks, np.int32), phys(np.concatenate(key_pos).astype(np.int64)),
                 np.concatenate(masks), vq, xv, lr.astype(np.int64), tail_tok.astype(np.int64)], dev)
            xq = xq[None]
            positions = [vq_d, key_pos_d, rope, None, attn_scores, mask_d]
            lengths = [start_layer, vblocks_d, None, tb_t, None, active, len(mb), L, bm, bn, None, True]
            if any(S for (_, _, S) in verify_meta.values()):
                vlog = model(xq, use_cache=True, lengths=lengths, positions=positions,
                             **row_kw(lr_d)).logits.squeeze(0)
                if not rows_only:
                    vlog = vlog[lr_d]
                stats.forwards += 1
                stats.rows += len(vq)
                if vlog.dtype == torch.bfloat16 and vlog.is_cuda:
                    pv = ops.softmax_confidence(vlog.contiguous(), draft_tok)[0]
                else:
                    pv = F.softmax(vlog.to(torch.float64), dim=-1).gather(
                        1, draft_tok.clamp(min=0)[:, None]).view(-1)
                    pv = torch.where(draft_tok < 0, torch.zeros_like(pv), pv)
                pv = pv.cpu().numpy()
                del vlog
            else:
                pv = np.zeros(tail * len(verify_meta))
            off = 0
            for j, (a, T, S) in verify_meta.items():
                s = seqs[j]
                off += tail
                if S == 0:
                    keep_num[j] = 0
                    continue
                probs = pv[off - S:off].copy()
                if s.decoded_eos != -1:
                    probs[s.verify_pos[T:T + S] >= s.predicted_length] = 0
                cp = np.cumprod(probs)
                keep = int((cp >= gamma).sum())
                keep_num[j] = keep
                stats.verify_accepted += keep
                stats.decoded += keep
                if keep > 0:
                    new_pos = full_pos[j, s.nd:s.nd + keep].copy()
                    new_tok = x_draft[s.verify_pos[T:T + keep]]
                    x[new_pos] = new_tok
                    s.nd += keep
                    if s.decoded_eos == -1:
                        eos_pos = new_pos[new_tok == eos_id]
                        if len(eos_pos):
                            s.decoded_eos = int(eos_pos.max())
                            s.predicted_length = s.decoded_eos + 1
        else:
            for j in range(B):
                if active[j] == -1:
                    continue
                s = seqs[j]
                nm = len(s.masked)
                rows = slice(acc_masked, acc_masked + nm)
                acc_masked += nm
                conf = x0_p_all[rows].copy()
                toks = x0_all[rows]
                if s.decoded_eos != -1:
                    conf[s.masked >= s.predicted_length] = 0
                order = conf_order(conf)
                keep = max(int((conf[order] >= threshold).sum()), 1)
                full_pos[j, s.nd:s.nd + nm] = s.masked[order]
                new_pos = full_pos[j, s.nd:s.nd + keep].copy()
                new_tok = toks[order][:keep]
                keep_num[j] = keep
                x[new_pos] = new_tok
                s.nd += keep
                stats.decoded += keep
                if s.decoded_eos == -1:
                    eos_pos = new_pos[new_tok == eos_id]
                    if len(eos_pos):
                        s.decoded_eos = int(eos_pos.max())
                        s.predicted_length = s.decoded_eos + 1

        # ---- importance refresh (:364-381) and sequence completion (:385-433)
        cont = []
        for j in range(B):
            if active[j] == -1:
                continue
            s = seqs[j]
            n_steps[active[j]] += 1
            if (full_pos[j, s.nd:] < s.predicted_length).any():
                cont.append(j)
            else:
                i = active[j]
                pl = int(prompt_lengths[i])
                gen_ids = x[j * L + pl: j * L + s.nd].copy()
                if tokenizer is not None:
                    text = tokenizer.decode(gen_ids, skip_special_tokens=False)
                    for stop_seq in (stop_tokens or []):
                        if stop_seq in text:
                            text = text.split(stop_seq)[0]
                    ids = tokenizer(text)["input_ids"]
                    responses[i] = tokenizer.decode(ids, skip_special_tokens=True)
                else:
                    responses[i] = gen_ids.tolist()
                num_tokens += s.nd - pl
                max_num_tokens += gen_length
                release(j)
                if not admit(j):
                    idle(j)
        if cont:
            if gpu_rank:
                rank_done.synchronize()
                fp = fp_back.numpy().reshape(B, L)
                for j in cont:
                    n = seqs[j].nd - keep_num[j]
                    if n != rank_len[j]:
                        raise RuntimeError(f"ranked {rank_len[j]} slots of sequence {j}, "
                                           f"the refresh reads {n}")
                    full_pos[j, :n] = rows_p.logical_of[fp[j, :n]] if paged else fp[j, :n]
            else:
                sc = attn_scores.cpu().numpy()
                for j in cont:
                    n = seqs[j].nd - keep_num[j]
                    seg = full_pos[j, :n]
                    ph = phys(seg)
                    v = sc[ph]
                    v = np.where(v == 0, np.float32(0), v)
                    full_pos[j, :n] = seg[np.lexsort((-ph, v))]
            for j in cont:
                s = seqs[j]
                s.masked = full_pos[j, s.nd:s.nd + bm].copy()
                if track_num < 0:
                    s.tracked = np.concatenate([full_pos[j, :s.nd], full_pos[j, s.nd + bm:s.seqlen_k]])
                else:
                    t0 = max(0, s.nd - track_num * bm)
                    t1 = min(s.seqlen_k, s.nd + bm * mask_num)
                    s.tracked = np.concatenate([full_pos[j, t0:s.nd], full_pos[j, s.nd + bm:t1]])
                start_layer[j] = n_layers
        stats.steps += 1
        stats.per_step_s.append(time.perf_counter() - t_step)
        stats.per_step_decoded.append(stats.decoded - sum(stats.per_step_decoded))
        if all(a == -1 for a in active) and count >= len(prompts):
            break
        if max_steps is not None and stats.steps >= max_steps:
            break
        attn_scores.zero_()

    if torch.device(dev).type == "cuda":
        torch.cuda.synchronize(dev)
    stats.wall_s = time.perf_counter() - t_start
    stats.x_final = x.copy()
    return responses, num_tokens, max_num_tokens
