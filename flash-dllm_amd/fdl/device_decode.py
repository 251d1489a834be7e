"""Flash-Cache + Flash-Verify decoding with the bookkeeping on the device (fdl_sched_*).

The same decisions as fdl.generate.generate_with_Flash_dLLM (llada/generate.py:61-472), but
the per-step state (token ids, the slot order full_pos, the per-sequence counters) lives in
device memory and is updated by the scheduler kernels, so a denoising step is enqueued
without waiting for the GPU and the host synchronises once per step:

    pack (previous step) -> [sync: row counts, completions] -> pass-1 forward over the packed
    rows -> confidences -> pass-1 acceptance + verify lists -> verify forward -> draft-token
    probabilities -> verify acceptance -> importance ranking (in place on full_pos) -> pack

Completions and refills (generate.py:385-433) are handled on the host at the sync, with a
second synchronisation only on a step where a new prompt is admitted. The verify pass reads
the LM head on the last block_m / 2 rows of every verify block (its mask rows are the last S
of them), as the host scheduler does.

With kv_pages the K/V caches are a paged pool (fdl.schedule.PagedRows, the host loop's
bookkeeping): the scheduler's state stays in logical slots j * L + p; at the step's
synchronisation the host grows each row's pages to the highest position its next rows query
(FDL_SEQ_HI, written by fdl_sched_pack) and refreshes the device page table, and the forward
maps its slots on the device: the K/V write slots of the packed rows and the verify key list
through the page table, the ranking's segments to pool slots (pool-indexed importance, ties
broken by pool slot, as the host loop does) and back through the pool slot -> logical table.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np
import torch

from . import lib as _lib
from . import ops
from .schedule import (DEFAULT_PAGE_LOG2, AttnPlan, DeviceAttnPlan, PagedRows, PagePool,
                       contiguous_page_table, pages_reserved)

I64, I32 = torch.int64, torch.int32


class DeviceScheduler:
    """Device buffers and launch wrappers of the fdl_sched_* kernels."""

    def __init__(self, n_seq: int, max_length: int, block_m: int, track_num: int, mask_num: int,
                 verify: bool, mask_id: int, eos_id: int, threshold: float, gamma: float, device):
        B, L, bm = n_seq, max_length, block_m
        dev = torch.device(device)
        self.B, self.L, self.bm, self.dev = B, L, bm, dev
        self.x = torch.full((B * L,), mask_id, dtype=I64, device=dev)
        self.x_draft = torch.full((B * L,), mask_id, dtype=I64, device=dev)
        self.full_pos = torch.arange(B * L, dtype=I64, device=dev)
        self.seq = torch.zeros((B, _lib.SCHED_SEQ_FIELDS), dtype=I32, device=dev)
        self.seq[:, _lib.SEQ_ACTIVE] = -1
        self.summary = torch.zeros(_lib.SCHED_SUMMARY_FIELDS, dtype=I32, device=dev)
        self.q_cap = B * (L + bm)
        self.work_cap = B * (L // 256 + 3)
        self.qpos = torch.empty(self.q_cap, dtype=I64, device=dev)
        self.xq = torch.empty(self.q_cap, dtype=I64, device=dev)
        self.row_idx = torch.empty(self.q_cap, dtype=I32, device=dev)
        self.work = torch.empty((self.work_cap, 8), dtype=I32, device=dev)
        self.seg = torch.empty((B, 2), dtype=I32, device=dev)
        self.vpos = torch.empty(B * 2 * bm, dtype=I64, device=dev)
        self.xv = torch.empty(B * 2 * bm, dtype=I64, device=dev)
        self.key_pos = torch.empty(B * L, dtype=I64, device=dev)
        self.vblocks = torch.empty((B, 4), dtype=I32, device=dev)
        self.vmeta = torch.empty((B, 2), dtype=I32, device=dev)
        self.draft_tok = torch.empty(B * (bm // 2), dtype=I64, device=dev)
        self.state = _lib.SchedState(
            *(t.data_ptr() for t in (self.x, self.x_draft, self.full_pos, self.seq, self.summary,
                                     self.qpos, self.xq, self.row_idx, self.work, self.seg,
                                     self.vpos, self.xv, self.key_pos, self.vblocks, self.vmeta,
                                     self.draft_tok)),
            B, L, self.q_cap, self.work_cap, bm, track_num, mask_num, 1 if verify else 0,
            eos_id, float(threshold), float(gamma))
        self.page_table = contiguous_page_table(B, L)
        self.page_table_d = torch.from_numpy(self.page_table).to(dev)
        # host copies read at the step's synchronisation
        self.seq_h = torch.empty((B, _lib.SCHED_SEQ_FIELDS), dtype=I32, pin_memory=True)
        self.summary_h = torch.empty(_lib.SCHED_SUMMARY_FIELDS, dtype=I32, pin_memory=True)

    def _stream(self) -> int:
        return torch._C._cuda_getCurrentRawStream(self.dev.index)

    def pass1(self, conf: torch.Tensor, tok: torch.Tensor) -> None:
        _lib.call("fdl_sched_pass1", ctypes.byref(self.state), conf.data_ptr(), tok.data_ptr(),
                  self._stream())

    def verify_accept(self, prob: torch.Tensor) -> None:
        _lib.call("fdl_sched_verify_accept", ctypes.byref(self.state), prob.data_ptr(),
                  self._stream())

    def pack(self) -> None:
        _lib.call("fdl_sched_pack", ctypes.byref(self.state), self._stream())

    def read(self, stats=None) -> tuple[np.ndarray, np.ndarray]:
        """(per-sequence fields, summary): the step's synchronisation."""
        if stats is not None:
            stats.host_syncs += 1
        self.seq_h.copy_(self.seq, non_blocking=True)
        self.summary_h.copy_(self.summary, non_blocking=True)
        torch.cuda.current_stream(self.dev).synchronize()
        return self.seq_h.numpy().copy(), self.summary_h.numpy().copy()

    def plan(self, summ: np.ndarray, importance: bool) -> AttnPlan:
        n_long, n_mid, n_short = (int(summ[_lib.SUM_N_LONG]), int(summ[_lib.SUM_N_MID]),
                                  int(summ[_lib.SUM_N_SHORT]))
        q = int(summ[_lib.SUM_Q])
        return DeviceAttnPlan(self.work, self.row_idx, q, self.page_table, self.page_table_d,
                              DEFAULT_PAGE_LOG2, n_long, n_mid, n_long + n_mid + n_short,
                              importance)


class DevicePages:
    """Device copies of a paged pool's tables (fdl.schedule.PagedRows) and the slot maps of
    the device-scheduled decode: refreshed from the host tables when they change (at the
    step's synchronisation), used by device ops only (no host wait)."""

    def __init__(self, rows: PagedRows, dev):
        self.rows = rows
        B, P = rows.page_table.shape
        self.L, self.PL = rows.L, rows.PL
        self.page_table_d = torch.zeros((B, P), dtype=I32, device=dev)
        self.logical_of_d = torch.full((rows.pool.n_slots,), -1, dtype=I64, device=dev)
        self._pt_up = torch.empty((B, P), dtype=I32, pin_memory=True)
        self._lo_up = torch.empty(rows.pool.n_slots, dtype=I64, pin_memory=True)
        self._copied = torch.cuda.Event()
        self._version = -1

    def refresh(self) -> None:
        if self._version == self.rows.version:
            return
        self._copied.synchronize()  # the previous upload has left the pinned buffers
        self._pt_up.numpy()[:] = self.rows.page_table
        self._lo_up.numpy()[:] = self.rows.logical_of
        self.page_table_d.copy_(self._pt_up, non_blocking=True)
        self.logical_of_d.copy_(self._lo_up, non_blocking=True)
        self._copied.record()
        self._version = self.rows.version

    def phys(self, logical: torch.Tensor) -> torch.Tensor:
        """Pool slots of logical slots j * L + p (device; entries outside [0, B * L) are
        clamped into it, a position without a page maps into the row's first table entry)."""
        B = self.page_table_d.shape[0]
        lg = logical.clamp(0, B * self.L - 1)
        j, p = lg // self.L, lg % self.L
        page = self.page_table_d[j, p >> self.PL].to(I64)
        return (page << self.PL) | (p & ((1 << self.PL) - 1))


@torch.no_grad()
def generate_device_scheduled(model, prompts, prompt_lengths, batch_size, responses, n_steps,
                              gen_length, block_length, mask_id, threshold, gamma, track_num,
                              mask_num, eos_id, verify, stats, max_steps=None, kv_pages=None):
    """Returns (responses, num_tokens, max_num_tokens) like llada/generate.py:472; the
    responses are the generated token ids."""
    dev = model.device
    cfg = model.config
    bm, bn, B = block_length, 128, batch_size
    L = ((max(prompt_lengths) + gen_length + bm) // bn + 1) * bn
    d_model, n_heads = cfg.d_model, cfg.n_heads
    t_start = time.perf_counter()
    sch = DeviceScheduler(B, L, bm, track_num, mask_num, verify, mask_id, eos_id, threshold,
                          gamma, dev)
    paged = kv_pages is not None
    if paged:
        pool = PagePool(kv_pages, DEFAULT_PAGE_LOG2)
        rows_p = PagedRows(pool, B, L)
        pages = DevicePages(rows_p, dev)
        sch.page_table, sch.page_table_d = rows_p.page_table, pages.page_table_d
        n_slots = pool.n_slots
        sch.key_pos.zero_()  # every entry a valid logical slot for the page-table gather
        fp_pool = torch.empty(B * L, dtype=I64, device=dev)
        col = torch.arange(L, device=dev)
    else:
        n_slots = B * L
    from .generate import get_rotary_embedding
    sin, cos = get_rotary_embedding(L, d_model // n_heads, cfg.rope_theta, dev)
    rope = [sin.repeat(B, 1).contiguous(), cos.repeat(B, 1).contiguous()]
    for blk in model.model.transformer.blocks:
        blk.k_cache = torch.empty((n_slots, d_model), dtype=model.dtype, device=dev)
        blk.v_cache = torch.empty((n_slots, d_model), dtype=model.dtype, device=dev)
    attn_scores = torch.zeros(n_slots, dtype=torch.float32, device=dev)
    empty_i32 = torch.zeros(0, dtype=I32, device=dev)
    empty_blocks = torch.zeros((0, 4), dtype=I64)
    active = [-1] * B
    count = 0
    num_tokens = max_num_tokens = 0
    tail = bm // 2

    def admit(j: int) -> bool:
        nonlocal count
        if count >= len(prompts):
            return False
        i = count
        pl = int(prompt_lengths[i])
        sk = (pl + gen_length) // bn * bn + bn
        if paged:
            need = pages_reserved(pool, L, sk, pl, gen_length, bm)
            if not rows_p.fits(need):
                return False
            rows_p.admit(j, need, sk)
        row = torch.full((L,), mask_id, dtype=I64)
        row[:pl] = torch.as_tensor(prompts[i], dtype=I64)[:pl]
        draft = row.clone()
        row[pl + gen_length:] = eos_id
        sch.x[j * L:(j + 1) * L].copy_(row)
        sch.x_draft[j * L:(j + 1) * L].copy_(draft)
        sch.full_pos[j * L:(j + 1) * L].copy_(torch.arange(j * L, (j + 1) * L, dtype=I64))
        f = np.zeros(_lib.SCHED_SEQ_FIELDS, np.int32)
        f[_lib.SEQ_ACTIVE] = i
        f[_lib.SEQ_ND] = pl
        f[_lib.SEQ_SEQLEN_K] = sk
        f[_lib.SEQ_PRED] = pl + gen_length + j * L
        f[_lib.SEQ_EOS] = -1
        f[_lib.SEQ_FRESH] = 1
        sch.seq[j].copy_(torch.from_numpy(f))
        active[j] = i
        count += 1
        return True

    def idle(j: int) -> None:
        active[j] = -1
        sch.seq[j, _lib.SEQ_ACTIVE] = -1

    def admit_idle() -> bool:
        """Fills idle rows with the next prompts while their pages fit (in order)."""
        got = False
        for j in range(B):
            if active[j] == -1:
                if not admit(j):
                    break
                got = True
        return got

    for j in range(B):
        if not admit(j):
            idle(j)
    sch.pack()
    seq_h, summ = sch.read(stats)
    while True:
        t_step = time.perf_counter()
        if int(summ[_lib.SUM_OVERFLOW]):
            raise RuntimeError("device scheduler: packed rows or work items beyond the buffers")
        if (seq_h[:, _lib.SEQ_ERR] != 0).any():
            raise NotImplementedError(
                f"verify needs at least {2 * bm} decoded slots before the block; use prompts "
                "of at least 2 * block_length tokens")
        # completions (generate.py:385-433)
        admitted = False
        for j in range(B):
            if active[j] == -1 or not seq_h[j, _lib.SEQ_DONE]:
                continue
            i = active[j]
            pl = int(prompt_lengths[i])
            nd = int(seq_h[j, _lib.SEQ_ND])
            responses[i] = sch.x[j * L + pl: j * L + nd].tolist()
            num_tokens += nd - pl
            max_num_tokens += gen_length
            if paged:
                rows_p.release(j)
            if admit(j):
                admitted = True
            else:
                idle(j)
        if paged:
            # idle rows take the next prompts in order while their reservations fit (the host
            # loop's rule: a row whose refill did not fit may take it once others finish)
            admitted = admit_idle() or admitted
        if admitted:
            sch.pack()
            seq_h, summ = sch.read(stats)
        act = [j for j in range(B) if active[j] != -1]
        if not act:
            if paged and count < len(prompts):
                sk = (int(prompt_lengths[count]) + gen_length) // bn * bn + bn
                need = pages_reserved(pool, L, sk, int(prompt_lengths[count]), gen_length, bm)
                raise MemoryError(f"prompt {count} needs {need} pages; the pool has {kv_pages}")
            break
        if paged:
            # pages for every position the step's rows query and write (FDL_SEQ_HI)
            for j in act:
                hi = int(seq_h[j, _lib.SEQ_HI])
                if hi >= 0:
                    rows_p.grow(j, hi + 1)
            pages.refresh()
        for j in act:
            n_steps[active[j]] += 1
        # ---- pass 1 over the packed rows
        Q, nmr = int(summ[_lib.SUM_Q]), int(summ[_lib.SUM_N_MASKED_ROWS])
        imp_rows = {j for j in act if seq_h[j, _lib.SEQ_N_MASKED] > 0}
        plan = sch.plan(summ, importance=bool(imp_rows))
        plan.defer_last_importance = True
        if paged:
            plan.kv_slot = pages.phys(sch.qpos[:Q])  # K/V write slots; qpos picks RoPE rows
        positions = [sch.qpos[:Q], empty_i32, rope, plan, attn_scores, []]
        lengths = [[-1] * B, None, empty_blocks, empty_blocks, empty_blocks, active,
                   len(imp_rows), L, bm, bn, None, False]
        logits = model(sch.xq[:Q][None], use_cache=True, lengths=lengths, positions=positions,
                       logit_rows=torch.arange(nmr, device=dev)).logits.squeeze(0)
        stats.forwards += 1
        stats.rows += Q
        conf, tok = ops.softmax_confidence(logits[:nmr].contiguous())
        del logits
        sch.pass1(conf, tok)
        n_act = len(act)
        if verify:
            nv = n_act * 2 * bm
            lr = torch.cat([torch.arange(a * 2 * bm + 2 * bm - tail, (a + 1) * 2 * bm)
                            for a in range(n_act)]).to(dev)
            keys = pages.phys(sch.key_pos) if paged else sch.key_pos
            positions = [sch.vpos[:nv], keys, rope, None, attn_scores, sch.vmeta[:n_act]]
            lengths = [[-1] * B, sch.vblocks[:n_act], None, empty_blocks, None, active,
                       0, L, bm, bn, None, True]
            vlog = model(sch.xv[:nv][None], use_cache=True, lengths=lengths, positions=positions,
                         logit_rows=lr).logits.squeeze(0)
            stats.forwards += 1
            stats.rows += nv
            prob = ops.softmax_confidence(vlog.contiguous(), sch.draft_tok[:n_act * tail])[0]
            del vlog
            sch.verify_accept(prob)
        # ---- importance ranking of every active row, in place on full_pos (generate.py:364-366)
        seg_keys = torch.tensor([[j, int(seq_h[j, _lib.SEQ_SEQLEN_K])] for j in act], dtype=I32)
        seg_keys = seg_keys.pin_memory().to(dev, non_blocking=True)
        part, scale = plan.deferred_importance or (None, 1.0)
        if part is not None and not all(j in imp_rows for j in act):
            ops.importance_accumulate(part, plan, scale, attn_scores)
            part = None
            stats.split_rank_steps += 1
        elif part is not None:
            stats.fused_rank_steps += 1
        if paged:
            # rank the segments as pool slots (pool-indexed scores, ties to the lower pool
            # slot), then write them back as logical slots; entries outside the segments
            # keep their logical value
            fp_pool.copy_(pages.phys(sch.full_pos))
            ops.importance_rank(attn_scores, fp_pool, sch.seg[:n_act], L, imp_part=part,
                                scale=scale, plan=plan, seg_keys=seg_keys)
            seg = sch.seg[:n_act].to(I64)
            n_of_row = torch.zeros(B, dtype=I64, device=dev).index_copy_(0, seg[:, 0] // L,
                                                                          seg[:, 1])
            inside = (col[None, :] < n_of_row[:, None]).reshape(-1)
            back = pages.logical_of_d[fp_pool]
            sch.full_pos.copy_(torch.where(inside, back, sch.full_pos))
        else:
            ops.importance_rank(attn_scores, sch.full_pos, sch.seg[:n_act], L, imp_part=part,
                                scale=scale, plan=plan, seg_keys=seg_keys)
        attn_scores.zero_()
        # ---- the next step's rows (generate.py:367-383, :439-467)
        sch.pack()
        seq_h, summ = sch.read(stats)
        stats.steps += 1
        stats.decoded = int(summ[_lib.SUM_DECODED])
        stats.verify_accepted = int(summ[_lib.SUM_VERIFY_ACCEPTED])
        stats.per_step_s.append(time.perf_counter() - t_step)
        stats.per_step_decoded.append(stats.decoded - sum(stats.per_step_decoded))
        if max_steps is not None and stats.steps >= max_steps:
            break
    torch.cuda.synchronize(dev)
    stats.wall_s = time.perf_counter() - t_start
    return responses, num_tokens, max_num_tokens
