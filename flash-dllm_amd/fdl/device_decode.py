"""Flash-Cache + Flash-Verify decoding with the bookkeeping on the device (fdl_sched_*).

The same decisions as fdl.generate.generate_with_Flash_dLLM (llada/generate.py:61-472) with
the fixed-stride cache layout, but the per-step state (token ids, the slot order full_pos,
the per-sequence counters) lives in device memory and is updated by the scheduler kernels,
so a denoising step is enqueued without waiting for the GPU and the host synchronises once
per step:

    pack (previous step) -> [sync: row counts, completions] -> pass-1 forward over the packed
    rows -> confidences -> pass-1 acceptance + verify lists -> verify forward -> draft-token
    probabilities -> verify acceptance -> importance ranking (in place on full_pos) -> pack

Completions and refills (generate.py:385-433) are handled on the host at the sync, with a
second synchronisation only on a step where a new prompt is admitted. The verify pass reads
the LM head on the last block_m / 2 rows of every verify block (its mask rows are the last S
of them), as the host scheduler does.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np
import torch

from . import lib as _lib
from . import ops
from .schedule import DEFAULT_PAGE_LOG2, AttnPlan, DeviceAttnPlan, contiguous_page_table

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


@torch.no_grad()
def generate_device_scheduled(model, prompts, prompt_lengths, batch_size, responses, n_steps,
                              gen_length, block_length, mask_id, threshold, gamma, track_num,
                              mask_num, eos_id, verify, stats, max_steps=None):
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
    from .generate import get_rotary_embedding
    sin, cos = get_rotary_embedding(L, d_model // n_heads, cfg.rope_theta, dev)
    rope = [sin.repeat(B, 1).contiguous(), cos.repeat(B, 1).contiguous()]
    for blk in model.model.transformer.blocks:
        blk.k_cache = torch.empty((B * L, d_model), dtype=model.dtype, device=dev)
        blk.v_cache = torch.empty((B * L, d_model), dtype=model.dtype, device=dev)
    attn_scores = torch.zeros(B * L, dtype=torch.float32, device=dev)
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
        f[_lib.SEQ_SEQLEN_K] = (pl + gen_length) // bn * bn + bn
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
            if admit(j):
                admitted = True
            else:
                idle(j)
        if admitted:
            sch.pack()
            seq_h, summ = sch.read(stats)
        act = [j for j in range(B) if active[j] != -1]
        if not act:
            break
        for j in act:
            n_steps[active[j]] += 1
        # ---- pass 1 over the packed rows
        Q, nmr = int(summ[_lib.SUM_Q]), int(summ[_lib.SUM_N_MASKED_ROWS])
        imp_rows = {j for j in act if seq_h[j, _lib.SEQ_N_MASKED] > 0}
        plan = sch.plan(summ, importance=bool(imp_rows))
        plan.defer_last_importance = True
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
            positions = [sch.vpos[:nv], sch.key_pos, rope, None, attn_scores, sch.vmeta[:n_act]]
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
