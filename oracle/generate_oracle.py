"""Literal CPU restatement of the Flash-dLLM decode loop (llada/generate.py:61-472).

TEST INFRASTRUCTURE ONLY: the oracle that the product scheduler
(flash-dllm_amd/fdl/generate.py) is checked against, step for step, on a tiny model. It
follows the reference's control flow and tensor bookkeeping one statement group at a time
(device tensors, per-sequence Python loops); the only decisions it fixes that the
reference leaves open are the two sort tie rules:
  * confidence sort (:230, :343): ties keep row order (NaN first, as torch sorts it);
  * importance sort (:365): ascending by score, ties put the higher slot first (so the
    highest-ranked tail prefers lower slots).
It calls `model(x_query, use_cache=True, lengths=..., positions=...)` exactly like the
reference and reads all logits rows. The tokenizer-dependent text handling (:385-402) is
replaced by storing the generated token ids. The RoPE tables are the correctly rounded
float32 tables of flash_cache_oracle.rope_tables (:44-50).

How it is pinned (tests/test_generate_kat.py): a scripted model sets every logit row's
float64 softmax maximum and every importance score, and the decisions are checked against
values worked out by hand from the reference's rules:
  pass-1 acceptance   max(#conf >= threshold, 1), the EOS length mask zeroing confidences
                      at or past the predicted length (a 0.95 there must lose)     (pinned)
  refresh order       ascending scores, ties to the higher slot                    (pinned)
  tracked set         track_num 1, 2, -1 and a mask_num 2 look-ahead window        (pinned)
  verify lists, mask  fill/draft/mask rows, key list and m11..m22 for (T, S) = (4, 2),
                      the candidate-free (8, 0) case                                (pinned)
  verify acceptance   cumprod prefix >= gamma (0.95, 0.92 -> 1 accepted, not 2)    (pinned)
  refill              the next prompt loaded into the finished row                  (pinned)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def _make_blocks(j, seqlen_k, start_m, end_m, block_m, device):
    """llada/generate.py:52-58."""
    q_starts = torch.arange(start_m, end_m, block_m, device=device)
    q_ends = q_starts + block_m
    q_ends[-1] = end_m
    batchs = torch.full_like(q_starts, j)
    k_ends = torch.full_like(q_starts, seqlen_k[j])
    return torch.stack((batchs, k_ends, q_starts, q_ends), dim=1)


def _rope(seq_len, dim, theta, device):
    """llada/generate.py:44-50, correctly rounded (flash_cache_oracle.rope_tables)."""
    from .flash_cache_oracle import rope_tables
    sin, cos = rope_tables(seq_len, dim, theta)
    return torch.from_numpy(sin).to(device), torch.from_numpy(cos).to(device)


def _stable_desc(v: torch.Tensor) -> torch.Tensor:
    """`v.sort(descending=True)` order (generate.py:230, :343): NaN first, as torch sorts it,
    then descending; ties in row order."""
    a = v.cpu().numpy().astype(np.float64)
    nan = np.isnan(a)
    return torch.from_numpy(np.lexsort((-np.where(nan, 0.0, a), ~nan))).to(v.device)


def _importance_asc(scores: torch.Tensor, slots: torch.Tensor) -> torch.Tensor:
    sc = scores.cpu().numpy().astype(np.float32)
    sl = slots.cpu().numpy()
    sc = np.where(sc == 0, np.float32(0), sc)
    return torch.from_numpy(np.lexsort((-sl, sc))).to(slots.device)


@torch.no_grad()
def generate_oracle(model, prompts, prompt_lengths, batch_size, n_steps, gen_length, block_length,
                    mask_id, threshold, gamma, track_num, mask_num, eos_id, verify):
    """Returns (responses dict: prompt index -> generated ids, num_tokens, max_num_tokens)."""
    dev = model.device
    block_m = block_length
    block_n = 128
    max_length = max(prompt_lengths) + gen_length + block_m
    max_length = (max_length // block_n + 1) * block_n
    d_model = model.config.d_model
    n_layers = model.config.n_layers
    n_heads = model.config.n_heads
    responses = {}
    num_tokens = 0
    max_num_tokens = 0
    empty_int32 = torch.tensor([], device=dev, dtype=torch.int32)
    count = 0
    x = torch.full((batch_size * max_length,), mask_id, dtype=torch.long, device=dev)
    x_draft = torch.full((batch_size * max_length,), mask_id, dtype=torch.long, device=dev)
    full_pos = torch.arange(batch_size * max_length, device=dev).reshape(batch_size, max_length)
    attn_scores = torch.zeros((batch_size * max_length,), dtype=torch.float32, device=dev)
    num_decoded, query_masked_pos, query_tracked_pos, query_verify_pos = [], [], [], []
    predicted_length, decoded_eos_pos, start_layer, active_batch, seqlen_keep, seqlen_k = [], [], [], [], [], []

    for j in range(batch_size):
        pl = prompt_lengths[count]
        x[j * max_length: j * max_length + pl] = prompts[count]
        x_draft[j * max_length: j * max_length + pl] = prompts[count]
        x[j * max_length + pl + gen_length: (j + 1) * max_length] = eos_id
        seqlen_k.append((pl + gen_length) // block_n * block_n + block_n)
        num_decoded.append(pl)
        query_masked_pos.append(full_pos[j, num_decoded[j]: num_decoded[j] + block_m])
        query_tracked_pos.append(torch.cat([full_pos[j, :num_decoded[j]],
                                            full_pos[j, num_decoded[j] + block_m: seqlen_k[j]]]))
        predicted_length.append(num_decoded[j] + gen_length + j * max_length)
        decoded_eos_pos.append(-1)
        start_layer.append(-1)
        active_batch.append(count)
        query_verify_pos.append(empty_int32)
        seqlen_keep.append(0)
        count += 1

    def pack():
        acc = 0
        mbl, tbl = [], []
        for j in range(batch_size):
            if query_masked_pos[j].shape[0] > 0:
                mbl.append(_make_blocks(j, seqlen_k, acc, acc + query_masked_pos[j].shape[0], block_m, dev))
                acc += query_masked_pos[j].shape[0]
        for j in range(batch_size):
            if query_tracked_pos[j].shape[0] > 0:
                tbl.append(_make_blocks(j, seqlen_k, acc, acc + query_tracked_pos[j].shape[0], block_m, dev))
                acc += query_tracked_pos[j].shape[0]
        mb = torch.cat(mbl, 0) if mbl else torch.zeros((0, 4), dtype=torch.long, device=dev)
        tb = torch.cat(tbl, 0) if tbl else torch.zeros((0, 4), dtype=torch.long, device=dev)
        qp = torch.cat(query_masked_pos + query_tracked_pos, dim=0).long()
        return mb, tb, qp

    query_masked_blocks, query_tracked_blocks, query_pos_flat = pack()
    x_query = x[query_pos_flat].unsqueeze(0)
    pos_sin, pos_cos = _rope(max_length, d_model // n_heads, model.config.rope_theta, dev)
    rotary_emb_pos = [pos_sin.repeat(batch_size, 1), pos_cos.repeat(batch_size, 1)]
    for blk in model.model.transformer.blocks:
        blk.k_cache = torch.empty((max_length * batch_size, d_model), dtype=model.dtype, device=dev)
        blk.v_cache = torch.empty((max_length * batch_size, d_model), dtype=model.dtype, device=dev)

    while True:
        query_blocks = torch.cat([query_masked_blocks, query_tracked_blocks], dim=0)
        positions = [query_pos_flat, empty_int32, rotary_emb_pos, [], attn_scores, []]
        lengths = [start_layer, None, query_masked_blocks, query_tracked_blocks, query_blocks, active_batch,
                   query_masked_blocks.shape[0], max_length, block_m, block_n, None, False]
        logits = model(x_query, use_cache=True, lengths=lengths, positions=positions).logits.squeeze(0)
        x_query = x_query.squeeze(0)
        acc_seqlen_masked = 0
        x_verify, key_pos_flat, attn_mask, query_verify_blocks = [], [], [], []
        acc_seqlen_q = acc_seqlen_k = 0
        keep = {}
        if verify:
            for j, i in enumerate(active_batch):
                if i == -1:
                    continue
                lm = logits[acc_seqlen_masked: acc_seqlen_masked + block_m]
                acc_seqlen_masked += query_masked_pos[j].shape[0]
                query_masked_pos[j] = query_masked_pos[j][:block_m]
                p = F.softmax(lm.to(torch.float64), dim=-1)
                x0_p, x0 = torch.max(p, dim=-1)
                if decoded_eos_pos[j] != -1:
                    lmask = query_masked_pos[j] >= predicted_length[j]
                    x0_p[lmask] = 0
                    length_num = query_masked_pos[j].shape[0] - int(lmask.sum())
                else:
                    length_num = query_masked_pos[j].shape[0]
                sidx = _stable_desc(x0_p)
                k = max(int((x0_p >= threshold).sum()), 1)
                x_draft[query_masked_pos[j]] = x0
                nd = num_decoded[j]
                full_pos[j, nd: nd + query_masked_pos[j].shape[0]] = query_masked_pos[j][sidx]
                pnew = full_pos[j, nd: nd + k]
                tnew = x0[sidx][:k]
                x[pnew] = tnew
                num_decoded[j] += k
                if decoded_eos_pos[j] == -1:
                    pe = pnew[tnew.eq(eos_id)]
                    if pe.shape[0] > 0:
                        decoded_eos_pos[j] = int(pe.max())
                        predicted_length[j] = decoded_eos_pos[j] + 1
                S = min(max(length_num - k, 0), block_m // 2)
                seqlen_keep[j] = block_m * 2 - S * 2
                T = seqlen_keep[j]
                m = torch.ones((block_m * 2, block_m * 2), device=dev, dtype=torch.bool)
                idx = torch.arange(S, device=dev)
                m11 = idx.view(-1, 1) >= idx.view(1, -1)
                m12 = idx.view(-1, 1) < idx.view(1, -1)
                m21 = idx.view(-1, 1) > idx.view(1, -1)
                m22 = idx.view(-1, 1) <= idx.view(1, -1)
                m[:T, T:T + S] = False
                m[T:T + S + S, T:T + S + S] = torch.cat([torch.cat([m11, m12], 1), torch.cat([m21, m22], 1)], 0)
                attn_mask.append(m)
                nd = num_decoded[j]
                cand = full_pos[j, nd: nd + S]
                fill = full_pos[j, nd - T: nd]
                x_verify.append(torch.cat([x[fill], x_draft[cand], x[cand]], 0))
                query_verify_pos[j] = torch.cat([fill, cand, cand], 0)
                key_pos_flat.append(torch.cat([full_pos[j, :nd - T], full_pos[j, nd + S: seqlen_k[j]]], 0))
                query_verify_blocks.append((acc_seqlen_k, acc_seqlen_k + key_pos_flat[-1].shape[0],
                                            acc_seqlen_q, acc_seqlen_q + query_verify_pos[j].shape[0]))
                acc_seqlen_q += query_verify_pos[j].shape[0]
                acc_seqlen_k += key_pos_flat[-1].shape[0]
            query_verify_blocks = torch.tensor(query_verify_blocks, device=dev, dtype=torch.int32)
            attn_mask = torch.cat(attn_mask, 0)
            query_pos_flat = torch.cat([query_verify_pos[j] for j in range(batch_size) if active_batch[j] != -1], 0)
            key_pos_flat = torch.cat(key_pos_flat, 0)
            x_query = torch.cat(x_verify, 0).unsqueeze(0)
            positions = [query_pos_flat, key_pos_flat, rotary_emb_pos, [], attn_scores, attn_mask]
            lengths = [start_layer, query_verify_blocks, None, query_tracked_blocks, None, active_batch,
                       0, max_length, block_m, block_n, None, True]
            logits = model(x_query, use_cache=True, lengths=lengths, positions=positions).logits.squeeze(0)
            x_query = x_query.squeeze(0)

        acc_v = 0
        for j, i in enumerate(active_batch):
            if i == -1:
                continue
            n_steps[i] += 1
            if verify:
                T = seqlen_keep[j]
                S = (block_m * 2 - T) // 2
                k = 0
                if S > 0:
                    lv = logits[acc_v + T + S: acc_v + T + 2 * S]
                    xv = x_query[acc_v + T: acc_v + T + S]
                    pv = F.softmax(lv.to(torch.float64), dim=-1).gather(1, xv.unsqueeze(1)).view(-1)
                    if decoded_eos_pos[j] != -1:
                        pv[query_pos_flat[acc_v + T: acc_v + T + S] >= predicted_length[j]] = 0
                    pv = pv.cumprod(dim=0)
                    k = int((pv >= gamma).sum())
                    pnew = full_pos[j, num_decoded[j]: num_decoded[j] + k]
                    tnew = xv[:k]
                acc_v += query_verify_pos[j].shape[0]
            else:
                lm = logits[acc_seqlen_masked: acc_seqlen_masked + query_masked_pos[j].shape[0]]
                acc_seqlen_masked += query_masked_pos[j].shape[0]
                p = F.softmax(lm.to(torch.float64), dim=-1)
                x0_p, x0 = torch.max(p, dim=-1)
                if decoded_eos_pos[j] != -1:
                    x0_p[query_masked_pos[j] >= predicted_length[j]] = 0
                sidx = _stable_desc(x0_p)
                k = max(int((x0_p[sidx] >= threshold).sum()), 1)
                nd = num_decoded[j]
                full_pos[j, nd: nd + query_masked_pos[j].shape[0]] = query_masked_pos[j][sidx]
                pnew = full_pos[j, nd: nd + k]
                tnew = x0[sidx][:k]
            keep[j] = k
            if k > 0:
                x[pnew] = tnew
                num_decoded[j] += k
                if decoded_eos_pos[j] == -1:
                    pe = pnew[tnew.eq(eos_id)]
                    if pe.shape[0] > 0:
                        decoded_eos_pos[j] = int(pe.max())
                        predicted_length[j] = decoded_eos_pos[j] + 1
            nd = num_decoded[j]
            if (full_pos[j, nd:] < predicted_length[j]).any():
                seg = full_pos[j, :nd - k]
                full_pos[j, :nd - k] = seg[_importance_asc(attn_scores[seg], seg)]
                query_masked_pos[j] = full_pos[j, nd: nd + block_m]
                if track_num < 0:
                    query_tracked_pos[j] = torch.cat([full_pos[j, :nd], full_pos[j, nd + block_m: seqlen_k[j]]])
                else:
                    t0 = max(0, nd - track_num * block_m)
                    t1 = min(seqlen_k[j], nd + block_m * mask_num)
                    query_tracked_pos[j] = torch.cat([full_pos[j, t0:nd], full_pos[j, nd + block_m: t1]])
                start_layer[j] = n_layers
            else:
                pl = prompt_lengths[i]
                responses[i] = x[j * max_length + pl: j * max_length + nd].tolist()
                num_tokens += nd - pl
                max_num_tokens += gen_length
                if count < len(prompts):
                    active_batch[j] = count
                    pl = prompt_lengths[count]
                    x[j * max_length: (j + 1) * max_length] = mask_id
                    x[j * max_length: j * max_length + pl] = prompts[count]
                    x[j * max_length + pl + gen_length: (j + 1) * max_length] = eos_id
                    seqlen_k[j] = (pl + gen_length) // block_n * block_n + block_n
                    x_draft[j * max_length: (j + 1) * max_length] = mask_id
                    x_draft[j * max_length: j * max_length + pl] = prompts[count]
                    num_decoded[j] = pl
                    full_pos[j] = torch.arange(j * max_length, (j + 1) * max_length, device=dev)
                    query_verify_pos[j] = empty_int32
                    query_masked_pos[j] = full_pos[j, pl: pl + block_m]
                    query_tracked_pos[j] = torch.cat([full_pos[j, :pl], full_pos[j, pl + block_m: seqlen_k[j]]])
                    predicted_length[j] = pl + gen_length + j * max_length
                    start_layer[j] = -1
                    decoded_eos_pos[j] = -1
                    count += 1
                else:
                    active_batch[j] = -1
                    query_masked_pos[j] = empty_int32
                    query_tracked_pos[j] = empty_int32
                    query_verify_pos[j] = empty_int32
        if sum(active_batch) == -batch_size:
            break
        query_masked_blocks, query_tracked_blocks, query_pos_flat = pack()
        x_query = x[query_pos_flat].unsqueeze(0)
        attn_scores.fill_(0)
    return responses, num_tokens, max_num_tokens
