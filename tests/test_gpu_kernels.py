"""Parity of the HIP kernels (through the C ABI) with the numpy oracle on seeded inputs.

Bars: cache-slot writes and top-k / ranking bit-exact; bf16 Q/K/V/attention outputs within
atol 2e-2 / rtol 1e-2 of the float32 oracle; importance scores within 1e-3."""
import numpy as np
import pytest
import torch

from oracle import flash_cache_oracle as orc
from fdl import lib, ops
from fdl.schedule import SeqRows, contiguous_page_table, make_plan, seqs_from_reference_blocks

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ATOL, RTOL = 2e-2, 1e-2
POISON = 1232.0  # exactly representable in bf16 (1.0011010b x 2^10)


def _bf16(shape, gen, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)


def _np(t):
    return t.float().cpu().numpy()


def _rope(L, theta=500000.0, hd=128, repeat=1):
    sin, cos = orc.rope_tables(L, hd, theta)
    return (torch.from_numpy(np.tile(sin, (repeat, 1))).to(DEV),
            torch.from_numpy(np.tile(cos, (repeat, 1))).to(DEV))


def _close(got, exp, atol=ATOL, rtol=RTOL, what=""):
    np.testing.assert_allclose(got, exp, atol=atol, rtol=rtol, err_msg=what)


# ------------------------------------------------------------------- fused projection

def _qkv_case(seed, n_heads, Q, n_slots, slots, kv_packed=False, theta=500000.0, L=None):
    gen = torch.Generator().manual_seed(seed)
    D = n_heads * 128
    x = _bf16((Q, D), gen)
    wq, wk, wv = (_bf16((D, D), gen, 0.02) for _ in range(3))
    L = L or n_slots
    sin, cos = _rope(L, theta, repeat=max(1, n_slots // L))
    slot = torch.as_tensor(slots, dtype=torch.int64)
    q_out = torch.zeros((Q, D), dtype=torch.bfloat16, device=DEV)
    rows_kv = Q if kv_packed else n_slots
    kc = torch.full((rows_kv, D), POISON, dtype=torch.bfloat16, device=DEV)
    vc = torch.full((rows_kv, D), POISON, dtype=torch.bfloat16, device=DEV)
    xd, wqd, wkd, wvd = (t.to(DEV) for t in (x, wq, wk, wv))
    ops.qkv_rope_cache(xd, wqd, wkd, wvd, sin, cos, slot.to(DEV), q_out, kc, vc, n_heads,
                       kv_packed=kv_packed)
    torch.cuda.synchronize()
    s_np, c_np = sin.cpu().numpy(), cos.cpu().numpy()
    if kv_packed:
        q_ref, k_ref, v_ref = orc.qkv_proj_cache(_np(x), _np(wq), _np(wk), _np(wv), s_np, c_np,
                                                 slot.numpy(), n_heads, None, None)
    else:
        q_ref, k_ref, v_ref = orc.qkv_proj_cache(
            _np(x), _np(wq), _np(wk), _np(wv), s_np, c_np, slot.numpy(), n_heads,
            np.full((n_slots, D), POISON, np.float32), np.full((n_slots, D), POISON, np.float32))
    return q_out, kc, vc, q_ref, k_ref, v_ref, slot.numpy()


def test_qkv_rope_cache_40_rows_one_sequence():
    """40 query rows (32-token masked block + 8 tracked slots), d_model 4096, 32 heads,
    theta 5e5, cache of 512 slots: Q/K/V within tolerance, untouched slots bit-exact."""
    rng = np.random.default_rng(1)
    slots = np.concatenate([np.arange(192, 224), rng.choice(192, 8, replace=False)])
    q, kc, vc, q_ref, k_ref, v_ref, s = _qkv_case(1, 32, 40, 512, slots)
    _close(_np(q), q_ref, what="Q")
    _close(_np(kc)[s], k_ref[s], what="K rows")
    _close(_np(vc)[s], v_ref[s], what="V rows")
    untouched = np.setdiff1d(np.arange(512), s)
    assert np.all(_np(kc)[untouched] == POISON) and np.all(_np(vc)[untouched] == POISON)


def test_qkv_rope_cache_512_rows_batch8():
    """512 rows over 8 sequences of a 896-slot stride (32 masked + 32 tracked each)."""
    rng = np.random.default_rng(2)
    B, L = 8, 896
    slots = []
    for b in range(B):
        f = 256 + 32 * int(rng.integers(0, 16))
        slots.append(b * L + np.arange(f, f + 32))
    for b in range(B):
        f = int(slots[b][0] - b * L)
        slots.append(b * L + rng.choice(f, 32, replace=False))
    slots = np.concatenate(slots)
    q, kc, vc, q_ref, k_ref, v_ref, s = _qkv_case(2, 32, 512, B * L, slots, L=L)
    _close(_np(q), q_ref, what="Q")
    _close(_np(kc)[s], k_ref[s], what="K rows")
    _close(_np(vc)[s], v_ref[s], what="V rows")
    untouched = np.setdiff1d(np.arange(B * L), s)
    assert np.all(_np(kc)[untouched] == POISON) and np.all(_np(vc)[untouched] == POISON)


@pytest.mark.parametrize("Q", [1, 17, 129, 300, 700, 1100])
def test_qkv_rope_cache_ragged_rows_small_model(Q):
    """Ragged row counts on a 4-head model; together they cover every tile plan of the
    kernel (up to 64, 384 and 1024 rows, and above), including tiles whose pair block
    straddles two of the three matrices."""
    rng = np.random.default_rng(Q)
    n_slots = max(1024, 2 * Q)
    slots = rng.choice(n_slots, Q, replace=False)
    q, kc, vc, q_ref, k_ref, v_ref, s = _qkv_case(10 + Q, 4, Q, n_slots, slots, theta=10000.0)
    _close(_np(q), q_ref, what="Q")
    _close(_np(kc)[s], k_ref[s], what="K rows")
    _close(_np(vc)[s], v_ref[s], what="V rows")
    untouched = np.setdiff1d(np.arange(n_slots), s)
    assert np.all(_np(kc)[untouched] == POISON)


@pytest.mark.parametrize("kv_packed", [False, True])
def test_qkv_rope_cache_streamed_tail(kv_packed):
    """576 rows at d_model 4096: four 128-row tiles fill one round of workgroups and the
    last 64 rows go to the weight-streaming kernel in a second launch; both launches must
    land their rows (Q, K/V rows or packed K/V) within tolerance."""
    rng = np.random.default_rng(5)
    Q, n_slots = 576, 2048
    slots = rng.choice(n_slots, Q, replace=False)
    q, kc, vc, q_ref, k_ref, v_ref, s = _qkv_case(5, 32, Q, n_slots, slots, kv_packed=kv_packed)
    _close(_np(q), q_ref, what="Q")
    if kv_packed:
        _close(_np(kc), k_ref, what="K packed")
        _close(_np(vc), v_ref, what="V packed")
    else:
        _close(_np(kc)[s], k_ref[s], what="K rows")
        _close(_np(vc)[s], v_ref[s], what="V rows")
        untouched = np.setdiff1d(np.arange(n_slots), s)
        assert np.all(_np(kc)[untouched] == POISON) and np.all(_np(vc)[untouched] == POISON)


@pytest.mark.parametrize("Q", [64, 600])
def test_qkv_packed_verify_mode(Q):
    rng = np.random.default_rng(3)
    slots = rng.integers(0, 256, Q)  # repeated slots are legal when nothing is scattered
    q, k, v, q_ref, k_ref, v_ref, _ = _qkv_case(3, 4, Q, 256, slots, kv_packed=True)
    _close(_np(q), q_ref, what="Q")
    _close(_np(k), k_ref, what="K packed")
    _close(_np(v), v_ref, what="V packed")


# ------------------------------------------------------------------ block attention

def _ref_tables(B, L, k_ends, masked_n, tracked):
    """Reference-format packed schedule: masked rows of every sequence, then tracked rows
    (llada/generate.py:146-167). Returns (slots, masked_blocks, tracked_blocks)."""
    slots, masked, tracked_b = [], [], []
    acc = 0
    for b in range(B):
        f = masked_n[b][0]
        s = b * L + np.arange(f, f + masked_n[b][1])
        masked.append(orc.make_blocks(b, k_ends, acc, acc + len(s), 32))
        slots.append(s)
        acc += len(s)
    for b in range(B):
        s = b * L + np.asarray(tracked[b], dtype=np.int64)
        if len(s):
            tracked_b.append(orc.make_blocks(b, k_ends, acc, acc + len(s), 32))
            slots.append(s)
            acc += len(s)
    return (np.concatenate(slots), np.concatenate(masked),
            np.concatenate(tracked_b) if tracked_b else np.zeros((0, 4), np.int64))


def _attn_inputs(seed, Q, n_slots, n_heads):
    gen = torch.Generator().manual_seed(seed)
    D = n_heads * 128
    return _bf16((Q, D), gen), _bf16((n_slots, D), gen), _bf16((n_slots, D), gen)


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM])
def test_block_attention_batch8_cache768(imp_mode):
    """8 sequences, k_end 768 of a 896 stride, 32 masked + 32 tracked rows each, 32 heads;
    masked and tracked rows share one tile per sequence."""
    rng = np.random.default_rng(4)
    B, L, H = 8, 896, 32
    k_ends = [768] * B
    masked_n, tracked = [], []
    for b in range(B):
        f = 256 + 32 * int(rng.integers(0, 16))
        masked_n.append((f, 32))
        tracked.append(rng.choice(f, 32, replace=False))
    slots, mb, tb = _ref_tables(B, L, k_ends, masked_n, tracked)
    Q = len(slots)
    q, kc, vc = _attn_inputs(5, Q, B * L, H)
    plan = make_plan(seqs_from_reference_blocks(mb, tb, importance=imp_mode != lib.IMP_NONE),
                     contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    assert plan.n_work == B  # one tile per sequence
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV)
    scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    qd, kd, vd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    ops.block_attention(qd, kd, vd, plan, out, H, scale, imp_mode, imp if imp_mode else None)
    if imp_mode:
        ops.importance_accumulate(imp, plan, 1.0 / (32 * H) if imp_mode == lib.IMP_RAW_LOGIT else 1.0, scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    ref = orc.block_attention(qn, kn, vn, np.concatenate([mb, tb]), L, H, scale)
    _close(_np(out), ref, what="attention out")
    if imp_mode == lib.IMP_RAW_LOGIT:
        S = orc.importance_raw_S(qn, kn, mb, B, L, H, 32)
        exp = orc.importance_accumulate(np.zeros(B * L, np.float32), S)
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="raw importance")
    elif imp_mode == lib.IMP_SOFTMAX_COLSUM:
        exp = orc.importance_softmax_colsum(qn, kn, mb, B, L, H, scale)
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="softmax importance")


def test_block_attention_paged_stress():
    """Block-table stress: 6 sequences, k_end in [512, 1536], query lengths in [1, 96] or a
    full recompute (q = k), 32-slot pages randomly permuted over a global pool."""
    rng = np.random.default_rng(6)
    B, H, P = 6, 4, 32
    k_ends = [int(rng.integers(512, 1537)) for _ in range(B)]
    k_ends[1] = 1536
    max_pages = 1536 // P
    n_pages = sum((k + P - 1) // P for k in k_ends) + 7
    perm = rng.permutation(n_pages)
    table = np.zeros((B, max_pages), np.int32)
    nxt = 0
    for b in range(B):
        for p in range((k_ends[b] + P - 1) // P):
            table[b, p] = perm[nxt]
            nxt += 1
    seqs, row = [], 0
    for b in range(B):
        qn = k_ends[b] if b in (1, 4) else int(rng.integers(1, 97))
        rows = np.arange(row, row + qn)
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=rows, n_imp=min(qn, 32)))
        row += qn
    Q = row
    q, kc, vc = _attn_inputs(7, Q, n_pages * P, H)
    plan = make_plan(seqs, table, 5, device=DEV)
    plan.validate(Q, n_pages * P)
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, n_pages * P), dtype=torch.float32, device=DEV)
    scores = torch.zeros(n_pages * P, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, lib.IMP_RAW_LOGIT, imp)
    ops.importance_accumulate(imp, plan, 1.0, scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    got = _np(out)
    sc = scores.cpu().numpy()
    for sq in seqs:
        blk = np.array([[sq.batch, sq.k_end, sq.rows[0], sq.rows[-1] + 1]])
        ref = orc.block_attention(qn, kn, vn, blk, 0, H, scale, page_table=table, page_size=P)
        _close(got[sq.rows], ref[sq.rows], what=f"seq {sq.batch}")
        keys = orc.key_slots(sq.batch, sq.k_end, 0, table, P)
        exp = np.zeros(len(keys))
        for h in range(H):
            cols = slice(h * 128, (h + 1) * 128)
            exp += (qn[sq.rows[:sq.n_imp]][:, cols] @ kn[keys][:, cols].T).sum(0)
        _close(sc[keys], exp, atol=2e-3, rtol=1e-4, what=f"importance seq {sq.batch}")


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM])
def test_block_attention_full_recompute_tiles(imp_mode):
    """Full recomputes (q = k: 256-row tiles, with 188- and 1-row remainders) next to a
    100-row (128-row class) and a 40-row (64-row class) sequence, ragged k_end, 32
    importance rows per sequence."""
    B, L, H = 5, 1024, 4
    k_ends = [1024, 700, 513, 300, 200]
    n_q = [1024, 700, 513, 100, 40]
    seqs, blocks, mb, q0 = [], [], [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q[b]),
                            n_imp=32 if imp_mode else 0))
        blocks.append((b, k_ends[b], q0, q0 + n_q[b]))
        mb.append((b, k_ends[b], q0, q0 + 32))
        q0 += n_q[b]
    Q = q0
    q, kc, vc = _attn_inputs(11, Q, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    assert plan.n_long == 10 and plan.n_mid == 1 and plan.n_work == 12
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV)
    scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode,
                        imp if imp_mode else None)
    if imp_mode:
        ops.importance_accumulate(imp, plan, 1.0 / (32 * H) if imp_mode == lib.IMP_RAW_LOGIT else 1.0,
                                  scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    ref = orc.block_attention(qn, kn, vn, np.array(blocks), L, H, scale)
    _close(_np(out), ref, what="attention out")
    mb = np.array(mb)
    if imp_mode == lib.IMP_RAW_LOGIT:
        S = orc.importance_raw_S(qn, kn, mb, B, L, H, 32)
        exp = orc.importance_accumulate(np.zeros(B * L, np.float32), S)
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="raw importance")
    elif imp_mode == lib.IMP_SOFTMAX_COLSUM:
        exp = orc.importance_softmax_colsum(qn, kn, mb, B, L, H, scale)
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="softmax importance")


def test_block_attention_softmax_importance_store_and_two_pass():
    """64-row tiles with softmax-colsum importance on all three of the kernel's paths: the
    probabilities kept on chip (at most 32 importance rows and 24 key blocks: 32 rows over
    1000 keys, 17 rows over 768 keys, 32 rows over one block), in the workspace (25 blocks)
    and the second pass over K (48 rows)."""
    B, L, H = 5, 1664, 4
    k_ends = [1000, 500, 768, 64, 1600]
    n_q = [50, 60, 40, 64, 40]
    n_imp = [32, 48, 17, 32, 32]
    seqs, blocks, mb, q0 = [], [], [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q[b]),
                            n_imp=n_imp[b]))
        blocks.append((b, k_ends[b], q0, q0 + n_q[b]))
        mb.append((b, k_ends[b], q0, q0 + n_imp[b]))
        q0 += n_q[b]
    Q = q0
    q, kc, vc = _attn_inputs(12, Q, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    assert plan.n_long == 0 and plan.n_mid == 0 and plan.n_work == B
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV)
    scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale,
                        lib.IMP_SOFTMAX_COLSUM, imp)
    ops.importance_accumulate(imp, plan, 1.0, scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    _close(_np(out), orc.block_attention(qn, kn, vn, np.array(blocks), L, H, scale),
           what="attention out")
    exp = orc.importance_softmax_colsum(qn, kn, np.array(mb), B, L, H, scale)
    _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="softmax importance")


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM])
def test_block_attention_short_key_ranges(imp_mode):
    """Key ranges at the edges of the LDS ring (three 64-key stages, two of them requested
    before the first block is handed over): 1 to 191 keys, in 64-row tiles (with 32
    importance rows: probabilities kept on chip; with 48: the second pass over K, whose
    blocks may all still be resident) and in 128-row tiles, against the oracle."""
    B, L, H = 8, 256, 4
    k_ends = [1, 40, 64, 65, 127, 129, 191, 192]
    n_q = [3, 40, 64, 60, 100, 120, 64, 90]
    n_imp = [1, 32, 48, 32, 48, 32, 48, 32]
    seqs, blocks, mb, q0 = [], [], [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q[b]),
                            n_imp=n_imp[b] if imp_mode else 0))
        blocks.append((b, k_ends[b], q0, q0 + n_q[b]))
        mb.append((b, k_ends[b], q0, q0 + n_imp[b]))
        q0 += n_q[b]
    Q = q0
    q, kc, vc = _attn_inputs(21, Q, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    assert plan.n_long == 0 and plan.n_mid == 3
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV) if imp_mode else None
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode, imp)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    _close(_np(out), orc.block_attention(qn, kn, vn, np.array(blocks), L, H, scale),
           what="attention out")
    if imp_mode:
        bm = max(n_imp)  # the raw mode's mean over block_m rows and heads
        scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
        ops.importance_accumulate(imp, plan, 1.0 / (bm * H) if imp_mode == lib.IMP_RAW_LOGIT
                                  else 1.0, scores)
        torch.cuda.synchronize()
        if imp_mode == lib.IMP_RAW_LOGIT:
            exp = orc.importance_accumulate(np.zeros(B * L, np.float32),
                                            orc.importance_raw_S(qn, kn, np.array(mb), B, L, H, bm))
        else:
            exp = orc.importance_softmax_colsum(qn, kn, np.array(mb), B, L, H, scale)
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="importance")


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT])
def test_block_attention_long_tiles_few_key_blocks(imp_mode):
    """256-row tiles over one to three key blocks (the two-group kernel requests two blocks
    before the first hand-over and the third after it): 200 rows over 40, 64, 100, 128 and
    170 keys, against the oracle."""
    B, L, H = 5, 256, 2
    k_ends = [40, 64, 100, 128, 170]
    n_q = 200
    seqs, blocks, mb, q0 = [], [], [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q),
                            n_imp=32 if imp_mode else 0))
        blocks.append((b, k_ends[b], q0, q0 + n_q))
        mb.append((b, k_ends[b], q0, q0 + 32))
        q0 += n_q
    Q = q0
    q, kc, vc = _attn_inputs(22, Q, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    assert plan.n_long == B
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV) if imp_mode else None
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode, imp)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    _close(_np(out), orc.block_attention(qn, kn, vn, np.array(blocks), L, H, scale),
           what="attention out")
    if imp_mode:
        scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
        ops.importance_accumulate(imp, plan, 1.0 / (32 * H), scores)
        torch.cuda.synchronize()
        exp = orc.importance_accumulate(np.zeros(B * L, np.float32),
                                        orc.importance_raw_S(qn, kn, np.array(mb), B, L, H, 32))
        _close(scores.cpu().numpy(), exp, atol=1e-3, rtol=1e-3, what="raw importance")


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT])
def test_block_attention_key_ranges_beyond_the_staged_slot_map(imp_mode):
    """Key ranges longer than the 2048 keys whose slots a workgroup stages in LDS (slots then
    come straight from the page table, raw importance is stored directly): a 2500-key
    sequence with 40 rows (64-row tile), one with 100 rows (128-row tile), and a 300-row
    recompute over 3000 keys (256-row tiles), permuted 32-slot pages."""
    rng = np.random.default_rng(13)
    B, H, P = 3, 4, 32
    k_ends = [2500, 2200, 3000]
    n_q = [40, 100, 300]
    max_pages = 3000 // P + 1
    n_pages = sum((k + P - 1) // P for k in k_ends) + 5
    perm = rng.permutation(n_pages)
    table = np.zeros((B, max_pages), np.int32)
    nxt = 0
    for b in range(B):
        n = (k_ends[b] + P - 1) // P
        table[b, :n] = perm[nxt:nxt + n]
        nxt += n
    seqs, q0 = [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q[b]),
                            n_imp=32 if imp_mode else 0))
        q0 += n_q[b]
    Q = q0
    q, kc, vc = _attn_inputs(14, Q, n_pages * P, H)
    plan = make_plan(seqs, table, 5, device=DEV)
    plan.validate(Q, n_pages * P)
    assert plan.n_long == 2 and plan.n_mid == 1 and plan.n_work == 4
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, n_pages * P), dtype=torch.float32, device=DEV)
    scores = torch.zeros(n_pages * P, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode,
                        imp if imp_mode else None)
    if imp_mode:
        ops.importance_accumulate(imp, plan, 1.0, scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    got = _np(out)
    sc = scores.cpu().numpy()
    for sq in seqs:
        keys = orc.key_slots(sq.batch, sq.k_end, 0, table, P)
        ref = orc.attend(qn[sq.rows], kn[keys], vn[keys], H, scale)
        _close(got[sq.rows], ref, what=f"seq {sq.batch} ({sq.k_end} keys, {len(sq.rows)} rows)")
        if imp_mode:
            exp = kn[keys] @ qn[sq.rows[:sq.n_imp]].astype(np.float64).sum(0)
            _close(sc[keys], exp, atol=2e-3, rtol=1e-4, what=f"importance seq {sq.batch}")


def test_verify_attention_key_list_beyond_the_staged_slot_map():
    """Verify blocks whose cache-key lists exceed 2048 entries (3000-slot caches)."""
    H, bm, n_blk, L = 4, 32, 3, 3000
    key_pos, vblocks, mask, _ = _verify_case(15, n_blk, L, H, bm)
    assert np.all(vblocks[:, 1] - vblocks[:, 0] > 2048)
    rows = 2 * bm
    gen = torch.Generator().manual_seed(16)
    D = H * 128
    q, k1, v1 = (_bf16((n_blk * rows, D), gen) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen) for _ in range(2))
    out = torch.full((n_blk * rows, D), POISON, dtype=torch.bfloat16, device=DEV)
    scale = orc.softmax_scale(128)
    ops.verify_attention(q.to(DEV), k1.to(DEV), v1.to(DEV), kc.to(DEV), vc.to(DEV),
                         torch.from_numpy(key_pos).to(DEV), torch.from_numpy(vblocks).to(DEV),
                         torch.from_numpy(mask).to(DEV), rows, out, H, scale)
    torch.cuda.synchronize()
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, rows, H, scale)
    _close(_np(out), ref, what="verify attention, long key lists")


@pytest.mark.parametrize("imp_mode", [lib.IMP_NONE, lib.IMP_RAW_LOGIT])
@pytest.mark.parametrize("case", ["one_sequence_384", "ragged_3"])
def test_block_attention_key_split_matches_one_workgroup(imp_mode, case):
    """A launch that fills at most half of the device splits every tile's key blocks over
    several workgroups and merges their rows: one sequence of 40 rows over 384 keys with 32
    heads (eight parts for six blocks, two of them empty), and three sequences over 1000,
    130 and 64 keys with 8 heads (eight parts: two blocks each, mostly empty parts). The
    output agrees with the unsplit launch within bf16 rounding and with the oracle; the raw
    importance is bit-identical (each key's sum is formed by one workgroup either way)."""
    if case == "one_sequence_384":
        H, L, k_ends, n_q, n_imp = 32, 384, [384], [40], [32]
    else:
        H, L, k_ends, n_q, n_imp = 8, 1024, [1000, 130, 64], [50, 33, 64], [32, 17, 32]
    B = len(k_ends)
    seqs, blocks, q0 = [], [], 0
    for b in range(B):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(q0, q0 + n_q[b]),
                            n_imp=n_imp[b] if imp_mode else 0))
        blocks.append((b, k_ends[b], q0, q0 + n_q[b]))
        q0 += n_q[b]
    Q = q0
    q, kc, vc = _attn_inputs(31, Q, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    plan.validate(Q, B * L)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert ops.attention_split_floats(plan, H, cus) > 0  # the launch does split
    scale = orc.softmax_scale(128)
    outs, imps = [], []
    for split in (True, False):
        out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
        imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV)
        ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode,
                            imp if imp_mode else None, key_split=split)
        torch.cuda.synchronize()
        outs.append(_np(out))
        imps.append(imp.cpu())
    np.testing.assert_allclose(outs[0], outs[1], atol=1e-2, rtol=1e-2, err_msg="split vs unsplit")
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    _close(outs[0], orc.block_attention(qn, kn, vn, np.array(blocks), L, H, scale),
           what="split attention out")
    if imp_mode:
        assert torch.equal(imps[0], imps[1])


def test_block_attention_leaves_other_rows_untouched():
    B, L, H = 2, 128, 2
    seqs = [SeqRows(0, 100, np.array([5, 1, 9])), SeqRows(1, 128, np.array([0, 7]))]
    q, kc, vc = _attn_inputs(8, 12, B * L, H)
    plan = make_plan(seqs, contiguous_page_table(B, L), device=DEV)
    out = torch.full((12, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, 0.088)
    torch.cuda.synchronize()
    got = _np(out)
    written = [5, 1, 9, 0, 7]
    assert np.all(got[np.setdiff1d(np.arange(12), written)] == POISON)
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    _close(got[[5, 1, 9]], orc.attend(qn[[5, 1, 9]], kn[:100], vn[:100], H, 0.088))
    _close(got[[0, 7]], orc.attend(qn[[0, 7]], kn[L:2 * L], vn[L:2 * L], H, 0.088))


# ------------------------------------------------------------------------- ranking

@pytest.mark.parametrize("L", [50, 120, 200, 500, 896, 2000, 4000])
def test_importance_rank_bit_exact(L):
    """Every sort-network size (64 .. 4096 keys; one key per thread up to 1024), ragged
    segments incl. 0 and 1 entries, many ties and signed zeros."""
    rng = np.random.default_rng(9)
    B = 8
    scores = (rng.integers(-40, 40, B * L).astype(np.float32) * np.float32(0.25))
    scores[rng.choice(B * L, 50)] = -0.0
    full_pos = np.arange(B * L, dtype=np.int64).reshape(B, L)
    for b in range(B):
        full_pos[b] = full_pos[b][rng.permutation(L)]
    lens = [int(rng.integers(0, L)) for _ in range(B)]
    lens[0], lens[1], lens[2] = 0, 1, L - 1  # L - 1 selects the network size
    seg = np.array([[b * L, lens[b]] for b in range(B)], np.int32)
    k = 32
    slots_d = torch.from_numpy(full_pos.copy()).to(DEV)
    topk_d = torch.zeros((B, k), dtype=torch.int64, device=DEV)
    ops.importance_rank(torch.from_numpy(scores).to(DEV), slots_d, torch.from_numpy(seg).to(DEV),
                        max(lens), topk_d, k)
    torch.cuda.synchronize()
    got = slots_d.cpu().numpy()
    for b in range(B):
        seg_slots = full_pos[b, :lens[b]]
        np.testing.assert_array_equal(got[b, :lens[b]], orc.rank_ascending(scores, seg_slots))
        np.testing.assert_array_equal(got[b, lens[b]:], full_pos[b, lens[b]:])
        np.testing.assert_array_equal(topk_d[b].cpu().numpy(), orc.topk(scores, seg_slots, k))


def test_importance_rank_max_segment():
    rng = np.random.default_rng(10)
    n = 8192
    scores = rng.standard_normal(n).astype(np.float32)
    slots = rng.permutation(n).astype(np.int64)
    slots_d = torch.from_numpy(slots.copy()).to(DEV)
    topk_d = torch.zeros((1, 64), dtype=torch.int64, device=DEV)
    ops.importance_rank(torch.from_numpy(scores).to(DEV), slots_d,
                        torch.tensor([[0, n]], dtype=torch.int32, device=DEV), n, topk_d, 64)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(slots_d.cpu().numpy(), orc.rank_ascending(scores, slots))
    np.testing.assert_array_equal(topk_d[0].cpu().numpy(), orc.topk(scores, slots, 64))


@pytest.mark.parametrize("L,H", [(704, 32), (3008, 20)])
def test_importance_accumulate_rank_matches_separate_kernels(L, H):
    """fdl_importance_accumulate_rank = fdl_importance_accumulate over each segment's
    sequence keys followed by fdl_importance_rank, bit for bit (every score, order, top-k):
    one key per thread (704) and four (3008), 32 heads and 20 (a partial batch of head
    loads), permuted pages, segments longer and shorter than the key count (entries past
    the keys keep their score), a sequence with no segment (its keys untouched)."""
    from fdl.schedule import SeqRows, make_plan
    rng = np.random.default_rng(12)
    B, k, P = 6, 32, 32
    n_pages = B * L // P
    table = rng.permutation(n_pages).astype(np.int32).reshape(B, L // P)
    n = n_pages * P
    part = torch.from_numpy(rng.standard_normal((H, n)).astype(np.float32)).to(DEV)
    base = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(DEV)
    k_end = [int(v) for v in rng.integers(1, L + 1, B)]
    lens = [int(v) for v in rng.integers(1, L + 1, B)]
    k_end[0], lens[0] = L, L
    k_end[1], lens[1] = L // 2, L  # ranked entries past the keys
    ranked_rows = [0, 1, 2, 3, 5]  # row 4 has no segment
    slots_of = [((table[b].astype(np.int64)[np.arange(L) // P] * P) + np.arange(L) % P)
                for b in range(B)]
    full_pos = np.full((B, L), -7, dtype=np.int64)
    for b in range(B):
        full_pos[b] = slots_of[b][rng.permutation(L)]
        full_pos[b, :lens[b]] = slots_of[b][rng.permutation(lens[b])]
    seg = torch.from_numpy(np.array([[b * L, lens[b]] for b in ranked_rows], np.int32)).to(DEV)
    seg_keys = torch.from_numpy(np.array([[b, k_end[b]] for b in ranked_rows], np.int32)).to(DEV)
    scale = 1.0 / (32 * H)
    plan = make_plan([SeqRows(batch=b, k_end=k_end[b], rows=np.array([i]), n_imp=1)
                      for i, b in enumerate(ranked_rows)], table, device=DEV)
    sa, pa = base.clone(), torch.from_numpy(full_pos.copy()).to(DEV)
    ta = torch.zeros((len(ranked_rows), k), dtype=torch.int64, device=DEV)
    ops.importance_accumulate(part, plan, scale, sa)
    ops.importance_rank(sa, pa, seg, max(lens), ta, k)
    sb, pb = base.clone(), torch.from_numpy(full_pos.copy()).to(DEV)
    tb = torch.zeros_like(ta)
    ops.importance_rank(sb, pb, seg, max(lens), tb, k, imp_part=part, scale=scale, plan=plan,
                        seg_keys=seg_keys)
    torch.cuda.synchronize()
    assert torch.equal(sb, sa) and torch.equal(pb, pa) and torch.equal(tb, ta)
    # against float64 sums and the oracle's order of the stored scores
    keys = np.concatenate([slots_of[b][:k_end[b]] for b in ranked_rows])
    exp = base.cpu().double().numpy()
    exp[keys] += scale * part.cpu().double().numpy()[:, keys].sum(0)
    got = sb.cpu().numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)
    other = np.setdiff1d(np.arange(n), keys)
    np.testing.assert_array_equal(got[other], base.cpu().numpy()[other])
    pn = pb.cpu().numpy()
    for b in ranked_rows:
        np.testing.assert_array_equal(pn[b, :lens[b]], orc.rank_ascending(got, full_pos[b, :lens[b]]))


# -------------------------------------------------------------------------- verify

def _verify_case(seed, n_blk, k_cache_len, H, bm=32, with_ts=False, s_min=4):
    """Verify blocks in the reference layout (llada/generate.py:260-292): T fill rows,
    S draft rows, S mask rows; keys are all cache slots except fill and candidates. With
    with_ts, also returns the (T, S) of every block."""
    rng = np.random.default_rng(seed)
    rows = 2 * bm
    L = k_cache_len
    key_pos, vblocks, masks, qslots, ts = [], [], [], [], []
    acc_k = 0
    for j in range(n_blk):
        S = int(rng.integers(s_min, bm // 2 + 1))
        T = rows - 2 * S
        ts.append((T, S))
        nd = int(rng.integers(T + 64, L - S - 1))
        order = np.arange(L)
        fill = order[nd - T:nd]
        cand = order[nd:nd + S]
        keys = np.concatenate([order[:nd - T], order[nd + S:]]) + j * L
        key_pos.append(keys)
        vblocks.append((acc_k, acc_k + len(keys), j * rows, (j + 1) * rows))
        acc_k += len(keys)
        masks.append(orc.verify_mask(T, S, bm))
        qslots.append(np.concatenate([fill, cand, cand]) + j * L)
    out = (np.concatenate(key_pos).astype(np.int64), np.asarray(vblocks, np.int32),
           np.concatenate(masks), np.concatenate(qslots).astype(np.int64))
    return out + (np.asarray(ts, np.int32),) if with_ts else out


@pytest.mark.parametrize("bm", [32, 64, 128])
def test_verify_attention_block_rows_up_to_256_and_closed_form_mask(bm):
    """Verify blocks of 2 block_m = 64, 128 and 256 rows (the reference's block_length 32,
    64 and the default 128): 64-row tiles, 128-row tiles, and two 128-row workgroups per
    block, each attending to every in-block key (1, 2 or 4 in-block key blocks). The
    attention with the reference's dense mask matches the oracle, and the closed-form mask
    from each block's (T, S) gives the same output bit for bit."""
    H, n_blk, L = 8, 6, 1024
    key_pos, vblocks, mask, _, ts = _verify_case(21 + bm, n_blk, L, H, bm, with_ts=True, s_min=1)
    rows = 2 * bm
    gen = torch.Generator().manual_seed(22)
    D = H * 128
    q, k1, v1 = (_bf16((n_blk * rows, D), gen) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen) for _ in range(2))
    args = [t.to(DEV) for t in (q, k1, v1, kc, vc)] + [torch.from_numpy(key_pos).to(DEV),
                                                       torch.from_numpy(vblocks).to(DEV)]
    scale = orc.softmax_scale(128)
    out_dense = torch.full((n_blk * rows, D), POISON, dtype=torch.bfloat16, device=DEV)
    out_ts = torch.full_like(out_dense, POISON)
    ops.verify_attention(*args, torch.from_numpy(mask).to(DEV), rows, out_dense, H, scale)
    ops.verify_attention(*args, torch.from_numpy(ts).to(DEV), rows, out_ts, H, scale)
    torch.cuda.synchronize()
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, rows, H, scale)
    _close(_np(out_dense), ref, what=f"verify attention, {rows}-row blocks")
    assert torch.equal(out_ts, out_dense)


def test_verify_attention_closed_form_without_fill_rows():
    """T = 0 (2S rows of drafts then masks, the verify-query workload's layout): the
    closed-form mask against the oracle's mask construction."""
    H, n_blk, L, bm = 4, 5, 512, 16
    rng = np.random.default_rng(31)
    key_pos, vblocks, masks, ts = [], [], [], []
    acc_k = acc_q = 0
    for j in range(n_blk):
        S = int(rng.integers(1, bm + 1))
        cand = j * L + 200 + np.arange(S)
        keys = np.setdiff1d(j * L + np.arange(L), cand)
        key_pos.append(keys)
        vblocks.append((acc_k, acc_k + len(keys), acc_q, acc_q + 2 * S))
        acc_k += len(keys)
        acc_q += 2 * S
        masks.append(orc.verify_mask(0, S, bm))
        ts.append((0, S))
    key_pos = np.concatenate(key_pos).astype(np.int64)
    vblocks = np.asarray(vblocks, np.int32)
    mask = np.concatenate(masks)
    gen = torch.Generator().manual_seed(32)
    D = H * 128
    q, k1, v1 = (_bf16((acc_q, D), gen) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen) for _ in range(2))
    out = torch.full((acc_q, D), POISON, dtype=torch.bfloat16, device=DEV)
    ops.verify_attention(*(t.to(DEV) for t in (q, k1, v1, kc, vc)), torch.from_numpy(key_pos).to(DEV),
                         torch.from_numpy(vblocks).to(DEV),
                         torch.from_numpy(np.asarray(ts, np.int32)).to(DEV), 2 * bm, out, H,
                         orc.softmax_scale(128))
    torch.cuda.synchronize()
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, 2 * bm, H, orc.softmax_scale(128))
    _close(_np(out), ref, what="verify attention, closed-form mask, no fill rows")


def test_verify_attention_batch16_cache1024():
    """16 verify blocks over 1024-slot caches, S in [4, 16] candidates (2S draft/mask rows)
    plus fill rows, 32 heads; own-draft masking from the reference's mask construction."""
    H, bm, n_blk, L = 32, 32, 16, 1024
    key_pos, vblocks, mask, _ = _verify_case(11, n_blk, L, H, bm)
    rows = 2 * bm
    gen = torch.Generator().manual_seed(12)
    D = H * 128
    q, k1, v1 = (_bf16((n_blk * rows, D), gen) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen) for _ in range(2))
    out = torch.full((n_blk * rows, D), POISON, dtype=torch.bfloat16, device=DEV)
    scale = orc.softmax_scale(128)
    ops.verify_attention(q.to(DEV), k1.to(DEV), v1.to(DEV), kc.to(DEV), vc.to(DEV),
                         torch.from_numpy(key_pos).to(DEV), torch.from_numpy(vblocks).to(DEV),
                         torch.from_numpy(mask).to(DEV), rows, out, H, scale)
    torch.cuda.synchronize()
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, rows, H, scale)
    _close(_np(out), ref, what="verify attention")


@pytest.mark.parametrize("bm", [32, 64, 128])
def test_verify_attention_two_heads_per_workgroup_matches_one(bm):
    """A verify grid of more than one round of workgroups (9 blocks x 32 heads, above the
    device's CU count) runs two heads per workgroup, the second head's key blocks streaming
    through the LDS ring behind the first head's. Every (block, head) output equals, bit for
    bit, the one-head launch of that block alone (9 calls of one block: 32 workgroups
    each); 64-, 128- and 256-row blocks (64-row tiles, 128-row tiles, two 128-row tiles)."""
    H, n_blk, L = 32, 9, 512
    key_pos, vblocks, _, _, ts = _verify_case(41 + bm, n_blk, L, H, bm, with_ts=True, s_min=1)
    rows = 2 * bm
    gen = torch.Generator().manual_seed(42 + bm)
    D = H * 128
    q, k1, v1 = (_bf16((n_blk * rows, D), gen).to(DEV) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen).to(DEV) for _ in range(2))
    kp = torch.from_numpy(key_pos).to(DEV)
    vb = torch.from_numpy(vblocks).to(DEV)
    tsd = torch.from_numpy(ts).to(DEV)
    scale = orc.softmax_scale(128)
    out_all = torch.full((n_blk * rows, D), POISON, dtype=torch.bfloat16, device=DEV)
    ops.verify_attention(q, k1, v1, kc, vc, kp, vb, tsd, rows, out_all, H, scale)
    out_one = torch.full_like(out_all, POISON)
    for j in range(n_blk):
        ops.verify_attention(q, k1, v1, kc, vc, kp, vb[j:j + 1].contiguous(),
                             tsd[j:j + 1].contiguous(), rows, out_one, H, scale)
    torch.cuda.synchronize()
    assert not torch.equal(out_all, torch.full_like(out_all, POISON))
    assert torch.equal(out_all, out_one)


def test_verify_end_to_end_projection_and_attention():
    """Packed verify projection followed by verify attention, as the verify pass runs them
    (flash_cache_triton.py:499-535)."""
    H, bm, n_blk, L = 4, 8, 3, 256
    key_pos, vblocks, mask, qslots = _verify_case(13, n_blk, L, H, bm)
    rows = 2 * bm
    gen = torch.Generator().manual_seed(14)
    D = H * 128
    Q = n_blk * rows
    x = _bf16((Q, D), gen)
    wq, wk, wv = (_bf16((D, D), gen, 0.02) for _ in range(3))
    kc, vc = (_bf16((n_blk * L, D), gen) for _ in range(2))
    sin, cos = _rope(L, 500000.0, repeat=n_blk)
    q, k1, v1 = (torch.empty((Q, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    ops.qkv_rope_cache(x.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), sin, cos,
                       torch.from_numpy(qslots).to(DEV), q, k1, v1, H, kv_packed=True)
    out = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
    ops.verify_attention(q, k1, v1, kc.to(DEV), vc.to(DEV), torch.from_numpy(key_pos).to(DEV),
                         torch.from_numpy(vblocks).to(DEV), torch.from_numpy(mask).to(DEV), rows,
                         out, H, orc.softmax_scale(128))
    torch.cuda.synchronize()
    q_ref, k_ref, v_ref = orc.qkv_proj_cache(_np(x), _np(wq), _np(wk), _np(wv), sin.cpu().numpy(),
                                             cos.cpu().numpy(), qslots, H, None, None)
    # attention from the kernel's own bf16 projections isolates the attention error
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, rows, H, orc.softmax_scale(128))
    _close(_np(q), q_ref, what="verify Q")
    _close(_np(k1), k_ref, what="verify K")
    _close(_np(out), ref, what="verify attention")


@pytest.mark.parametrize("page_log2", [4, 7, 12])
def test_block_attention_page_sizes(page_log2):
    """Page sizes 16, 128 and 4096 slots (the ABI's range is 16-4096) in randomly permuted
    tables, cache lengths that are not multiples of the page size, every tile class (64-row,
    128-row, 256-row full recomputes) and key ranges past the staged slot map (2100 keys in
    a 64-row tile, 2200 in a full recompute: slots looked up from the page table in the
    loop), raw importance; against the oracle through the same page table, rows outside the
    tiles untouched."""
    P = 1 << page_log2
    rng = np.random.default_rng(40 + page_log2)
    H = 4
    k_ends = [300, 777, 1100, 2200, 517, 2100]
    q_lens = [40, 100, 1100, 2200, 517, 50]  # 64-row, 128-row, full, full, full, 64-row
    B = len(k_ends)
    max_pages = (max(k_ends) + P - 1) // P
    n_pages = sum((k + P - 1) // P for k in k_ends) + 3
    perm = rng.permutation(n_pages)
    table = np.zeros((B, max_pages), np.int32)
    nxt = 0
    for b in range(B):
        for p in range((k_ends[b] + P - 1) // P):
            table[b, p] = perm[nxt]
            nxt += 1
    seqs, row = [], 2  # rows 0 and 1 belong to no tile
    for b in range(B):
        rows = np.arange(row, row + q_lens[b])
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=rows, n_imp=min(q_lens[b], 32)))
        row += q_lens[b]
    Q = row
    n_slots = n_pages * P
    q, kc, vc = _attn_inputs(41 + page_log2, Q, n_slots, H)
    plan = make_plan(seqs, table, page_log2, device=DEV)
    plan.validate(Q, n_slots)
    assert plan.n_long > 0 and plan.n_mid > 0 and plan.n_work > plan.n_long + plan.n_mid
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, n_slots), dtype=torch.float32, device=DEV)
    scores = torch.zeros(n_slots, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale,
                        lib.IMP_RAW_LOGIT, imp)
    ops.importance_accumulate(imp, plan, 1.0, scores)
    torch.cuda.synchronize()
    qn, kn, vn = _np(q), _np(kc), _np(vc)
    got = _np(out)
    assert (got[:2] == POISON).all()
    sc = scores.cpu().numpy()
    for sq in seqs:
        blk = np.array([[sq.batch, sq.k_end, sq.rows[0], sq.rows[-1] + 1]])
        ref = orc.block_attention(qn, kn, vn, blk, 0, H, scale, page_table=table, page_size=P)
        _close(got[sq.rows], ref[sq.rows], what=f"page {P}, seq {sq.batch}")
        keys = orc.key_slots(sq.batch, sq.k_end, 0, table, P)
        exp = np.zeros(len(keys))
        for h in range(H):
            cols = slice(h * 128, (h + 1) * 128)
            exp += (qn[sq.rows[:sq.n_imp]][:, cols] @ kn[keys][:, cols].T).sum(0)
        _close(sc[keys], exp, atol=2e-3, rtol=1e-4, what=f"page {P}, importance seq {sq.batch}")


@pytest.mark.parametrize("n_heads,Q", [(2, 40), (2, 100), (2, 300), (6, 40), (6, 300), (20, 64),
                                       (20, 700), (40, 40), (40, 200)])
def test_qkv_rope_cache_head_counts(n_heads, Q):
    """Head counts 2, 6, 20 and 40 (d_model 256-5120): tile counts that are not multiples of
    the eight XCDs (6 heads: 36 weight-streaming tiles), the three launch shapes, and
    reductions of 4 steps, fewer than the 6 or 8 steps the weight-streaming shapes request
    before their loop, against the oracle; untouched cache rows keep their contents."""
    rng = np.random.default_rng(100 + n_heads + Q)
    n_slots = max(1024, 2 * Q)
    slots = rng.choice(n_slots, Q, replace=False)
    q, kc, vc, q_ref, k_ref, v_ref, s = _qkv_case(200 + Q, n_heads, Q, n_slots, slots)
    _close(_np(q), q_ref, what="Q")
    _close(_np(kc)[s], k_ref[s], what="K rows")
    _close(_np(vc)[s], v_ref[s], what="V rows")
    untouched = np.setdiff1d(np.arange(n_slots), s)
    assert np.all(_np(kc)[untouched] == POISON) and np.all(_np(vc)[untouched] == POISON)


def _f64_attention(qr, keys_k, keys_v, scale):
    s = (qr @ keys_k.T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return p @ keys_v, p


@pytest.mark.parametrize("seed", range(6))
def test_block_attention_random_plans(seed):
    """Seeded random launches: 1-7 sequences with key ranges [k_begin, k_end), k_end up to
    1300 (a quarter of them starting past 0), 1-200 query rows or a full recompute (q = k),
    every sequence's rows scattered over the packed row space, pages of 16-256 slots
    permuted over a pool, one, two or four heads, the three importance modes in turn. The
    outputs against float64 softmax attention over each sequence's keys; the per-head
    importance partials at every key slot (zero for sequences without importance rows and
    for slots outside every key range)."""
    rng = np.random.default_rng(1000 + seed)
    imp_mode = (lib.IMP_NONE, lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM)[seed % 3]
    H = int(rng.choice([1, 2, 4]))
    page_log2 = int(rng.choice([4, 5, 6, 8]))
    P = 1 << page_log2
    B = int(rng.integers(1, 8))
    specs = []
    for _ in range(B):
        k_end = int(rng.integers(1, 1301))
        k_begin = int(rng.integers(0, k_end)) if rng.random() < 0.25 else 0
        nq = k_end - k_begin if rng.random() < 0.2 else int(rng.integers(1, 201))
        n_imp = 0 if imp_mode == lib.IMP_NONE else int(rng.integers(0, min(nq, 64) + 1))
        specs.append((k_begin, k_end, nq, n_imp))
    max_pages = (1300 + P - 1) // P
    n_pages = sum((k + P - 1) // P for _, k, _, _ in specs) + 5
    perm = rng.permutation(n_pages)
    table = np.zeros((B, max_pages), np.int32)
    nxt = 0
    for b, (_, k_end, _, _) in enumerate(specs):
        for p in range((k_end + P - 1) // P):
            table[b, p] = perm[nxt]
            nxt += 1
    Q = sum(s[2] for s in specs)
    row_perm = rng.permutation(Q)
    seqs, off = [], 0
    for b, (k_begin, k_end, nq, n_imp) in enumerate(specs):
        seqs.append(SeqRows(batch=b, k_end=k_end, rows=row_perm[off:off + nq], n_imp=n_imp,
                            k_begin=k_begin))
        off += nq
    n_slots = n_pages * P
    q, kc, vc = _attn_inputs(2000 + seed, Q, n_slots, H)
    plan = make_plan(seqs, table, page_log2, device=DEV)
    plan.validate(Q, n_slots)
    out = torch.full((Q, H * 128), POISON, dtype=torch.bfloat16, device=DEV)
    imp = torch.zeros((H, n_slots), dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(128)
    print(f"seed {seed}: H {H}, page {P}, imp {imp_mode}, specs {specs}", flush=True)
    ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), plan, out, H, scale, imp_mode,
                        imp if imp_mode else None)
    torch.cuda.synchronize()
    qn, kn, vn = (_np(t).astype(np.float64) for t in (q, kc, vc))
    got, gimp = _np(out), imp.cpu().numpy()
    covered = np.zeros(n_slots, bool)
    for b, sq in enumerate(seqs):
        keys = orc.key_slots(b, sq.k_end, 0, table, P, k_begin=sq.k_begin)
        covered[keys] = True
        for h in range(H):
            cols = slice(h * 128, (h + 1) * 128)
            o, p = _f64_attention(qn[sq.rows][:, cols], kn[keys][:, cols], vn[keys][:, cols],
                                  scale)
            _close(got[sq.rows][:, cols], o, what=f"seq {b} head {h}")
            if imp_mode == lib.IMP_RAW_LOGIT:
                exp = (qn[sq.rows[:sq.n_imp]][:, cols] @ kn[keys][:, cols].T).sum(0)
                _close(gimp[h, keys], exp, atol=5e-3, rtol=1e-4, what=f"raw imp seq {b} head {h}")
            elif imp_mode == lib.IMP_SOFTMAX_COLSUM:
                exp = p[:sq.n_imp].sum(0)
                _close(gimp[h, keys], exp, atol=1e-3, rtol=1e-3, what=f"softmax imp seq {b} head {h}")
    assert not gimp[:, ~covered].any()


def test_qkv_rope_halves_flag():
    """FDL_QKV_ROPE_HALVES_EQUAL. With the reference's tables (every row repeats its first
    half) the projection that reads one half equals the one that reads both, bit for bit, and
    the wrapper detects the repetition. Tables whose halves differ are detected as such and
    projected with both halves (against the oracle); with the flag forced on them, the high
    half's sin/cos are not read (the output changes)."""
    H, Q, L = 4, 300, 512
    gen = torch.Generator().manual_seed(41)
    D = H * 128
    x = _bf16((Q, D), gen)
    w = [_bf16((D, D), gen, 0.02) for _ in range(3)]
    slots = torch.from_numpy(np.random.default_rng(42).permutation(L)[:Q].astype(np.int64))
    sin, cos = _rope(L)
    assert ops.tables_repeat_halves(sin, cos)
    xd, wd, sd = x.to(DEV), [t.to(DEV) for t in w], slots.to(DEV)

    def run(s, c, flag):
        q = torch.zeros((Q, D), dtype=torch.bfloat16, device=DEV)
        kc = torch.full((L, D), POISON, dtype=torch.bfloat16, device=DEV)
        vc = torch.full_like(kc, POISON)
        ops.qkv_rope_cache(xd, *wd, s, c, sd, q, kc, vc, H, rope_halves_equal=flag)
        torch.cuda.synchronize()
        return q, kc, vc

    both, half, auto = run(sin, cos, False), run(sin, cos, True), run(sin, cos, None)
    for t0, t1, t2 in zip(both, half, auto):
        assert torch.equal(t0, t1) and torch.equal(t0, t2)
    ang = np.random.default_rng(43).uniform(-3.0, 3.0, (L, 128)).astype(np.float32)
    s2, c2 = torch.from_numpy(np.sin(ang)).to(DEV), torch.from_numpy(np.cos(ang)).to(DEV)
    assert not ops.tables_repeat_halves(s2, c2)
    q, kc, vc = run(s2, c2, None)
    poison = np.full((L, D), POISON, np.float32)
    q_ref, k_ref, v_ref = orc.qkv_proj_cache(_np(x), _np(w[0]), _np(w[1]), _np(w[2]),
                                             s2.cpu().numpy(), c2.cpu().numpy(), slots.numpy(),
                                             H, poison, poison)
    _close(_np(q), q_ref, what="q, halves differ")
    _close(_np(kc), k_ref, what="k cache, halves differ")
    _close(_np(vc), v_ref, what="v cache, halves differ")
    assert not torch.equal(run(s2, c2, True)[0], q)


@pytest.mark.parametrize("seed", range(4))
def test_verify_attention_random_blocks(seed):
    """Seeded random Flash-Verify launches: block_m 8-128 (blocks of up to 256 rows), 1-40
    blocks (past 256 workgroups two heads share one), one to eight heads, each block with
    its own (T, S) (T fill rows, S drafts and S masks, fewer rows than the block holds) and a
    key list of 0-2500 cache slots in random order; the closed-form mask in even seeds, the
    reference's dense mask in odd ones. Against the oracle; rows outside the blocks keep their
    contents."""
    rng = np.random.default_rng(3000 + seed)
    H = int(rng.choice([1, 2, 4, 8]))
    bm = int(rng.choice([8, 16, 32, 64, 128]))
    n_blk = int(rng.integers(1, 41))
    if seed == 3:
        H, n_blk = 8, 40  # 320 (block, head) pairs: two heads per workgroup
    rows_cap = 2 * bm
    L = 2600
    key_pos, vblocks, masks, ts = [], [], [], []
    acc_k = acc_q = 0
    for _ in range(n_blk):
        S = int(rng.integers(1, bm + 1))
        T = int(rng.integers(0, rows_cap - 2 * S + 1))
        nk = int(rng.integers(0, 2501))
        keys = rng.choice(L, nk, replace=False)
        key_pos.append(keys)
        vblocks.append((acc_k, acc_k + nk, acc_q, acc_q + T + 2 * S))
        acc_k += nk
        acc_q += T + 2 * S
        masks.append(orc.verify_mask(T, S, bm))
        ts.append((T, S))
    Q = acc_q + 3  # three rows past the last block stay untouched
    key_pos = np.concatenate(key_pos).astype(np.int64)
    vblocks = np.asarray(vblocks, np.int32)
    mask = np.concatenate(masks)
    lib.call("fdl_validate_vblocks", vblocks.ctypes.data, n_blk,
             key_pos.ctypes.data if key_pos.size else None, key_pos.size, Q, L, rows_cap)
    gen = torch.Generator().manual_seed(3100 + seed)
    D = H * 128
    q, k1, v1 = (_bf16((Q, D), gen) for _ in range(3))
    kc, vc = (_bf16((L, D), gen) for _ in range(2))
    out = torch.full((Q, D), POISON, dtype=torch.bfloat16, device=DEV)
    meta = (torch.from_numpy(np.asarray(ts, np.int32)) if seed % 2 == 0
            else torch.from_numpy(mask))
    print(f"seed {seed}: H {H}, block_m {bm}, {n_blk} blocks, {key_pos.size} keys", flush=True)
    ops.verify_attention(*(t.to(DEV) for t in (q, k1, v1, kc, vc)),
                         torch.from_numpy(key_pos).to(DEV), torch.from_numpy(vblocks).to(DEV),
                         meta.to(DEV), rows_cap, out, H, orc.softmax_scale(128))
    torch.cuda.synchronize()
    ref = orc.verify_attention(_np(q), _np(k1), _np(v1), _np(kc), _np(vc), key_pos, mask,
                               vblocks, rows_cap, H, orc.softmax_scale(128))
    got = _np(out)
    _close(got[:acc_q], ref[:acc_q], what=f"verify attention, seed {seed}")
    assert np.all(got[acc_q:] == POISON)
