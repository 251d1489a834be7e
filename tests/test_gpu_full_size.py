"""Parity at the full sizes of the block-table stress and Flash-Verify workloads (d_model
4096, 32 heads, bf16): the whole batch runs on the GPU through the C ABI, and sampled
pieces of it are checked against the oracle on the CPU (projected rows, cache rows,
(row, head) attention outputs, importance slots), so the CPU side stays at seconds.
Untouched cache rows are compared bit for bit on the GPU.

Bars as elsewhere: bf16 outputs within atol 2e-2 / rtol 1e-2 of the float32 oracle; raw
importance within 2e-3 absolute (its terms are sums over 4096 products)."""
import numpy as np
import pytest
import torch

from oracle import flash_cache_oracle as orc
from fdl import lib, ops
from fdl.generate import verify_mask
from fdl.schedule import SeqRows, make_plan

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
H, HD = 32, 128
D = H * HD
ATOL, RTOL = 2e-2, 1e-2
THETA = 500000.0


def _bf(gen, *shape, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)


def _np(t):
    return t.float().cpu().numpy()


def _rope(n):
    sin, cos = orc.rope_tables(n, HD, THETA)
    return sin, cos


def test_block_table_stress_full_size_sampled():
    """32 sequences, k_end uniform in [512, 1536], a quarter full recomputes (q = k, 256-row
    tiles), the rest 1-96 query rows (masked block at a frontier + decoded slots), 32-slot
    pages permuted over one pool; fused QKV + cache write, block attention with raw
    importance, head reduction."""
    rng = np.random.default_rng(31)
    gen = torch.Generator().manual_seed(31)
    NB, P = 32, 32
    k_ends = rng.integers(512, 1537, NB)
    full = rng.random(NB) < 0.25
    full[0] = True
    pages = [(int(k) + P - 1) // P for k in k_ends]
    n_pages = int(sum(pages)) + 3
    perm = rng.permutation(n_pages)
    table = np.zeros((NB, max(pages)), np.int32)
    nxt = 0
    for b in range(NB):
        table[b, :pages[b]] = perm[nxt:nxt + pages[b]]
        nxt += pages[b]
    n_slots = n_pages * P
    seqs, logical_all, row = [], [], 0
    for b in range(NB):
        k = int(k_ends[b])
        if full[b]:
            logical = np.arange(k)
        else:
            qn = int(rng.integers(1, 97))
            m = min(qn, 32)
            f = int(rng.integers(96, k - 32 + 1))
            rest = rng.choice(f, qn - m, replace=False) if qn > m else np.zeros(0, np.int64)
            logical = np.concatenate([np.arange(f, f + m), rest]).astype(np.int64)
        logical_all.append(logical)
        seqs.append(SeqRows(batch=b, k_end=k, rows=np.arange(row, row + len(logical)),
                            n_imp=min(len(logical), 32)))
        row += len(logical)
    Q = row
    slots = np.concatenate([table[b, lg // P].astype(np.int64) * P + lg % P
                            for b, lg in enumerate(logical_all)])
    rope_row = np.concatenate(logical_all)
    sin, cos = _rope(1536)

    x = _bf(gen, Q, D)
    w = [_bf(gen, D, D, std=0.02) for _ in range(3)]
    kc0, vc0 = _bf(gen, n_slots, D), _bf(gen, n_slots, D)
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    q = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
    ops.qkv_rope_cache(x.to(DEV), *(t.to(DEV) for t in w), torch.from_numpy(sin).to(DEV),
                       torch.from_numpy(cos).to(DEV), torch.from_numpy(slots).to(DEV), q, kc,
                       vc, H, rope_row=torch.from_numpy(rope_row).to(DEV))
    plan = make_plan(seqs, table, 5, device=DEV)
    plan.validate(Q, n_slots)
    att = torch.empty_like(q)
    imp = torch.zeros((H, n_slots), dtype=torch.float32, device=DEV)
    scores = torch.zeros(n_slots, dtype=torch.float32, device=DEV)
    scale = orc.softmax_scale(HD)
    ops.block_attention(q, kc, vc, plan, att, H, scale, lib.IMP_RAW_LOGIT, imp)
    ops.importance_accumulate(imp, plan, 1.0, scores)
    torch.cuda.synchronize()

    # cache rows other than the written slots are untouched (bit for bit, on the GPU)
    untouched = torch.ones(n_slots, dtype=torch.bool, device=DEV)
    untouched[torch.from_numpy(slots).to(DEV)] = False
    assert torch.equal(kc[untouched], kc0.to(DEV)[untouched])
    assert torch.equal(vc[untouched], vc0.to(DEV)[untouched])

    # projected rows: a sample of 48 rows, Q and the written K/V cache rows
    pick = rng.choice(Q, 48, replace=False)
    q_ref, k_ref, v_ref = orc.qkv_proj_cache(_np(x[pick]), *(_np(t) for t in w), sin, cos,
                                             slots[pick], H, None, None, rope_row=rope_row[pick])
    np.testing.assert_allclose(_np(q[pick]), q_ref, atol=ATOL, rtol=RTOL, err_msg="Q rows")
    sl = torch.from_numpy(slots[pick]).to(DEV)
    np.testing.assert_allclose(_np(kc[sl]), k_ref, atol=ATOL, rtol=RTOL, err_msg="K rows")
    np.testing.assert_allclose(_np(vc[sl]), v_ref, atol=ATOL, rtol=RTOL, err_msg="V rows")

    # attention: 96 sampled (row, head) pairs, a third of them from full recomputes
    qn = _np(q)
    row_seq = np.concatenate([np.full(len(s.rows), i) for i, s in enumerate(seqs)])
    full_rows = np.flatnonzero(full[row_seq])
    rows = np.concatenate([rng.choice(full_rows, 32, replace=False), rng.choice(Q, 64, replace=False)])
    heads = rng.integers(0, H, len(rows))
    got = _np(att)
    kcn, vcn = kc.cpu(), vc.cpu()
    for r, h in zip(rows, heads):
        sq = seqs[row_seq[r]]
        keys = orc.key_slots(sq.batch, sq.k_end, 0, table, P)
        cols = slice(h * HD, (h + 1) * HD)
        ref = orc.attend(qn[r:r + 1, cols], kcn[keys][:, cols].float().numpy(),
                         vcn[keys][:, cols].float().numpy(), 1, scale)
        np.testing.assert_allclose(got[r, cols], ref[0], atol=ATOL, rtol=RTOL,
                                   err_msg=f"row {r} head {h} (sequence {sq.batch})")

    # raw importance: scores[slot(n)] = sum over the first n_imp rows of q_r . k_n (all heads)
    sc = scores.cpu().numpy()
    for sq in seqs[:8]:
        keys = orc.key_slots(sq.batch, sq.k_end, 0, table, P)
        sample = rng.choice(keys, 16, replace=False)
        qsum = qn[sq.rows[:sq.n_imp]].astype(np.float64).sum(0)
        exp = kcn[sample].double().numpy() @ qsum
        np.testing.assert_allclose(sc[sample], exp, atol=2e-3, rtol=1e-4,
                                   err_msg=f"importance, sequence {sq.batch}")


def test_flash_verify_full_size_sampled():
    """16 sequences with 1024-slot caches, 4-32 candidates each as draft and mask rows
    (packed without padding): packed verify QKV, then verify attention over the cache keys
    (every slot but the candidates) and the in-block keys under the verify mask; four whole
    blocks checked against the oracle, all heads."""
    rng = np.random.default_rng(41)
    gen = torch.Generator().manual_seed(41)
    NV, LC, BM = 16, 1024, 32
    kv = rng.integers(4, 33, NV)
    key_pos, vblocks, masks, qslots = [], [], [], []
    k0 = q0 = 0
    for b in range(NV):
        S = int(kv[b])
        cand = b * LC + 512 + np.arange(S)
        keys = np.setdiff1d(b * LC + np.arange(LC), cand)
        key_pos.append(keys)
        vblocks.append([k0, k0 + len(keys), q0, q0 + 2 * S])
        k0 += len(keys)
        q0 += 2 * S
        masks.append(verify_mask(0, S, BM))
        qslots.append(np.concatenate([cand, cand]))
    QV = q0
    key_pos = np.concatenate(key_pos).astype(np.int64)
    vblocks = np.array(vblocks, dtype=np.int32)
    mask = np.concatenate(masks).astype(np.uint8)
    qs = np.concatenate(qslots).astype(np.int64)
    sin, cos = _rope(LC)
    sin, cos = np.tile(sin, (NV, 1)), np.tile(cos, (NV, 1))

    xv = _bf(gen, QV, D)
    w = [_bf(gen, D, D, std=0.02) for _ in range(3)]
    kcv, vcv = _bf(gen, NV * LC, D), _bf(gen, NV * LC, D)
    qv, k1, v1 = (torch.empty((QV, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    ops.qkv_rope_cache(xv.to(DEV), *(t.to(DEV) for t in w), torch.from_numpy(sin).to(DEV),
                       torch.from_numpy(cos).to(DEV), torch.from_numpy(qs).to(DEV), qv, k1, v1,
                       H, kv_packed=True)
    attv = torch.empty_like(qv)
    scale = orc.softmax_scale(HD)
    ops.verify_attention(qv, k1, v1, kcv.to(DEV), vcv.to(DEV), torch.from_numpy(key_pos).to(DEV),
                         torch.from_numpy(vblocks).to(DEV), torch.from_numpy(mask).to(DEV), 2 * BM,
                         attv, H, scale)
    torch.cuda.synchronize()

    pick = rng.choice(QV, 32, replace=False)
    q_ref, k_ref, v_ref = orc.qkv_proj_cache(_np(xv[pick]), *(_np(t) for t in w), sin, cos,
                                             qs[pick], H, None, None)
    np.testing.assert_allclose(_np(qv[pick]), q_ref, atol=ATOL, rtol=RTOL, err_msg="Q rows")
    np.testing.assert_allclose(_np(k1[pick]), k_ref, atol=ATOL, rtol=RTOL, err_msg="packed K")
    np.testing.assert_allclose(_np(v1[pick]), v_ref, atol=ATOL, rtol=RTOL, err_msg="packed V")

    qn, k1n, v1n, kcn, vcn = _np(qv), _np(k1), _np(v1), _np(kcv), _np(vcv)
    got = _np(attv)
    for v in rng.choice(NV, 4, replace=False):
        kk0, kk1, r0, r1 = (int(t) for t in vblocks[v])
        ref = orc.verify_attention(qn[r0:r1], k1n[r0:r1], v1n[r0:r1], kcn, vcn, key_pos,
                                   mask[v * 2 * BM:(v + 1) * 2 * BM],
                                   np.array([[kk0, kk1, 0, r1 - r0]]), 2 * BM, H, scale)
        np.testing.assert_allclose(got[r0:r1], ref, atol=ATOL, rtol=RTOL,
                                   err_msg=f"verify block {v}")


def test_page_placement_invariance_full_size():
    """The block-table stress batch at full size (32 sequences, 6842 rows, every tile class)
    with its K/V pages moved to other physical pages and the page table rewritten to match:
    the fused projection (rows scattered to the moved slots, RoPE by logical position) and
    the block attention with raw importance give bit-identical results, the importance
    partials at the moved slots. Keys are visited in logical order whatever their placement,
    so any difference would be an addressing error."""
    import bench
    st = bench.build_stress(seed=7)
    P, n_slots, Q = st["P"], st["n_slots"], st["Q"]
    n_pages = n_slots // P
    rng = np.random.default_rng(77)
    newpos = rng.permutation(n_pages)  # physical page p moves to newpos[p]
    moved = (newpos[np.arange(n_slots) // P] * P + np.arange(n_slots) % P).astype(np.int64)
    table2 = newpos[st["table"]].astype(np.int32)
    sin, cos = st["sin"].to(DEV), st["cos"].to(DEV)
    x = st["x"].to(DEV)
    w = [t.to(DEV) for t in st["w"]]
    rope_row = torch.from_numpy(st["rope_row"]).to(DEV)
    results = []
    for layout in (0, 1):
        if layout == 0:
            kc, vc = st["kc"].to(DEV), st["vc"].to(DEV)
            slots, table = st["slots"], st["table"]
        else:
            kc = torch.empty((n_slots, D), dtype=torch.bfloat16, device=DEV)
            vc = torch.empty_like(kc)
            kc[torch.from_numpy(moved).to(DEV)] = st["kc"].to(DEV)
            vc[torch.from_numpy(moved).to(DEV)] = st["vc"].to(DEV)
            slots, table = moved[st["slots"]], table2
        q = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
        ops.qkv_rope_cache(x, *w, sin, cos, torch.from_numpy(slots).to(DEV), q, kc, vc, H,
                           rope_row=rope_row)
        plan = make_plan(st["seqs"], table, 5, device=DEV)
        plan.validate(Q, n_slots)
        out = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
        imp = torch.zeros((H, n_slots), dtype=torch.float32, device=DEV)
        ops.block_attention(q, kc, vc, plan, out, H, 1.0 / np.sqrt(HD), lib.IMP_RAW_LOGIT, imp)
        torch.cuda.synchronize()
        results.append((q, kc, vc, out, imp))
    (q1, kc1, vc1, out1, imp1), (q2, kc2, vc2, out2, imp2) = results
    mv = torch.from_numpy(moved).to(DEV)
    assert torch.equal(q1, q2)
    assert torch.equal(kc2[mv], kc1) and torch.equal(vc2[mv], vc1)
    assert torch.equal(out1, out2)
    assert torch.equal(imp2[:, mv], imp1)
    assert imp1.abs().sum() > 0


def test_row_order_invariance_full_size():
    """The block-table stress batch at full size without importance, each sequence's query
    rows listed in a shuffled order: rows land in other tiles, wavefronts and lanes (and
    other 256-row tiles of the full recomputes), and every output row is bit-identical,
    since a row's attention is computed over the same keys in the same order wherever it
    sits."""
    import bench
    st = bench.build_stress(seed=9)
    P, n_slots, Q = st["P"], st["n_slots"], st["Q"]
    rng = np.random.default_rng(91)
    gen = torch.Generator().manual_seed(92)
    q = _bf(gen, Q, D).to(DEV)
    kc, vc = st["kc"].to(DEV), st["vc"].to(DEV)
    shuffled = [SeqRows(batch=s.batch, k_end=s.k_end, rows=rng.permutation(s.rows), n_imp=0)
                for s in st["seqs"]]
    outs = []
    for seqs in (st["seqs"], shuffled):
        plan = make_plan(seqs, st["table"], 5, device=DEV)
        out = torch.empty((Q, D), dtype=torch.bfloat16, device=DEV)
        ops.block_attention(q, kc, vc, plan, out, H, 1.0 / np.sqrt(HD))
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_verify_block_order_invariance_full_size():
    """The Flash-Verify batch at full size (16 blocks x 32 heads: two heads per workgroup),
    its packed projection, then the verify attention with the closed-form masks over the
    blocks listed forward and reversed: every block's rows are bit-identical (a block's
    rows attend to its own key list and in-block keys in the same order either way)."""
    import bench
    vf = bench.build_verify(seed=11)
    Q = vf["Q"]
    x = vf["x"].to(DEV)
    w = [t.to(DEV) for t in vf["w"]]
    sin, cos = vf["sin"].to(DEV), vf["cos"].to(DEV)
    q, k1, v1 = (torch.empty((Q, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    ops.qkv_rope_cache(x, *w, sin, cos, torch.from_numpy(vf["slots"]).to(DEV), q, k1, v1, H,
                       kv_packed=True)
    kc, vc = vf["kc"].to(DEV), vf["vc"].to(DEV)
    kp = torch.from_numpy(vf["key_pos"]).to(DEV)
    ts = np.array([[0, int(s)] for s in vf["kv"]], np.int32)  # T = 0 fill rows, S candidates
    rows = 2 * vf["BMV"]
    outs = []
    for order in (np.arange(vf["NV"]), np.arange(vf["NV"])[::-1]):
        vb = torch.from_numpy(np.ascontiguousarray(vf["vblocks"][order])).to(DEV)
        tsd = torch.from_numpy(np.ascontiguousarray(ts[order])).to(DEV)
        out = torch.full((Q, D), 7.0, dtype=torch.bfloat16, device=DEV)
        ops.verify_attention(q, k1, v1, kc, vc, kp, vb, tsd, rows, out, H, 1.0 / np.sqrt(HD))
        outs.append(out)
    torch.cuda.synchronize()
    assert vf["NV"] * H > 256
    assert torch.equal(outs[0], outs[1])
    assert not (outs[0] == 7.0).all(dim=1).any()  # every row written
