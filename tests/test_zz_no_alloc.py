"""fdl_block_attention_scores_noalloc (the entry point that allocates nothing) against
fdl_block_attention + fdl_importance_accumulate with a caller workspace, through the C ABI:
attention output and scores bit for bit, on two calls in a row, the second one smaller
(the library's static scratch keeps the first call's partials); and captured in a HIP graph,
every replay equal to the eager call."""
import numpy as np
import pytest
import torch

from fdl import lib, ops
from fdl.schedule import LONG_TILE_ROWS, MAX_TILE_ROWS, MID_TILE_ROWS, SeqRows, make_plan

DEV = "cuda:0"


def _classes(plan):
    n_short = plan.n_work - plan.n_long - plan.n_mid
    return [(0, plan.n_long, LONG_TILE_ROWS), (plan.n_long, plan.n_mid, MID_TILE_ROWS),
            (plan.n_long + plan.n_mid, n_short, MAX_TILE_ROWS)]


def _case(seed, n_seq, k_ends, q_rows, H, P=32):
    """Sequences b with k_ends[b] keys in permuted pages and q_rows[b] query rows (the first
    min(32, rows) of them importance rows)."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    D = H * 128
    pages = [(k + P - 1) // P for k in k_ends]
    n_pages = sum(pages) + 3
    perm = rng.permutation(n_pages)
    table = np.zeros((n_seq, max(pages)), np.int32)
    nxt = 0
    for b in range(n_seq):
        table[b, :pages[b]] = perm[nxt:nxt + pages[b]]
        nxt += pages[b]
    seqs, row = [], 0
    for b in range(n_seq):
        seqs.append(SeqRows(batch=b, k_end=k_ends[b], rows=np.arange(row, row + q_rows[b]),
                            n_imp=min(32, q_rows[b])))
        row += q_rows[b]
    n_slots = n_pages * P
    q = torch.randn((row, D), generator=gen).to(torch.bfloat16).to(DEV)
    kc = torch.randn((n_slots, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((n_slots, D), generator=gen).to(torch.bfloat16).to(DEV)
    scores0 = torch.randn(n_slots, generator=gen).to(DEV)
    plan = make_plan(seqs, table, 5, device=DEV)
    plan.validate(row, n_slots)
    return q, kc, vc, plan, scores0, H


def _run_both(case, imp_mode):
    q, kc, vc, plan, scores0, H = case
    D = q.shape[1]
    n_slots = kc.shape[0]
    scale = 1.0 / np.sqrt(128)
    imp_scale = 1.0 / (32 * H) if imp_mode == lib.IMP_RAW_LOGIT else 1.0
    stream = torch.cuda.current_stream().cuda_stream
    out_ref = torch.zeros_like(q)
    out_new = torch.zeros_like(q)
    sc_ref = scores0.clone()
    sc_new = scores0.clone()
    imp = torch.zeros((H, n_slots), dtype=torch.float32, device=DEV)
    # the workspace entry point keeps the softmax probabilities for one pass as the
    # scratch of the allocation-free one does for these sizes; in the other modes neither
    # leg gets a workspace (one would let fdl_block_attention split the keys of a launch
    # that fills at most a quarter of the device, which the allocation-free entry never does)
    ws = None
    if imp_mode == lib.IMP_SOFTMAX_COLSUM:
        ws = torch.empty(max(ops.attention_workspace_floats(plan, H), 4), dtype=torch.float32,
                         device=DEV)
    n_idx = max(int(plan.row_idx.size), 1)
    for first, count, tile_rows in _classes(plan):
        if count == 0:
            continue
        common = (kc.data_ptr(), vc.data_ptr(), q.shape[0], n_slots, D, H, 128,
                  plan.page_table_d.data_ptr(), plan.page_table.shape[0], plan.page_table.shape[1],
                  plan.page_log2, plan.work_d[first:].data_ptr(), count, plan.row_idx_d.data_ptr(),
                  n_idx, tile_rows, scale)
        lib.call("fdl_block_attention", q.data_ptr(), *common, out_ref.data_ptr(), imp_mode,
                 imp.data_ptr() if imp_mode else None, None if ws is None else ws.data_ptr(),
                 0 if ws is None else ws.numel(), stream)
        if imp_mode:
            lib.call("fdl_importance_accumulate", imp.data_ptr(), H, n_slots,
                     plan.page_table_d.data_ptr(), plan.page_table.shape[0],
                     plan.page_table.shape[1], plan.page_log2, plan.work_d[first:].data_ptr(),
                     count, imp_scale, sc_ref.data_ptr(), stream)
        lib.call("fdl_block_attention_scores_noalloc", q.data_ptr(), *common, out_new.data_ptr(),
                 imp_mode, imp_scale, sc_new.data_ptr(), stream)
    torch.cuda.synchronize()
    return out_ref, out_new, sc_ref, sc_new


@pytest.mark.gpu
@pytest.mark.parametrize("imp_mode", [lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM, lib.IMP_NONE])
def test_noalloc_matches_workspace_entry_points_twice(imp_mode):
    # first call: 5 sequences over every tile class (a 300-row full recompute: long tiles,
    # 100 rows: a mid tile, 64 and 40 rows: short tiles, 1 row), 32 heads
    big = _case(21, 5, [300, 700, 900, 513, 128], [300, 100, 64, 40, 1], 32)
    # second call, smaller: 2 sequences, fewer keys and heads
    small = _case(22, 2, [200, 96], [48, 20], 8)
    for case in (big, small):
        out_ref, out_new, sc_ref, sc_new = _run_both(case, imp_mode)
        assert torch.equal(out_new, out_ref)
        assert torch.equal(sc_new, sc_ref)
        if imp_mode != lib.IMP_NONE:
            assert not torch.equal(sc_new, case[4])  # the scores did move


def test_noalloc_rejects_partials_beyond_the_scratch():
    # 32 heads x 300000 slots x 4 bytes > 32 MiB: rejected on the host before any GPU work
    with pytest.raises(lib.FdlError) as ei:
        lib.call("fdl_block_attention_scores_noalloc", None, None, None, 4, 300000, 4096, 32, 128,
                 None, 1, 1, 5, None, 1, None, 1, 64, 0.1, None, lib.IMP_RAW_LOGIT, 1.0, None, None)
    assert ei.value.status == lib.FDL_ERR_UNSUPPORTED
    assert "scratch" in str(ei.value)


@pytest.mark.gpu
@pytest.mark.parametrize("imp_mode", [lib.IMP_RAW_LOGIT, lib.IMP_SOFTMAX_COLSUM])
def test_noalloc_captured_in_a_graph(imp_mode):
    """The allocation-free entry point as its callers use it: captured in a HIP graph (every
    tile class of the 5-sequence case), replayed four times with the scores reset and the
    output poisoned by eager work between the replays; every replay equals the eager call."""
    q, kc, vc, plan, scores0, H = _case(23, 5, [300, 700, 900, 513, 128],
                                        [300, 100, 64, 40, 1], 32)
    n_slots, D = kc.shape[0], q.shape[1]
    scale = 1.0 / np.sqrt(128)
    imp_scale = 1.0 / (32 * H) if imp_mode == lib.IMP_RAW_LOGIT else 1.0
    out = torch.empty_like(q)
    sc = torch.empty_like(scores0)
    n_idx = max(int(plan.row_idx.size), 1)

    def call(stream):
        for first, count, tile_rows in _classes(plan):
            if count:
                lib.call("fdl_block_attention_scores_noalloc", q.data_ptr(), kc.data_ptr(),
                         vc.data_ptr(), q.shape[0], n_slots, D, H, 128,
                         plan.page_table_d.data_ptr(), plan.page_table.shape[0],
                         plan.page_table.shape[1], plan.page_log2,
                         plan.work_d[first:].data_ptr(), count, plan.row_idx_d.data_ptr(), n_idx,
                         tile_rows, scale, out.data_ptr(), imp_mode, imp_scale, sc.data_ptr(),
                         stream)

    def reset():
        sc.copy_(scores0)
        out.fill_(float("nan"))

    reset()
    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = (out.clone(), sc.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]), f"replay {rep}: output"
        assert torch.equal(sc, eager[1]), f"replay {rep}: scores"
