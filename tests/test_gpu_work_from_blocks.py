"""fdl_work_from_blocks: the work list built on the GPU from the reference's block tables
(rows (batch, k_end, q0, q1) in block_m chunks, llada/generate.py:52-58, :146-163) has the
tiles of the host builder (fdl.schedule.build_work over seqs_from_reference_blocks), and the
block attention gives the same output and importance with either plan."""
import numpy as np
import pytest
import torch

from fdl import lib, ops
from fdl.schedule import (DEFAULT_PAGE_LOG2, contiguous_page_table, make_plan,
                          seqs_from_reference_blocks)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _make_blocks(j, k_end, q0, q1, bm):
    """The reference's make_blocks: rows [q0, q1) in chunks of block_m."""
    starts = np.arange(q0, q1, bm)
    ends = np.minimum(starts + bm, q1)
    return np.stack([np.full_like(starts, j), np.full_like(starts, k_end), starts, ends], axis=1)


def _tables(seq_rows, bm=32):
    """seq_rows: per sequence (k_end, masked rows, tracked rows); reference packing: masked
    rows of every sequence, then tracked rows."""
    mb, tb, acc = [], [], 0
    for j, (k, m, _) in enumerate(seq_rows):
        if m:
            mb.append(_make_blocks(j, k, acc, acc + m, bm))
            acc += m
    for j, (k, _, t) in enumerate(seq_rows):
        if t:
            tb.append(_make_blocks(j, k, acc, acc + t, bm))
            acc += t
    cat = lambda x: np.concatenate(x) if x else np.zeros((0, 4), np.int64)  # noqa: E731
    return cat(mb).astype(np.int64), cat(tb).astype(np.int64), acc


def _tiles(work, row_idx, first, count):
    out = []
    for w in work[first:first + count]:
        if w[4] == 0:
            continue
        out.append((int(w[0]), int(w[1]), int(w[2]), int(w[5]), tuple(row_idx[w[3]:w[3] + w[4]])))
    return sorted(out)


# per case: per sequence (k_end, masked rows, tracked rows), block_m
CASES = {
    "decode": ([(768, 32, 32)] * 8, 32),
    "mixed": ([(768, 32, 32), (512, 32, 64), (1024, 32, 0), (640, 0, 48), (900, 32, 600),
               (1500, 32, 1468), (384, 32, 8), (256, 0, 256)], 32),
    "full_recompute": ([(1024, 32, 992)] * 4, 32),
    # the reference's evaluation preset (batch 32, block 16; llada/eval_gsm8k.sh:7-15): at
    # step 0 every slot is tracked (generate.py:129-134): 32 x 88 = 2816 table entries,
    # passing through the builder's LDS in three chunks
    "eval_preset_step0": ([(1408, 16, 1392)] * 32, 16),
    "eval_preset_steady": ([(1408, 16, 16 + 16 * (j % 3)) for j in range(32)], 16),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_device_work_list_matches_host_builder(case):
    rows, bm = CASES[case]
    B, L = len(rows), 1536
    mb, tb, Q = _tables(rows, bm)
    print(f"{case}: {len(mb) + len(tb)} table entries, {Q} rows", flush=True)
    table = contiguous_page_table(B, L)
    table_d = torch.from_numpy(table).to(DEV)
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    dplan = ops.work_from_blocks(torch.from_numpy(mb).to(DEV), torch.from_numpy(tb).to(DEV), B, Q,
                                 table, table_d, DEFAULT_PAGE_LOG2, status=status)
    hplan = make_plan(seqs_from_reference_blocks(mb, tb, importance=True), table, device=DEV)
    torch.cuda.synchronize()
    st = status.cpu().numpy()
    assert st[3] == 0, st
    assert (st[0], st[1], st[2]) == (hplan.n_long, hplan.n_mid, hplan.n_work - hplan.n_long - hplan.n_mid)
    wd, rd = dplan.work_d.cpu().numpy(), dplan.row_idx_d.cpu().numpy()
    regions = [(0, dplan.n_long, 0, hplan.n_long), (dplan.n_long, dplan.n_mid, hplan.n_long, hplan.n_mid),
               (dplan.n_long + dplan.n_mid, dplan.n_work - dplan.n_long - dplan.n_mid,
                hplan.n_long + hplan.n_mid, hplan.n_work - hplan.n_long - hplan.n_mid)]
    for df, dc, hf, hc in regions:
        assert _tiles(wd, rd, df, dc) == _tiles(hplan.work, hplan.row_idx, hf, hc)
        # the items past the built ones are empty
        assert not wd[df + len(_tiles(wd, rd, df, dc)):df + dc].any()

    # same attention output and raw importance with either plan
    H, D = 4, 512
    gen = torch.Generator().manual_seed(len(case))
    kc = torch.randn((B * L, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((B * L, D), generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.randn((Q, D), generator=gen).to(torch.bfloat16).to(DEV)
    outs = []
    for plan in (hplan, dplan):
        out = torch.zeros_like(q)
        imp = torch.zeros((H, B * L), dtype=torch.float32, device=DEV)
        ops.block_attention(q, kc, vc, plan, out, H, 0.088, lib.IMP_RAW_LOGIT, imp)
        scores = torch.zeros(B * L, dtype=torch.float32, device=DEV)
        ops.importance_accumulate(imp, plan, 0.5, scores)
        outs.append((out, scores))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


def test_device_work_list_flags_out_of_range_entries():
    mb, tb, Q = _tables([(768, 32, 32)] * 2)
    mb[0, 3] = Q + 5  # q1 beyond the rows
    table = contiguous_page_table(2, 1024)
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    ops.work_from_blocks(torch.from_numpy(mb).to(DEV), torch.from_numpy(tb).to(DEV), 2, Q, table,
                         torch.from_numpy(table).to(DEV), DEFAULT_PAGE_LOG2, status=status)
    assert int(status[3].item()) & 1
