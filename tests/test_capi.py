"""C-ABI library checks that need no GPU: the library loads, exports every entry point
include/fdl.h declares, and rejects bad arguments on the host before any GPU work."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from fdl import lib
from fdl.schedule import SeqRows, build_work, contiguous_page_table

HEADER = Path(__file__).resolve().parent.parent / "include" / "fdl.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fdl_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = lib.load()
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(lib.SIGNATURES), "ctypes signatures out of sync with fdl.h"
    assert L.fdl_abi_version() == lib.ABI_VERSION


def _expect(status, name, *args):
    with pytest.raises(lib.FdlError) as ei:
        lib.call(name, *args)
    assert ei.value.status == status
    return str(ei.value)


def test_launchers_reject_bad_scalars_without_gpu():
    # null pointers, wrong head_dim, inconsistent d_model: all caught before any HIP call
    msg = _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_qkv_rope_cache", None, None, None, None, None, None,
                  10, None, None, 4, 4096, 64, 64, None, None, None, 10, 0, None)
    assert "head_dim" in msg
    _expect(lib.FDL_ERR_SHAPE, "fdl_qkv_rope_cache", None, None, None, None, None, None,
            10, None, None, 4, 4000, 32, 128, None, None, None, 10, 0, None)
    _expect(lib.FDL_ERR_NULL, "fdl_qkv_rope_cache", None, None, None, None, None, None,
            10, None, None, 4, 4096, 32, 128, None, None, None, 10, 0, None)
    _expect(lib.FDL_ERR_SHAPE, "fdl_qkv_rope_cache", None, None, None, None, None, None,
            10, None, None, 4, 4096, 32, 128, None, None, None, 7, 1, None)
    # flags: FDL_QKV_KV_PACKED (1) and FDL_QKV_ROPE_HALVES_EQUAL (2) only
    assert "flags" in _expect(lib.FDL_ERR_SHAPE, "fdl_qkv_rope_cache", None, None, None, None,
                              None, None, 10, None, None, 4, 4096, 32, 128, None, None, None,
                              4, 4, None)
    _expect(lib.FDL_ERR_NULL, "fdl_qkv_rope_cache", None, None, None, None, None, None,
            10, None, None, 4, 4096, 32, 128, None, None, None, 4, 3, None)
    # zero rows is a no-op
    lib.call("fdl_qkv_rope_cache", None, None, None, None, None, None, 0, None, None, 0,
             4096, 32, 128, None, None, None, 0, 0, None)
    _expect(lib.FDL_ERR_NULL, "fdl_block_attention", None, None, None, 4, 4, 4096, 32, 128,
            None, 1, 1, 5, None, 1, None, 1, 64, 0.1, None, 0, None, None, 0, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_block_attention", None, None, None, 4, 4, 2048, 32, 64,
            None, 1, 1, 5, None, 1, None, 1, 64, 0.1, None, 0, None, None, 0, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_block_attention", None, None, None, 4, 4, 4096, 32, 128,
            None, 1, 1, 5, None, 1, None, 1, 96, 0.1, None, 0, None, None, 0, None)
    lib.call("fdl_block_attention", None, None, None, 4, 4, 4096, 32, 128, None, 1, 1, 5, None,
             0, None, 1, 64, 0.1, None, 0, None, None, 0, None)
    _expect(lib.FDL_ERR_NULL, "fdl_importance_rank", None, 10, None, 10, None, 1, 16, None, 0, None)
    _expect(lib.FDL_ERR_NULL, "fdl_importance_accumulate_rank", None, 32, 1.0, None, 1, 4, 5,
            None, None, 10, None, 10, None, 1, 16, None, 0, None)
    assert lib.load().fdl_last_error().decode().startswith("fdl_importance_accumulate_rank")
    _expect(lib.FDL_ERR_SHAPE, "fdl_importance_accumulate_rank", None, 0, 1.0, None, 1, 4, 5,
            None, None, 10, None, 10, None, 1, 16, None, 0, None)
    _expect(lib.FDL_ERR_SHAPE, "fdl_importance_accumulate_rank", None, 32, 1.0, None, 1, 4, 17,
            None, None, 10, None, 10, None, 1, 16, None, 0, None)
    _expect(lib.FDL_ERR_NULL, "fdl_verify_attention", None, None, None, None, None, 4, 4, 4096, 32,
            128, None, 0, None, 1, None, None, 64, 0.1, None, None)
    _expect(lib.FDL_ERR_NULL, "fdl_importance_accumulate", None, 32, 10, None, 1, 1, 5, None, 1,
            1.0, None, None)
    assert lib.load().fdl_last_error().decode().startswith("fdl_importance_accumulate")
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_silu_mul_rows", None, None, 4, 12, 16, 1, None, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_silu_mul_rows", None, None, 4, 16, 8, 1, None, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_silu_mul_rows", None, None, 4, 16, 32, 4, None, None)
    _expect(lib.FDL_ERR_NULL, "fdl_silu_mul_rows", None, None, 4, 16, 32, 2, None, None)
    lib.call("fdl_silu_mul_rows", None, None, 0, 16, 32, 1, None, None)  # zero rows: no-op
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_split_reduce_residual", None, 0, 4, 16, None, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_split_reduce_residual", None, 4, 4, 12, None, None)
    _expect(lib.FDL_ERR_NULL, "fdl_split_reduce_residual", None, 4, 4, 16, None, None)
    lib.call("fdl_split_reduce_residual", None, 4, 0, 16, None, None)  # zero rows: no-op
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_softmax_confidence", None, 4, 12, None, None, None, None)
    _expect(lib.FDL_ERR_NULL, "fdl_softmax_confidence", None, 4, 16, None, None, None, None)
    lib.call("fdl_softmax_confidence", None, 0, 16, None, None, None, None)  # zero rows: no-op
    # scheduler state: NULL state, sizes out of range, missing arrays
    st = lib.SchedState()
    assert ctypes.sizeof(lib.SchedState) == 16 * 8 + 4 * 8 + 4 * 4 + 8 + 2 * 8  # fdl_sched
    _expect(lib.FDL_ERR_NULL, "fdl_sched_pass1", None, None, None, None)
    st.n_seq, st.block_m, st.max_length = 0, 32, 1024
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_sched_pass1", ctypes.byref(st), None, None, None)
    st.n_seq, st.block_m = 8, 1
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_sched_pack", ctypes.byref(st), None)
    st.block_m, st.max_length = 32, 16
    _expect(lib.FDL_ERR_SHAPE, "fdl_sched_verify_accept", ctypes.byref(st), None, None)
    st.max_length = 1024
    msg = _expect(lib.FDL_ERR_NULL, "fdl_sched_pack", ctypes.byref(st), None)
    assert "fdl_sched_pack: a state array" in msg
    for name in ("x", "x_draft", "full_pos", "seq", "summary", "seg"):
        setattr(st, name, 8)  # never dereferenced: rejected before any launch
    st.verify = 1
    assert "verify" in _expect(lib.FDL_ERR_NULL, "fdl_sched_pass1", ctypes.byref(st), None, None,
                               None)
    _expect(lib.FDL_ERR_NULL, "fdl_sched_verify_accept", ctypes.byref(st), None, None)
    for name in ("qpos", "xq", "row_idx", "work"):
        setattr(st, name, 8)
    st.q_cap = -1
    _expect(lib.FDL_ERR_SHAPE, "fdl_sched_pack", ctypes.byref(st), None)
    # device work list from block tables: too many entries, no sequences, NULL tables
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_work_from_blocks", None, 1 << 29, None, 1 << 29, 8, 64,
            1024, None, 0, 8, 8, None, None, None)
    _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_work_from_blocks", None, 1, None, 1, 0, 64, 1024, None,
            0, 8, 8, None, None, None)
    _expect(lib.FDL_ERR_NULL, "fdl_work_from_blocks", None, 1, None, 1, 8, 64, 1024, None, 0, 8,
            8, None, None, None)
    # every other entry point: an empty call returns before any pointer is read
    lib.call("fdl_importance_rank", None, 10, None, 10, None, 0, 16, None, 0, None)
    lib.call("fdl_importance_accumulate_rank", None, 32, 1.0, None, 1, 4, 5, None, None, 10,
             None, 10, None, 0, 16, None, 0, None)
    lib.call("fdl_importance_accumulate", None, 32, 10, None, 1, 1, 5, None, 0, 1.0, None, None)
    lib.call("fdl_verify_attention", None, None, None, None, None, 4, 4, 4096, 32, 128, None, 0,
             None, 0, None, None, 64, 0.1, None, None)
    lib.call("fdl_rms_norm", None, None, None, 0, 4096, 1e-5, None, None, None)
    lib.call("fdl_silu_mul", None, None, 0, None, None)


def test_elementwise_launchers_reject_bad_arguments_without_gpu():
    """RMSNorm and SiLU-gating: the width and count rules, eps, the residual / sum pairing and
    NULL or misaligned buffers are refused on the host before any launch."""
    buf = np.zeros(64, dtype=np.uint16)
    p = buf.ctypes.data
    assert p % 16 == 0
    _expect(lib.FDL_ERR_SHAPE, "fdl_rms_norm", p, None, p, -1, 16, 1e-5, None, p, None)
    for d in (0, 12, 8200):
        _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_rms_norm", p, None, p, 2, d, 1e-5, None, p, None)
    assert "eps" in _expect(lib.FDL_ERR_SHAPE, "fdl_rms_norm", p, None, p, 2, 16, -1.0, None, p,
                            None)
    for args in ((None, None, p), (p, None, None), (None, p, p)):
        x, out, w = args
        _expect(lib.FDL_ERR_NULL, "fdl_rms_norm", x, None, w, 2, 16, 1e-5, None, out, None)
    msg = _expect(lib.FDL_ERR_NULL, "fdl_rms_norm", p, p, p, 2, 16, 1e-5, None, p, None)
    assert "sum_out" in msg
    msg = _expect(lib.FDL_ERR_SHAPE, "fdl_rms_norm", p + 2, None, p, 2, 16, 1e-5, None, p, None)
    assert "aligned" in msg
    _expect(lib.FDL_ERR_SHAPE, "fdl_rms_norm", p, p + 4, p, 2, 16, 1e-5, p, p, None)
    for n in (-8, 12):
        _expect(lib.FDL_ERR_UNSUPPORTED, "fdl_silu_mul", p, p, n, p, None)
    for args in ((None, p, p), (p, None, p), (p, p, None)):
        _expect(lib.FDL_ERR_NULL, "fdl_silu_mul", args[0], args[1], 16, args[2], None)
    _expect(lib.FDL_ERR_SHAPE, "fdl_silu_mul", p, p, 16, p + 8, None)


def test_gate_up_weights_share_one_buffer():
    """LLaDABlock lays ff_proj / up_proj out as one [2h, d] buffer (values kept), so the
    block epilogue can run them as one GEMM; separate buffers are detected."""
    import torch
    import flash_cache_hip as fch
    from fdl.model import LLaDAConfig, LLaDALlamaBlock, fuse_gate_up_
    cfg = LLaDAConfig.llada_8b()
    cfg.d_model, cfg.n_heads, cfg.mlp_hidden_size = 64, 1, 96
    blk = LLaDALlamaBlock(cfg, 0, fch.flash_fused_elastic_cache)
    w = fch._adjacent_gate_up(blk)
    assert w is not None and w.shape == (192, 64)
    assert torch.equal(w[:96], blk.ff_proj.weight) and torch.equal(w[96:], blk.up_proj.weight)
    g0, u0 = blk.ff_proj.weight.detach().clone(), blk.up_proj.weight.detach().clone()
    blk.up_proj.weight = torch.nn.Parameter(u0.clone())
    assert fch._adjacent_gate_up(blk) is None
    fuse_gate_up_(blk)
    w = fch._adjacent_gate_up(blk)
    assert w is not None and torch.equal(w[:96], g0) and torch.equal(w[96:], u0)


def _arr(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a, a.ctypes.data


def test_validate_rows():
    s, sp = _arr([3, 1, 2], np.int64)
    lib.call("fdl_validate_rows", sp, None, 3, 8, 8, 0)
    msg = _expect(lib.FDL_ERR_RANGE, "fdl_validate_rows", sp, None, 3, 3, 8, 0)
    assert "slot 3" in msg
    d, dp = _arr([3, 1, 3], np.int64)
    assert "more than one row" in _expect(lib.FDL_ERR_RANGE, "fdl_validate_rows", dp, None, 3, 8, 8, 0)
    r, rp = _arr([0, 9, 1], np.int64)
    assert "rope row 9" in _expect(lib.FDL_ERR_RANGE, "fdl_validate_rows", sp, rp, 3, 8, 8, 0)
    # packed K/V: duplicate slots are fine (nothing is scattered), rope rows still checked
    lib.call("fdl_validate_rows", dp, None, 3, 3, 8, 1)
    # sizes that cannot be checked come back as errors, not as a terminated process
    assert "negative" in _expect(lib.FDL_ERR_SHAPE, "fdl_validate_rows", sp, None, 3, -1, 8, 0)
    assert "too large" in _expect(lib.FDL_ERR_SHAPE, "fdl_validate_rows", sp, None, 3,
                                  1 << 62, 8, 0)


def test_build_work_tile_classes():
    """More than 128 rows: 256-row tiles (remainder included); up to 128: one 128-row tile;
    up to 64: one 64-row tile. Importance rows stay in their sequence's first tile; every
    row is covered once."""
    seqs = [SeqRows(0, 600, np.arange(0, 600), 32), SeqRows(1, 300, np.arange(600, 900)),
            SeqRows(2, 100, np.arange(900, 1000), 8), SeqRows(3, 50, np.arange(1000, 1040))]
    work, rows, n_long, n_mid = build_work(seqs)
    assert sorted(work[:n_long, 4].tolist()) == [44, 88, 256, 256, 256]
    assert sorted(work[n_long:n_long + n_mid, 4].tolist()) == [100]
    assert sorted(work[n_long + n_mid:, 4].tolist()) == [40]
    assert sorted(rows.tolist()) == list(range(1040))
    imp = work[work[:, 5] > 0]
    assert sorted(imp[:, 5].tolist()) == [8, 32]
    for it in imp:
        first = {0: 0, 2: 900}[int(it[0])]
        assert rows[it[3]] == first
    with pytest.raises(ValueError):
        build_work([SeqRows(0, 64, np.arange(0, 10), 11)])


def test_attention_workspace_sizes():
    """Key-split workspace: a class whose tiles x heads fill at most a quarter of the
    compute units gets min(8, CUs / (tiles x heads), its largest tile's key blocks) parts of
    ATTN_PART_FLOATS per row-index entry and head if that is at least four, the 256-row
    class none; softmax-importance workspace only past
    ATTN_ONCHIP_BLOCKS key blocks. The constants match the header's."""
    from fdl import ops
    from fdl.schedule import make_plan
    hdr = (Path(__file__).resolve().parents[1] / "include" / "fdl.h").read_text()
    for name in ("ATTN_PART_FLOATS", "ATTN_MAX_KV_PARTS", "ATTN_ONCHIP_BLOCKS"):
        m = re.search(rf"#define FDL_{name} (\d+)", hdr)
        assert m and int(m.group(1)) == getattr(lib, name), name
    one = make_plan([SeqRows(0, 384, np.arange(40), 0)], contiguous_page_table(1, 384))
    # 384 keys = 6 key blocks: 6 parts, not 8 (two would be empty)
    assert ops.attention_split_floats(one, 32, 256) == 6 * 40 * 32 * lib.ATTN_PART_FLOATS
    assert ops.attention_split_floats(one, 32, 160) == 5 * 40 * 32 * lib.ATTN_PART_FLOATS
    short = make_plan([SeqRows(0, 192, np.arange(40), 0)], contiguous_page_table(1, 192))
    # 3 key blocks: 3 parts, the same bits as the 8 of a plan built on the device
    assert ops.attention_split_floats(short, 32, 256) == 3 * 40 * 32 * lib.ATTN_PART_FLOATS
    tiny = make_plan([SeqRows(0, 64, np.arange(40), 0)], contiguous_page_table(1, 64))
    assert ops.attention_split_floats(tiny, 32, 256) == 0  # one key block: one part, no split
    big = make_plan([SeqRows(0, 1024, np.arange(40), 0)], contiguous_page_table(1, 1024))
    assert ops.attention_split_floats(big, 32, 256) == 8 * 40 * 32 * lib.ATTN_PART_FLOATS
    assert ops.attention_split_floats(one, 32, 127) == 0  # 32 workgroups: over a quarter
    three = make_plan([SeqRows(b, 1024, np.arange(64 * b, 64 * b + 64), 0) for b in range(3)],
                      contiguous_page_table(3, 1024))
    assert ops.attention_split_floats(three, 16, 256) == 5 * 192 * 16 * lib.ATTN_PART_FLOATS
    assert ops.attention_split_floats(three, 32, 256) == 0  # 96 workgroups: two parts only
    full = make_plan([SeqRows(0, 600, np.arange(600), 0)], contiguous_page_table(1, 640))
    assert ops.attention_split_floats(full, 32, 256) == 0  # long tiles only
    soft = make_plan([SeqRows(0, 1536, np.arange(64), 32)], contiguous_page_table(1, 1536))
    assert ops.attention_workspace_floats(soft, 32) == 0  # 24 blocks: on chip
    soft = make_plan([SeqRows(0, 1600, np.arange(64), 32)], contiguous_page_table(1, 1600))
    assert ops.attention_workspace_floats(soft, 32) == 32 * 25 * lib.ATTN_WS_FLOATS_PER_BLOCK
    # only the 64-row class keeps probabilities in the workspace: 128-row and 256-row tiles
    # (8 full recomputes of 4096 keys, 32 heads) take a second pass over K and need none
    pt = contiguous_page_table(8, 4096)
    full = make_plan([SeqRows(b, 4096, np.arange(4096 * b, 4096 * b + 4096), 32) for b in range(8)], pt)
    assert full.n_long == 128 and ops.attention_workspace_floats(full, 32) == 0
    mid = make_plan([SeqRows(b, 4096, np.arange(100 * b, 100 * b + 100), 32) for b in range(8)], pt)
    assert mid.n_mid == 8 and ops.attention_workspace_floats(mid, 32) == 0
    # beside them, the 64-row tiles alone are counted (2 tiles x 32 heads x 30 blocks)
    mixed = make_plan([SeqRows(0, 4096, np.arange(4096), 32), SeqRows(1, 4096, np.arange(4096, 4196), 32),
                       SeqRows(2, 1920, np.arange(4196, 4260), 32), SeqRows(3, 1600, np.arange(4260, 4300), 8)],
                      pt)
    assert ops.attention_workspace_floats(mixed, 32) == 2 * 32 * 30 * lib.ATTN_WS_FLOATS_PER_BLOCK


def test_validate_work():
    pt = contiguous_page_table(2, 128)
    work, rows, n_long, n_mid = build_work([SeqRows(0, 100, np.arange(0, 40), 8),
                                            SeqRows(1, 128, np.arange(40, 150))])
    assert n_long == 0 and n_mid == 1 and work[0, 4] == 110
    w, wp = _arr(work, np.int32)
    r, rp = _arr(rows, np.int32)
    p, pp = _arr(pt, np.int32)
    lib.call("fdl_validate_work", wp, len(w), rp, len(r), 150, pp, 2, pt.shape[1], 5, 256)
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_work", wp, len(w), rp, len(r), 149, pp, 2, pt.shape[1], 5, 256)
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_work", wp, len(w), rp, len(r), 150, pp, 2, pt.shape[1], 5, 255)
    bad = w.copy()
    bad[0, 2] = 129  # k_end past the page table
    _, bp = _arr(bad, np.int32)
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_work", bp, len(w), rp, len(r), 150, pp, 2, pt.shape[1], 5, 256)
    bad = w.copy()
    bad[0, 4] = 129  # too many rows in a tile
    _, bp = _arr(bad, np.int32)
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_work", bp, len(w), rp, len(r), 150, pp, 2, pt.shape[1], 5, 256)
    _expect(lib.FDL_ERR_SHAPE, "fdl_validate_work", wp, len(w), rp, len(r), 150, pp, 2, pt.shape[1], 3, 256)


def test_validate_vblocks():
    vb, vp = _arr([[0, 3, 0, 8], [3, 5, 8, 16]], np.int32)
    ks, kp = _arr([1, 2, 3, 9, 10], np.int64)
    lib.call("fdl_validate_vblocks", vp, 2, kp, 5, 16, 11, 8)
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_vblocks", vp, 2, kp, 5, 16, 10, 8)   # slot 10
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_vblocks", vp, 2, kp, 4, 16, 11, 8)   # k1 > n_keys
    _expect(lib.FDL_ERR_RANGE, "fdl_validate_vblocks", vp, 2, kp, 5, 16, 11, 7)   # 8 rows > 7
    lib.call("fdl_validate_vblocks", vp, 2, kp, 5, 16, 11, 256)   # 2 * block_m up to 256
    _expect(lib.FDL_ERR_SHAPE, "fdl_validate_vblocks", vp, 2, kp, 5, 16, 11, 257)


def test_scheduler_record_fields_match_the_header():
    """The per-sequence and summary field indices the binding uses are the header's enums."""
    hdr = (Path(__file__).resolve().parents[1] / "include" / "fdl.h").read_text()
    fields = {m.group(1): int(m.group(2))
              for m in re.finditer(r"FDL_(SEQ_[A-Z0-9_]+|SUM_[A-Z0-9_]+) = (\d+)", hdr)}
    assert fields.pop("SEQ_HI") == lib.SEQ_HI == 15
    for name, value in fields.items():
        assert getattr(lib, name) == value, name
    assert re.search(r"FDL_SCHED_SEQ_FIELDS = (\d+)", hdr).group(1) == str(lib.SCHED_SEQ_FIELDS)


def test_projection_flags_match_the_header():
    hdr = HEADER.read_text()
    assert re.search(r"FDL_QKV_KV_PACKED = (\d+)", hdr).group(1) == str(lib.QKV_KV_PACKED)
    assert re.search(r"FDL_QKV_ROPE_HALVES_EQUAL = (\d+)", hdr).group(1) == str(
        lib.QKV_ROPE_HALVES_EQUAL)
    assert re.search(r"#define FDL_ABI_VERSION (\d+)", hdr).group(1) == str(lib.ABI_VERSION)
