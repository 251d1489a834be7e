"""ctypes binding of libfdl.so, the C ABI declared in include/fdl.h.

torch is imported first so that its HIP runtime (libamdhip64.so.7) is already loaded when
libfdl.so is opened: the dynamic loader then binds libfdl.so to that same runtime, and the
streams and device pointers torch hands out are valid inside the library.

There is no fallback: if libfdl.so is missing, every entry point raises FdlError.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime libfdl.so must share)

LIB_PATH = Path(__file__).resolve().parent.parent / "libfdl.so"

# status codes (include/fdl.h)
FDL_OK = 0
FDL_ERR_NULL = -1
FDL_ERR_SHAPE = -2
FDL_ERR_RANGE = -3
FDL_ERR_UNSUPPORTED = -4
FDL_ERR_HIP = -5

ABI_VERSION = 3  # FDL_ABI_VERSION of include/fdl.h
# fdl_qkv_rope_cache flags (FDL_QKV_KV_PACKED, FDL_QKV_ROPE_HALVES_EQUAL)
QKV_KV_PACKED = 1
QKV_ROPE_HALVES_EQUAL = 2
# fp32 workspace per 64-key block, head and tile of softmax importance (FDL_ATTN_WS_FLOATS_PER_BLOCK)
ATTN_WS_FLOATS_PER_BLOCK = 32 * 64 + 32
# key blocks whose softmax-importance probabilities a tile keeps on chip (FDL_ATTN_ONCHIP_BLOCKS)
ATTN_ONCHIP_BLOCKS = 24
# key-split attention: floats per (part, row-index entry, head) and the most parts per tile
# (FDL_ATTN_PART_FLOATS, FDL_ATTN_MAX_KV_PARTS)
ATTN_PART_FLOATS = 132
ATTN_MAX_KV_PARTS = 8

IMP_NONE = 0
IMP_RAW_LOGIT = 1
IMP_SOFTMAX_COLSUM = 2

_STATUS_NAMES = {
    FDL_ERR_NULL: "FDL_ERR_NULL",
    FDL_ERR_SHAPE: "FDL_ERR_SHAPE",
    FDL_ERR_RANGE: "FDL_ERR_RANGE",
    FDL_ERR_UNSUPPORTED: "FDL_ERR_UNSUPPORTED",
    FDL_ERR_HIP: "FDL_ERR_HIP",
}


class FdlError(RuntimeError):
    """A C-ABI call returned a non-zero status (or the library is missing)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> (restype, argtypes), in declaration order of include/fdl.h
SIGNATURES: dict[str, tuple] = {
    "fdl_last_error": (ctypes.c_char_p, []),
    "fdl_abi_version": (ctypes.c_int, []),
    "fdl_qkv_rope_cache": (ctypes.c_int, [
        _p, _p, _p, _p,          # x, wq, wk, wv
        _p, _p, _i64,            # rope_sin, rope_cos, n_rope_rows
        _p, _p, _i64,            # slot, rope_row, n_rows
        _i64, _i64, _i64,        # d_model, n_heads, head_dim
        _p, _p, _p, _i64, _i32,  # q_out, k_out, v_out, n_kv_rows, flags
        _p,                      # stream
    ]),
    "fdl_block_attention": (ctypes.c_int, [
        _p, _p, _p,                   # q, k_cache, v_cache
        _i64, _i64, _i64, _i64, _i64,  # n_q_rows, n_slots, d_model, n_heads, head_dim
        _p, _i64, _i64, _i32,         # page_table, n_seq, max_pages, page_log2
        _p, _i64, _p, _i64, _i32,     # work, n_work, row_idx, n_row_idx, tile_rows
        _f32, _p, _i32, _p,           # softmax_scale, out, imp_mode, imp_part
        _p, _i64,                     # workspace, workspace_floats
        _p,                           # stream
    ]),
    "fdl_block_attention_scores_noalloc": (ctypes.c_int, [
        _p, _p, _p,                   # q, k_cache, v_cache
        _i64, _i64, _i64, _i64, _i64,  # n_q_rows, n_slots, d_model, n_heads, head_dim
        _p, _i64, _i64, _i32,         # page_table, n_seq, max_pages, page_log2
        _p, _i64, _p, _i64, _i32,     # work, n_work, row_idx, n_row_idx, tile_rows
        _f32, _p, _i32, _f32, _p,     # softmax_scale, out, imp_mode, imp_scale, scores
        _p,                           # stream
    ]),
    "fdl_importance_accumulate": (ctypes.c_int, [
        _p, _i64, _i64,               # imp_part, n_heads, n_slots
        _p, _i64, _i64, _i32,         # page_table, n_seq, max_pages, page_log2
        _p, _i64, _f32, _p,           # work, n_work, scale, scores
        _p,                           # stream
    ]),
    "fdl_importance_rank": (ctypes.c_int, [
        _p, _i64, _p, _i64,           # scores, n_scores, slots, n_slot_entries
        _p, _i64, _i32,               # seg, n_seg, max_len
        _p, _i32, _p,                 # topk_out, k, stream
    ]),
    "fdl_importance_accumulate_rank": (ctypes.c_int, [
        _p, _i64, _f32,               # imp_part, n_heads, scale
        _p, _i64, _i64, _i32, _p,     # page_table, n_seq, max_pages, page_log2, seg_keys
        _p, _i64, _p, _i64,           # scores, n_scores, slots, n_slot_entries
        _p, _i64, _i32,               # seg, n_seg, max_len
        _p, _i32, _p,                 # topk_out, k, stream
    ]),
    "fdl_verify_attention": (ctypes.c_int, [
        _p, _p, _p, _p, _p,           # q, k_blk, v_blk, k_cache, v_cache
        _i64, _i64, _i64, _i64, _i64,  # n_q_rows, n_slots, d_model, n_heads, head_dim
        _p, _i64, _p, _i64,           # key_slots, n_keys, vblocks, n_vblocks
        _p, _p, _i32, _f32, _p, _p,   # mask, vmeta, block_rows, softmax_scale, out, stream
    ]),
    "fdl_rms_norm": (ctypes.c_int, [
        _p, _p, _p,                   # x, residual, weight
        _i64, _i64, _f32,             # n_rows, d, eps
        _p, _p, _p,                   # sum_out, out, stream
    ]),
    "fdl_silu_mul": (ctypes.c_int, [_p, _p, _i64, _p, _p]),  # gate, up, n, out, stream
    # gate, up, n_rows, width, ld, out, stream
    "fdl_silu_mul_rows": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "fdl_split_reduce_residual": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p]),
    # logits, n_rows, vocab, token, prob, arg, stream
    "fdl_softmax_confidence": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _p, _p]),
    # state, conf, tok, stream / state, prob, stream / state, stream
    "fdl_sched_pass1": (ctypes.c_int, [_p, _p, _p, _p]),
    "fdl_sched_verify_accept": (ctypes.c_int, [_p, _p, _p]),
    "fdl_sched_pack": (ctypes.c_int, [_p, _p]),
    "fdl_work_from_blocks": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64,
                                            _i64, _i64, _p, _p, _p]),
    "fdl_validate_rows": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i32]),
    "fdl_validate_work": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i32, _i64]),
    "fdl_validate_vblocks": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _i64, _i32]),
}

# fdl_sched (include/fdl.h): device pointers, sizes and parameters of the device scheduler
SCHED_SEQ_FIELDS = 16
SEQ_ACTIVE, SEQ_ND, SEQ_SEQLEN_K, SEQ_PRED, SEQ_EOS, SEQ_N_MASKED, SEQ_KEEP, SEQ_T, SEQ_S, \
    SEQ_DONE, SEQ_N_TRACKED, SEQ_T0, SEQ_T1, SEQ_FRESH, SEQ_ERR, SEQ_HI = range(16)
SCHED_SUMMARY_FIELDS = 16
SUM_Q, SUM_N_MASKED_ROWS, SUM_N_LONG, SUM_N_MID, SUM_N_SHORT, SUM_N_CONT, SUM_N_DONE, \
    SUM_OVERFLOW, SUM_DECODED, SUM_VERIFY_ACCEPTED = range(10)


class SchedState(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("x", "x_draft", "full_pos", "seq", "summary", "qpos", "xq",
                                  "row_idx", "work", "seg", "vpos", "xv", "key_pos", "vblocks",
                                  "vmeta", "draft_tok")] + \
        [(n, _i64) for n in ("n_seq", "max_length", "q_cap", "work_cap")] + \
        [(n, _i32) for n in ("block_m", "track_num", "mask_num", "verify")] + \
        [("eos_id", _i64), ("threshold", ctypes.c_double), ("gamma", ctypes.c_double)]


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Opens libfdl.so once; raises FdlError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("FDL_LIBRARY", LIB_PATH))
    if not path.exists():
        raise FdlError(FDL_ERR_UNSUPPORTED,
                       f"{path} not found: build it with `python flash-dllm_amd/build.py` "
                       "(there is no non-HIP fallback)")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.fdl_abi_version() != ABI_VERSION:
        raise FdlError(FDL_ERR_UNSUPPORTED,
                       f"{path}: ABI version {lib.fdl_abi_version()} != {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Calls entry point `name`; raises FdlError with the library's message on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != FDL_OK:
        msg = lib.fdl_last_error().decode(errors="replace")
        raise FdlError(status, msg or name)
