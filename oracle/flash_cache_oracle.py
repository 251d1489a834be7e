"""CPU restatement of the Flash-Cache hot path of Flash-dLLM, in numpy.

TEST INFRASTRUCTURE ONLY. This module is the oracle that the HIP kernels are checked
against. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only to check results or as the timed CPU baseline; the product path (the
flash-dllm_amd package) never imports or calls it.

Each function restates one piece of the reference and cites the file:line it follows
(paths relative to the reference repository root). Arithmetic is float32 with float32
accumulation unless stated; inputs that the GPU path holds in bf16 are passed in as the
float32 values of those bf16 numbers.

Layouts follow the reference:
  * hidden / Q / K / V rows are [rows, d_model]; head h is columns h*hd .. h*hd+hd-1;
  * the KV cache is [B * L, d_model]; logical key n of sequence b is cache row b*L + n;
  * block tables are rows (batch, k_end, q_start, q_end) (llada/generate.py:52-58);
  * verify block tables are rows (k0, k1, q0, q1) (llada/generate.py:284-292).

How each function is pinned (tests/test_oracle_*.py):
  rope_tables          closed form in float64; position-0 identity          (pinned)
  qkv_proj_cache       complex-rotation RoPE in float64 + float64 GEMM      (pinned)
  block_attention      torch scaled_dot_product_attention; one-key/equal-key
                       closed forms                                          (pinned)
  importance_raw_S     (sum_r q_r) . k_n closed form per head                (pinned)
  importance_accumulate  S.mean((0, 1)) of that closed form, same test       (pinned)
  importance_softmax   explicit softmax-matrix column sums                   (pinned)
  importance_f64       raw: exact rational sum (math.fsum of every product);
                       softmax: torch float64 softmax column sums            (pinned)
  verify_attention     torch SDPA with a boolean mask over gathered keys     (pinned)
  verify_mask          hand-worked matrices for (T, S) = (2, 3), (0, 2)      (pinned)
  rank_ascending/topk  brute force with Python sorted() on (score, slot)     (pinned)
  make_blocks          hand-worked tables                                    (pinned)
  key_slots            paged == contiguous attention over the same keys      (pinned)
  max_length_for, seqlen_k_for, softmax_scale
                       hand-worked values of the reference's formulas        (pinned)
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


# --------------------------------------------------------------------------------------
# RoPE tables and the fused projection
# --------------------------------------------------------------------------------------

def rope_tables(seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """sin, cos float32 [seq_len, head_dim] (llada/generate.py:44-50).

    The reference's float32 steps, each correctly rounded (what an exact float32 libm
    gives; the reference's own values depend on its device's pow/sin):
      e = fl(arange(0, hd, 2) / hd); inv_freq = fl(1 / fl(theta ** e));
      freqs = fl(p * inv_freq); table = cat(freqs, freqs) -> fl(sin), fl(cos).
    Every step is evaluated in float64 and rounded to float32 once.
    """
    e = np.arange(0, head_dim, 2, dtype=F32) / F32(head_dim)
    pw = (np.float64(theta) ** e.astype(np.float64)).astype(F32)
    inv_freq = (1.0 / pw.astype(np.float64)).astype(F32)
    seq = np.arange(seq_len, dtype=np.float64)
    freqs = (seq[:, None] * inv_freq.astype(np.float64)[None, :]).astype(F32)
    pos = np.concatenate([freqs, freqs], axis=-1).astype(np.float64)
    return np.sin(pos).astype(F32), np.cos(pos).astype(F32)


def rotate_pairs(t: np.ndarray, sin_rows: np.ndarray, cos_rows: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE of one head's columns [rows, hd] (flash_cache_triton.py:90-93).

    out[:, c]      = t[:, c] * cos[:, c]           - t[:, c+half] * sin[:, c]
    out[:, c+half] = t[:, c+half] * cos[:, c+half] + t[:, c] * sin[:, c+half]
    """
    half = t.shape[1] // 2
    t1, t2 = t[:, :half], t[:, half:]
    o1 = t1 * cos_rows[:, :half] - t2 * sin_rows[:, :half]
    o2 = t2 * cos_rows[:, half:] + t1 * sin_rows[:, half:]
    return np.concatenate([o1, o2], axis=1).astype(F32)


def qkv_proj_cache(x: np.ndarray, wq: np.ndarray, wk: np.ndarray, wv: np.ndarray,
                   sin: np.ndarray, cos: np.ndarray, pos: np.ndarray, n_heads: int,
                   k_cache: np.ndarray | None, v_cache: np.ndarray | None,
                   rope_row: np.ndarray | None = None):
    """Fused QKV projection + RoPE + cache write (flash_cache_triton.py:15-100).

    x [Q, D] (x_normed), w* [D, D] ([out, in]), sin/cos [R, hd], pos [Q] cache slots.
    Returns (q [Q, D], k_cache, v_cache) as float32; the caches are copies with rows
    pos[r] overwritten by row r's rotated K and V. With k_cache None the K/V rows are
    returned packed ([Q, D]), as _flash_verify_qkv_proj_fwd does
    (flash_cache_triton.py:331-338). rope_row selects the sin/cos row (default pos).
    """
    x = x.astype(F32)
    d_model = x.shape[1]
    hd = d_model // n_heads
    rr = pos if rope_row is None else rope_row
    s_rows, c_rows = sin[rr], cos[rr]
    qt = x @ wq.astype(F32).T
    kt = x @ wk.astype(F32).T
    vt = x @ wv.astype(F32).T
    q = np.empty_like(qt)
    k = np.empty_like(kt)
    for h in range(n_heads):
        cols = slice(h * hd, (h + 1) * hd)
        q[:, cols] = rotate_pairs(qt[:, cols], s_rows, c_rows)
        k[:, cols] = rotate_pairs(kt[:, cols], s_rows, c_rows)
    if k_cache is None:
        return q, k, vt
    kc = k_cache.astype(F32).copy()
    vc = v_cache.astype(F32).copy()
    kc[pos] = k
    vc[pos] = vt
    return q, kc, vc


# --------------------------------------------------------------------------------------
# Attention and importance
# --------------------------------------------------------------------------------------

def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(axis=1, keepdims=True)


def attend(q_rows: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, n_heads: int,
           scale: float, allow: np.ndarray | None = None) -> np.ndarray:
    """softmax(scale * q k^T) v per head, float32 [rows, D].

    The formula of flash_cache_triton.py:144-177 without the tiling (the online softmax is
    an exact rewrite of this), and of modeling_llada.py:126-145. `allow` [rows, keys] masks
    keys per row.
    """
    d_model = q_rows.shape[1]
    hd = d_model // n_heads
    out = np.zeros((q_rows.shape[0], d_model), dtype=F32)
    for h in range(n_heads):
        cols = slice(h * hd, (h + 1) * hd)
        s = (q_rows[:, cols].astype(F32) @ k_rows[:, cols].astype(F32).T) * F32(scale)
        if allow is not None:
            s = np.where(allow, s, -np.inf)
        out[:, cols] = _softmax_rows(s) @ v_rows[:, cols].astype(F32)
    return out


def block_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                    blocks: np.ndarray, max_length: int, n_heads: int, scale: float,
                    out: np.ndarray | None = None, page_table: np.ndarray | None = None,
                    page_size: int = 32) -> np.ndarray:
    """Masked / tracked block attention (flash_cache_triton.py:103-177 and :180-252).

    For each block row (b, k_end, q0, q1): rows [q0, q1) attend bidirectionally to keys
    n < k_end of sequence b, at cache row b*L + n (:122, :134-135) or, with a page table,
    at page_table[b][n // P] * P + n % P. Writes into `out` (float32 [Q, D]).
    """
    if out is None:
        out = np.zeros((q.shape[0], q.shape[1]), dtype=F32)
    for b, k_end, q0, q1 in np.asarray(blocks, dtype=np.int64):
        slots = key_slots(int(b), int(k_end), max_length, page_table, page_size)
        out[q0:q1] = attend(q[q0:q1], k_cache[slots], v_cache[slots], n_heads, scale)
    return out


def key_slots(b: int, k_end: int, max_length: int, page_table: np.ndarray | None = None,
              page_size: int = 32, k_begin: int = 0) -> np.ndarray:
    """Cache rows of keys [k_begin, k_end) of sequence b."""
    n = np.arange(k_begin, k_end, dtype=np.int64)
    if page_table is None:
        return b * max_length + n
    return page_table[b][n // page_size].astype(np.int64) * page_size + n % page_size


def importance_raw_S(q: np.ndarray, k_cache: np.ndarray, masked_blocks: np.ndarray,
                     n_batch: int, max_length: int, n_heads: int, block_m: int,
                     page_table: np.ndarray | None = None, page_size: int = 32) -> np.ndarray:
    """The raw-logit capture S[r - q0, h, b, n] = q_r^h . k_n^h (flash_cache_triton.py:155-158).

    Returns S float32 [block_m, n_heads, n_batch, max_length], zero where not written,
    as allocated at flash_cache_triton.py:538.
    """
    d_model = q.shape[1]
    hd = d_model // n_heads
    S = np.zeros((block_m, n_heads, n_batch, max_length), dtype=F32)
    for b, k_end, q0, q1 in np.asarray(masked_blocks, dtype=np.int64):
        slots = key_slots(int(b), int(k_end), max_length, page_table, page_size)
        for h in range(n_heads):
            cols = slice(h * hd, (h + 1) * hd)
            S[: q1 - q0, h, b, :k_end] = q[q0:q1, cols].astype(F32) @ k_cache[slots][:, cols].astype(F32).T
    return S


def importance_accumulate(attn_scores: np.ndarray, S: np.ndarray) -> np.ndarray:
    """attn_scores += S.mean((0, 1)).view(-1) (flash_cache_triton.py:614-615)."""
    return (attn_scores.astype(F32) + S.mean(axis=(0, 1), dtype=np.float64).astype(F32).reshape(-1)).astype(F32)


def importance_softmax_colsum(q: np.ndarray, k_cache: np.ndarray, masked_blocks: np.ndarray,
                              n_batch: int, max_length: int, n_heads: int, scale: float,
                              page_table: np.ndarray | None = None, page_size: int = 32) -> np.ndarray:
    """Attention-importance as column sums of softmax(scale q k^T) over the masked rows,
    summed over heads: scores[b*L + n] = sum_h sum_r P_h[r, n] (the column-sum definition
    of the importance used for the top-k refresh set). float32 [n_batch * max_length]."""
    d_model = q.shape[1]
    hd = d_model // n_heads
    scores = np.zeros(n_batch * max_length, dtype=np.float64)
    for b, k_end, q0, q1 in np.asarray(masked_blocks, dtype=np.int64):
        slots = key_slots(int(b), int(k_end), max_length, page_table, page_size)
        for h in range(n_heads):
            cols = slice(h * hd, (h + 1) * hd)
            s = (q[q0:q1, cols].astype(F32) @ k_cache[slots][:, cols].astype(F32).T) * F32(scale)
            scores[b * max_length: b * max_length + k_end] += _softmax_rows(s).sum(axis=0)
    return scores.astype(F32)


def importance_f64(q: np.ndarray, k_cache: np.ndarray, masked_blocks: np.ndarray,
                   n_batch: int, max_length: int, n_heads: int, mode: str, scale: float,
                   block_m: int, page_table: np.ndarray | None = None,
                   page_size: int = 32) -> np.ndarray:
    """One layer's importance scores in float64, the exact values that the float32 kernels
    approximate: float64 [n_batch * max_length], zero outside the masked blocks' keys.

    mode "raw":     mean over (block_m rows, heads) of S[r, h, b, n] = q_r^h . k_n^h
                    (flash_cache_triton.py:155-158 written, :614-615 reduced; rows past q1
                    of a ragged block are zero in S and still count in the mean).
    mode "softmax": sum over heads and rows r of softmax_n(scale q_r^h . k_n^h), the
                    column-sum definition of the importance.
    """
    d_model = q.shape[1]
    hd = d_model // n_heads
    scores = np.zeros(n_batch * max_length, dtype=np.float64)
    for b, k_end, q0, q1 in np.asarray(masked_blocks, dtype=np.int64):
        slots = key_slots(int(b), int(k_end), max_length, page_table, page_size)
        acc = np.zeros(int(k_end), dtype=np.float64)
        for h in range(n_heads):
            cols = slice(h * hd, (h + 1) * hd)
            s = q[q0:q1, cols].astype(np.float64) @ k_cache[slots][:, cols].astype(np.float64).T
            if mode == "raw":
                acc += s.sum(axis=0)
            else:
                s = s * scale
                e = np.exp(s - s.max(axis=1, keepdims=True))
                acc += (e / e.sum(axis=1, keepdims=True)).sum(axis=0)
        if mode == "raw":
            acc /= block_m * n_heads
        scores[slots] += acc
    return scores


# --------------------------------------------------------------------------------------
# Flash-Verify
# --------------------------------------------------------------------------------------

def verify_mask(T: int, S: int, block_m: int) -> np.ndarray:
    """Boolean [2bm, 2bm] verify mask, literally as llada/generate.py:262-269 builds it.

    Rows/columns: T fill rows, then S draft rows, then S mask rows. True = may attend.
    """
    m = np.ones((2 * block_m, 2 * block_m), dtype=bool)
    idx = np.arange(S)
    m11 = idx[:, None] >= idx[None, :]
    m12 = idx[:, None] < idx[None, :]
    m21 = idx[:, None] > idx[None, :]
    m22 = idx[:, None] <= idx[None, :]
    m[:T, T:T + S] = False
    top = np.concatenate([m11, m12], axis=1)
    bot = np.concatenate([m21, m22], axis=1)
    m[T:T + 2 * S, T:T + 2 * S] = np.concatenate([top, bot], axis=0)
    return m


def verify_attention(q: np.ndarray, k1: np.ndarray, v1: np.ndarray, k_cache: np.ndarray,
                     v_cache: np.ndarray, key_pos: np.ndarray, mask: np.ndarray,
                     vblocks: np.ndarray, block_rows: int, n_heads: int, scale: float) -> np.ndarray:
    """Verify attention (flash_cache_triton.py:341-428).

    Block v = (k0, k1, q0, q1): rows [q0, q1) attend to cache rows key_pos[k0:k1] and to
    in-block keys j < q1 - q0 (K1/V1 rows q0 + j) where mask[v*block_rows + i, j].
    The softmax is exact over both key sets. (The reference adds the in-block terms
    without raising the running maximum, :416-423; that is the same value whenever its
    exponentials do not overflow.)
    """
    out = np.zeros((q.shape[0], q.shape[1]), dtype=F32)
    for v, (k0, kk1, q0, q1) in enumerate(np.asarray(vblocks, dtype=np.int64)):
        nr = q1 - q0
        cache = key_pos[k0:kk1].astype(np.int64)
        k_rows = np.concatenate([k_cache[cache], k1[q0:q1]], axis=0)
        v_rows = np.concatenate([v_cache[cache], v1[q0:q1]], axis=0)
        allow = np.ones((nr, len(cache) + nr), dtype=bool)
        allow[:, len(cache):] = mask[v * block_rows: v * block_rows + nr, :nr]
        out[q0:q1] = attend(q[q0:q1], k_rows, v_rows, n_heads, scale, allow)
    return out


# --------------------------------------------------------------------------------------
# Ranking / top-k
# --------------------------------------------------------------------------------------

def rank_ascending(scores: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """The decoded-slot re-ordering of llada/generate.py:365-366: slots sorted ascending by
    attn_scores[slot]; ties (undefined in the reference's unstable sort) put the higher
    slot first, so that the highest-ranked entries (the tail) prefer lower slots."""
    slots = np.asarray(slots, dtype=np.int64)
    sc = np.asarray(scores, dtype=F32)[slots]
    sc = np.where(sc == 0, F32(0), sc)  # -0.0 ties with +0.0
    order = np.lexsort((-slots, sc))
    return slots[order]


def topk(scores: np.ndarray, slots: np.ndarray, k: int) -> np.ndarray:
    """The k highest-ranked slots in rank order (score descending, slot ascending), -1
    padded: the refresh selection of llada/generate.py:375-381."""
    asc = rank_ascending(scores, slots)
    top = asc[::-1][:k]
    return np.concatenate([top, -np.ones(k - len(top), dtype=np.int64)])


# --------------------------------------------------------------------------------------
# Schedule
# --------------------------------------------------------------------------------------

def make_blocks(j: int, seqlen_k: list[int], start_m: int, end_m: int, block_m: int) -> np.ndarray:
    """Rows (batch, k_end, q_start, q_end) splitting [start_m, end_m) into block_m chunks,
    the last one ragged (llada/generate.py:52-58)."""
    rows = []
    for s in range(start_m, end_m, block_m):
        rows.append((j, seqlen_k[j], s, min(s + block_m, end_m)))
    return np.asarray(rows, dtype=np.int64).reshape(-1, 4)


def max_length_for(prompt_lengths: list[int], gen_length: int, block_m: int, block_n: int = 128) -> int:
    """Per-sequence slot stride L (llada/generate.py:76-79)."""
    return ((max(prompt_lengths) + gen_length + block_m) // block_n + 1) * block_n


def seqlen_k_for(prompt_length: int, gen_length: int, block_n: int = 128) -> int:
    """Key count k_end of a sequence (llada/generate.py:122)."""
    return (prompt_length + gen_length) // block_n * block_n + block_n


def softmax_scale(head_dim: int) -> float:
    """Default softmax scale (flash_cache_triton.py:492)."""
    return 1.0 / math.sqrt(head_dim)
