"""Host-side schedule building for the block-table attention.

The reference launches masked-block attention and tracked-block attention separately
(flash_cache_triton.py:561-607), so every sequence's K/V are streamed twice. Here a
sequence's masked rows and tracked rows are packed into the same tiles (64, 128 or 256
query rows per tile): masked rows first, so that the first `n_imp` rows of the sequence's first
tile are the rows whose logits feed the importance scores (flash_cache_triton.py:155-158,
:614-615).

Work items (int32 x 8, see include/fdl.h):
    (batch, k_begin, k_end, row_off, n_rows, n_imp, 0, 0)
Tiles are issued longest-first (keys x row groups), so that the long full-recompute tiles
start before the short ones.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

MAX_TILE_ROWS = 64        # rows per tile of the short-row variant
MID_TILE_ROWS = 128       # rows per tile of the mid-row variant (65..128 rows)
LONG_TILE_ROWS = 256      # rows per tile of the long-row (full recompute) variant
DEFAULT_PAGE_LOG2 = 5  # 32-slot pages


@dataclass
class SeqRows:
    """The query rows of one sequence in one attention launch."""
    batch: int           # page-table row
    k_end: int           # keys [k_begin, k_end)
    rows: np.ndarray     # packed query-row indices, importance rows first
    n_imp: int = 0       # leading rows that feed the importance scores
    k_begin: int = 0


def contiguous_page_table(n_seq: int, max_length: int, page_log2: int = DEFAULT_PAGE_LOG2) -> np.ndarray:
    """The reference layout (slot = b * L + n, llada/generate.py:178-180) as a page table."""
    page = 1 << page_log2
    if max_length % page:
        raise ValueError(f"max_length {max_length} is not a multiple of the page size {page}")
    per = max_length // page
    return (np.arange(n_seq, dtype=np.int64)[:, None] * per + np.arange(per)[None, :]).astype(np.int32)


def page_slots(pages: np.ndarray, n: int, page_log2: int = DEFAULT_PAGE_LOG2) -> np.ndarray:
    """Slots of logical positions 0 .. n-1 of a sequence whose page-table row is `pages`."""
    p = np.arange(n, dtype=np.int64)
    return (np.asarray(pages, dtype=np.int64)[p >> page_log2] << page_log2) | (p & ((1 << page_log2) - 1))


class PagePool:
    """Fixed pool of K/V cache pages (2^page_log2 slots each) shared by the sequences of a
    decode. The reference gives every sequence a fixed stride of max_length slots
    (llada/generate.py:76-79, :178-180) and refills a finished sequence's row in place
    (:405-427); here a sequence holds only the pages its own length needs, returns them when
    it finishes, and a new sequence is admitted when enough pages are free.

    alloc() hands out the lowest free page ids in ascending order, and a sequence that grows
    asks for ids above its last page first, so within a sequence the slot order normally
    follows the logical position order (the importance ranking breaks score ties by slot;
    with ascending pages it breaks them as the contiguous layout does)."""

    def __init__(self, n_pages: int, page_log2: int = DEFAULT_PAGE_LOG2):
        if n_pages < 1:
            raise ValueError(f"a page pool needs at least one page (got {n_pages})")
        self.n_pages = int(n_pages)
        self.page_log2 = page_log2
        self._free = np.ones(self.n_pages, dtype=bool)

    @property
    def page_size(self) -> int:
        return 1 << self.page_log2

    @property
    def n_slots(self) -> int:
        return self.n_pages << self.page_log2

    @property
    def n_free(self) -> int:
        return int(self._free.sum())

    def pages_for(self, n_positions: int) -> int:
        return -(-int(n_positions) // self.page_size)

    def alloc(self, n: int, above: int = -1) -> np.ndarray:
        """n free pages (int32, ascending); the lowest free ids above `above` first, then the
        lowest below it. Raises MemoryError if fewer than n are free."""
        free = np.flatnonzero(self._free)
        if n > free.size:
            raise MemoryError(f"page pool: {n} pages requested, {free.size} of {self.n_pages} free")
        free = np.concatenate([free[free > above], free[free <= above]])
        got = free[:n]
        self._free[got] = False
        return got.astype(np.int32)

    def free(self, pages: np.ndarray) -> None:
        pages = np.asarray(pages, dtype=np.int64)
        if pages.size and (self._free[pages].any() or len(np.unique(pages)) != pages.size):
            raise ValueError("page pool: freeing a page that is not allocated")
        self._free[pages] = True


class PagedRows:
    """The rows of a decode batch over a PagePool: row j's page-table row (pages for its
    logical positions 0 .. 2^page_log2 * n_j - 1), the pages promised to it at admission
    beyond the ones it holds, and the pool slot -> logical slot (j * L + p) table. Shared by
    the host-scheduled and the device-scheduled decode loops (fdl.generate,
    fdl.device_decode), so both admit and grow rows identically."""

    def __init__(self, pool: PagePool, n_rows: int, max_length: int):
        self.pool = pool
        self.L = max_length
        self.PL = pool.page_log2
        self.page_table = np.zeros((n_rows, max_length >> self.PL), dtype=np.int32)
        self.logical_of = np.full(pool.n_slots, -1, dtype=np.int64)
        self.pages = [np.zeros(0, np.int32) for _ in range(n_rows)]
        self.reserved = [0] * n_rows
        self.version = 0  # changes with every page handed out or returned

    def fits(self, n_pages: int) -> bool:
        """A reservation of n_pages fits beside the ones promised to the other rows."""
        return self.pool.n_free - sum(self.reserved) >= n_pages

    def admit(self, j: int, reserve: int, n_positions: int) -> None:
        """Row j starts a sequence: `reserve` pages promised, n_positions covered now."""
        self.page_table[j] = 0
        self.reserved[j] = reserve
        self.grow(j, n_positions)

    def grow(self, j: int, n_positions: int) -> None:
        """Gives row j pages for logical positions 0 .. n_positions - 1: from its reservation
        first, ids above its last page first (slot order then follows position order)."""
        have = self.pages[j].size
        need = self.pool.pages_for(n_positions)
        if need <= have:
            return
        extra = self.pool.alloc(need - have, above=int(self.pages[j].max()) if have else -1)
        self.reserved[j] = max(0, self.reserved[j] - extra.size)
        self.page_table[j, have:need] = extra
        self.pages[j] = np.concatenate([self.pages[j], extra])
        self.logical_of[page_slots(extra, extra.size << self.PL, self.PL)] = \
            j * self.L + (have << self.PL) + np.arange(extra.size << self.PL)
        self.version += 1

    def release(self, j: int) -> None:
        """Row j's sequence finished: its pages return to the pool."""
        self.reserved[j] = 0
        if self.pages[j].size:
            self.logical_of[page_slots(self.pages[j], self.pages[j].size << self.PL, self.PL)] = -1
            self.pool.free(self.pages[j])
            self.pages[j] = np.zeros(0, np.int32)
            self.version += 1

    def phys(self, a: np.ndarray) -> np.ndarray:
        """Pool slots of logical slots j * L + p."""
        j, p = np.divmod(a, self.L)
        return (self.page_table[j, p >> self.PL].astype(np.int64) << self.PL) | \
            (p & ((1 << self.PL) - 1))


def pages_reserved(pool: PagePool, max_length: int, seqlen_k: int, prompt_len: int,
                   gen_length: int, block_m: int) -> int:
    """Pages a sequence is promised at admission: its seqlen_k keys, or up to
    prompt + gen + block_m - 1 positions (how far a masked block reaches while no token past
    prompt + gen is accepted ahead of earlier ones), within the row of max_length slots."""
    span = max(seqlen_k, prompt_len + gen_length + block_m - 1)
    return pool.pages_for(min(max_length, span))


def build_work(seqs: list[SeqRows], max_rows: int = MAX_TILE_ROWS, mid_rows: int = MID_TILE_ROWS,
               long_rows: int = LONG_TILE_ROWS) -> tuple[np.ndarray, np.ndarray, int, int]:
    """Splits each sequence's rows into tiles of three classes.

    Up to `max_rows` rows: one short tile. Up to `mid_rows`: one mid tile. More (full
    recomputes): tiles of `long_rows` rows, the last one with the remainder (a long tile
    costs the same whatever its row count, but the classes are separate launches, and a
    remainder in another class would run after the long tiles instead of among them).
    Returns (work int32 [n, 8], row_idx int32, n_long, n_mid): the first n_long work items
    are long tiles, the next n_mid mid tiles, the rest short tiles. Within each class
    tiles are ordered longest first. The importance rows of a sequence must fit in its
    first tile.
    """
    items = [[], [], []]
    row_chunks = []
    off = 0
    limits = (long_rows, mid_rows, max_rows)

    def cls_of(n: int) -> int:
        return 2 if n <= max_rows else (1 if n <= mid_rows else 0)

    for sq in seqs:
        rows = np.asarray(sq.rows, dtype=np.int32).reshape(-1)
        if sq.n_imp > len(rows):
            raise ValueError("n_imp exceeds the number of rows")
        t0 = 0
        cls = cls_of(len(rows))
        while t0 < len(rows):
            chunk = rows[t0:t0 + limits[cls]]
            n_imp = sq.n_imp if t0 == 0 else 0
            if n_imp > len(chunk):
                raise ValueError(f"{sq.n_imp} importance rows do not fit one {len(chunk)}-row tile")
            items[cls].append((sq.batch, sq.k_begin, sq.k_end, off, len(chunk), n_imp, 0, 0))
            row_chunks.append(chunk)
            off += len(chunk)
            t0 += len(chunk)
    if not row_chunks:
        return np.zeros((0, 8), dtype=np.int32), np.zeros(0, dtype=np.int32), 0, 0
    row_idx = np.concatenate(row_chunks).astype(np.int32)
    parts = []
    for cls, it in enumerate(items):
        w = np.asarray(it, dtype=np.int32).reshape(-1, 8)
        # longest first: keys x 16-row groups (long tiles: keys; every row group is computed)
        groups = 1 if cls == 0 else (w[:, 4].astype(np.int64) + 15) // 16
        cost = (w[:, 2].astype(np.int64) - w[:, 1]) * groups
        parts.append(w[np.argsort(-cost, kind="stable")])
    return np.ascontiguousarray(np.concatenate(parts)), row_idx, len(items[0]), len(items[1])


def seqs_from_reference_blocks(masked_blocks: np.ndarray, tracked_blocks: np.ndarray,
                               importance: bool) -> list[SeqRows]:
    """Groups the reference's block tables (rows (batch, k_end, q0, q1),
    llada/generate.py:52-58, :146-163, :439-465) by sequence: masked rows first, then
    tracked rows. With `importance`, the masked rows are the importance rows."""
    masked_blocks = np.asarray(masked_blocks, dtype=np.int64).reshape(-1, 4)
    tracked_blocks = np.asarray(tracked_blocks, dtype=np.int64).reshape(-1, 4)
    by_key: dict[tuple[int, int], list[list[np.ndarray]]] = {}
    order: list[tuple[int, int]] = []
    for kind, table in ((0, masked_blocks), (1, tracked_blocks)):
        for b, k_end, q0, q1 in table:
            key = (int(b), int(k_end))
            if key not in by_key:
                by_key[key] = [[], []]
                order.append(key)
            by_key[key][kind].append(np.arange(q0, q1, dtype=np.int32))
    seqs = []
    for key in order:
        m, t = by_key[key]
        m_rows = np.concatenate(m) if m else np.zeros(0, np.int32)
        t_rows = np.concatenate(t) if t else np.zeros(0, np.int32)
        seqs.append(SeqRows(batch=key[0], k_end=key[1], rows=np.concatenate([m_rows, t_rows]),
                            n_imp=len(m_rows) if importance else 0))
    return seqs


@dataclass
class AttnPlan:
    """A ready-to-launch attention schedule: host tables and their device copies."""
    work: np.ndarray
    row_idx: np.ndarray
    page_table: np.ndarray
    page_log2: int
    n_long: int = 0  # leading work items that are long (256-row) tiles
    n_mid: int = 0   # the next work items, mid (128-row) tiles
    # K/V cache slots of the packed query rows when they differ from the query positions
    # (a paged pool: the positions index the RoPE table, these slots the cache); device int64
    kv_slot: torch.Tensor = field(repr=False, default=None)
    # The caller ranks after the forward with fdl_importance_accumulate_rank: the last layer
    # leaves its per-head importance in deferred_importance = (imp_part, scale) instead of
    # reducing it into attn_scores.
    defer_last_importance: bool = False
    deferred_importance: tuple = field(repr=False, default=None)
    work_d: torch.Tensor = field(repr=False, default=None)
    row_idx_d: torch.Tensor = field(repr=False, default=None)
    page_table_d: torch.Tensor = field(repr=False, default=None)

    @property
    def n_work(self) -> int:
        return int(self.work.shape[0])

    @property
    def has_importance(self) -> bool:
        return bool(self.n_work and (self.work[:, 5] > 0).any())

    def to(self, device) -> "AttnPlan":
        """Copies the tables to `device` (one packed host->device copy)."""
        parts = [self.work.reshape(-1), self.row_idx.reshape(-1), self.page_table.reshape(-1)]
        flat = torch.from_numpy(np.concatenate(parts).astype(np.int32))
        if torch.device(device).type == "cuda":
            flat = flat.pin_memory()
        flat = flat.to(device, non_blocking=True)
        a = parts[0].size
        b = a + parts[1].size
        self.work_d = flat[:a].view(-1, 8)
        self.row_idx_d = flat[a:b]
        self.page_table_d = flat[b:].view(self.page_table.shape)
        return self

    def validate(self, n_q_rows: int, n_slots: int) -> None:
        """Runs the C-ABI host validator on the host tables (raises FdlError)."""
        from . import lib as _lib
        w = np.ascontiguousarray(self.work, dtype=np.int32)
        r = np.ascontiguousarray(self.row_idx, dtype=np.int32)
        if r.size == 0:
            r = np.zeros(1, np.int32)
        p = np.ascontiguousarray(self.page_table, dtype=np.int32)
        _lib.call("fdl_validate_work", w.ctypes.data, w.shape[0], r.ctypes.data, self.row_idx.size,
                  n_q_rows, p.ctypes.data, p.shape[0], p.shape[1], self.page_log2, n_slots)


class DeviceAttnPlan(AttnPlan):
    """An attention plan whose work items and row list were built on the device
    (fdl_sched_pack or fdl_work_from_blocks): the host knows only the class regions of the
    work array (their items past the built ones are empty) and the number of rows."""

    def __init__(self, work_d, row_idx_d, n_rows: int, page_table: np.ndarray, page_table_d,
                 page_log2: int, n_long: int, n_mid: int, n_work: int, importance: bool):
        super().__init__(work=np.zeros((0, 8), np.int32), row_idx=np.zeros(max(n_rows, 1), np.int32),
                         page_table=page_table, page_log2=page_log2, n_long=n_long, n_mid=n_mid)
        self._n_work = n_work
        self._importance = importance
        self.work_d = work_d
        self.row_idx_d = row_idx_d
        self.page_table_d = page_table_d

    @property
    def has_importance(self) -> bool:
        return self._importance

    @property
    def n_work(self) -> int:
        return self._n_work


def make_plan(seqs: list[SeqRows], page_table: np.ndarray, page_log2: int = DEFAULT_PAGE_LOG2,
              device=None, max_rows: int = MAX_TILE_ROWS) -> AttnPlan:
    work, row_idx, n_long, n_mid = build_work(seqs, max_rows)
    # the plan owns a copy: a caller may edit its table (a paged pool's refill) afterwards
    plan = AttnPlan(work=work, row_idx=row_idx, page_table=np.array(page_table, dtype=np.int32),
                    page_log2=page_log2, n_long=n_long, n_mid=n_mid)
    if device is not None:
        plan.to(device)
    return plan
