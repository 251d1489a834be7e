// Host-only part of the C ABI: error reporting, version and the table validators.
// Nothing here touches the GPU, so it runs (and is tested) on machines without one.
#include "fdl_host.h"

#include <stdarg.h>
#include <stdio.h>

#include <vector>

namespace fdl {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return FDL_OK;
}

}  // namespace fdl

extern "C" const char* fdl_last_error(void) { return fdl::g_last_error; }

extern "C" int fdl_abi_version(void) { return FDL_ABI_VERSION; }

extern "C" int fdl_validate_rows(const int64_t* slot, const int64_t* rope_row, int64_t n_rows,
                                 int64_t n_kv_rows, int64_t n_rope_rows, int32_t kv_packed) {
  FDL_REQUIRE(n_rows >= 0, FDL_ERR_SHAPE, "fdl_validate_rows: n_rows = %lld < 0",
              (long long)n_rows);
  FDL_REQUIRE(n_kv_rows >= 0 && n_rope_rows >= 0, FDL_ERR_SHAPE,
              "fdl_validate_rows: n_kv_rows = %lld, n_rope_rows = %lld (negative)",
              (long long)n_kv_rows, (long long)n_rope_rows);
  if (n_rows == 0) return fdl::ok();
  FDL_REQUIRE_PTR(slot);
  if (kv_packed) {
    FDL_REQUIRE(n_kv_rows == n_rows, FDL_ERR_SHAPE,
                "fdl_validate_rows: packed K/V needs n_kv_rows (%lld) == n_rows (%lld)",
                (long long)n_kv_rows, (long long)n_rows);
  }
  // one byte per cache row for the duplicate check (no exception may leave the C ABI)
  std::vector<uint8_t> seen;
  try {
    seen.assign(kv_packed ? 0 : static_cast<size_t>(n_kv_rows), 0);
  } catch (...) {
    return fdl::fail(FDL_ERR_SHAPE, "fdl_validate_rows: n_kv_rows = %lld is too large to check",
                     (long long)n_kv_rows);
  }
  for (int64_t r = 0; r < n_rows; ++r) {
    const int64_t s = slot[r];
    const int64_t rr = rope_row ? rope_row[r] : s;
    FDL_REQUIRE(rr >= 0 && rr < n_rope_rows, FDL_ERR_RANGE,
                "fdl_validate_rows: row %lld has rope row %lld outside [0, %lld)",
                (long long)r, (long long)rr, (long long)n_rope_rows);
    if (kv_packed) continue;
    FDL_REQUIRE(s >= 0 && s < n_kv_rows, FDL_ERR_RANGE,
                "fdl_validate_rows: row %lld has slot %lld outside [0, %lld)", (long long)r,
                (long long)s, (long long)n_kv_rows);
    FDL_REQUIRE(!seen[s], FDL_ERR_RANGE,
                "fdl_validate_rows: slot %lld is written by more than one row (row %lld)",
                (long long)s, (long long)r);
    seen[s] = 1;
  }
  return fdl::ok();
}

extern "C" int fdl_validate_work(const int32_t* work, int64_t n_work, const int32_t* row_idx,
                                 int64_t n_row_idx, int64_t n_q_rows,
                                 const int32_t* page_table, int64_t n_seq, int64_t max_pages,
                                 int32_t page_log2, int64_t n_slots) {
  FDL_REQUIRE(n_work >= 0, FDL_ERR_SHAPE, "fdl_validate_work: n_work < 0");
  if (n_work == 0) return fdl::ok();
  FDL_REQUIRE_PTR(work);
  FDL_REQUIRE_PTR(row_idx);
  FDL_REQUIRE_PTR(page_table);
  FDL_REQUIRE(page_log2 >= 4 && page_log2 <= 12, FDL_ERR_SHAPE,
              "fdl_validate_work: page_log2 = %d outside [4, 12]", page_log2);
  const int64_t page = int64_t(1) << page_log2;
  std::vector<int32_t> imp_tiles;  // importance tiles per sequence
  try {
    imp_tiles.assign(static_cast<size_t>(n_seq > 0 ? n_seq : 0), 0);
  } catch (...) {
    return fdl::fail(FDL_ERR_SHAPE, "fdl_validate_work: n_seq = %lld is too large to check",
                     (long long)n_seq);
  }
  for (int64_t w = 0; w < n_work; ++w) {
    const int32_t* it = work + 8 * w;
    const int32_t b = it[0], kb = it[1], ke = it[2], roff = it[3], nr = it[4], ni = it[5];
    FDL_REQUIRE(b >= 0 && b < n_seq, FDL_ERR_RANGE,
                "fdl_validate_work: work %lld names sequence %d outside [0, %lld)",
                (long long)w, b, (long long)n_seq);
    FDL_REQUIRE(kb >= 0 && kb <= ke && ke <= max_pages * page, FDL_ERR_RANGE,
                "fdl_validate_work: work %lld key range [%d, %d) outside [0, %lld)",
                (long long)w, kb, ke, (long long)(max_pages * page));
    FDL_REQUIRE(nr >= 1 && nr <= 256, FDL_ERR_RANGE,
                "fdl_validate_work: work %lld has %d rows (1..256 allowed)", (long long)w, nr);
    FDL_REQUIRE(ni >= 0 && ni <= nr, FDL_ERR_RANGE,
                "fdl_validate_work: work %lld has n_imp %d outside [0, %d]", (long long)w, ni,
                nr);
    FDL_REQUIRE(roff >= 0 && int64_t(roff) + nr <= n_row_idx, FDL_ERR_RANGE,
                "fdl_validate_work: work %lld rows [%d, %d) outside row_idx[0, %lld)",
                (long long)w, roff, roff + nr, (long long)n_row_idx);
    for (int32_t r = 0; r < nr; ++r) {
      const int32_t q = row_idx[roff + r];
      FDL_REQUIRE(q >= 0 && q < n_q_rows, FDL_ERR_RANGE,
                  "fdl_validate_work: work %lld row %d is query row %d outside [0, %lld)",
                  (long long)w, r, q, (long long)n_q_rows);
    }
    if (ni > 0) {
      FDL_REQUIRE(++imp_tiles[b] == 1, FDL_ERR_RANGE,
                  "fdl_validate_work: sequence %d has more than one importance tile", b);
    }
    if (ke > kb) {
      const int64_t p_lo = kb >> page_log2, p_hi = (int64_t(ke) - 1) >> page_log2;
      for (int64_t p = p_lo; p <= p_hi; ++p) {
        const int64_t phys = page_table[int64_t(b) * max_pages + p];
        FDL_REQUIRE(phys >= 0 && (phys + 1) * page <= n_slots, FDL_ERR_RANGE,
                    "fdl_validate_work: sequence %d page %lld maps to page %lld, outside "
                    "the %lld-slot cache",
                    b, (long long)p, (long long)phys, (long long)n_slots);
      }
    }
  }
  return fdl::ok();
}

extern "C" int fdl_validate_vblocks(const int32_t* vblocks, int64_t n_vblocks,
                                    const int64_t* key_slots, int64_t n_keys, int64_t n_q_rows,
                                    int64_t n_slots, int32_t block_rows) {
  FDL_REQUIRE(n_vblocks >= 0, FDL_ERR_SHAPE, "fdl_validate_vblocks: n_vblocks < 0");
  FDL_REQUIRE(block_rows >= 1 && block_rows <= 256, FDL_ERR_SHAPE,
              "fdl_validate_vblocks: block_rows = %d outside [1, 256]", block_rows);
  if (n_vblocks == 0) return fdl::ok();
  FDL_REQUIRE_PTR(vblocks);
  for (int64_t v = 0; v < n_vblocks; ++v) {
    const int32_t k0 = vblocks[4 * v], k1 = vblocks[4 * v + 1];
    const int32_t q0 = vblocks[4 * v + 2], q1 = vblocks[4 * v + 3];
    FDL_REQUIRE(k0 >= 0 && k0 <= k1 && k1 <= n_keys, FDL_ERR_RANGE,
                "fdl_validate_vblocks: block %lld keys [%d, %d) outside [0, %lld)",
                (long long)v, k0, k1, (long long)n_keys);
    FDL_REQUIRE(q0 >= 0 && q0 < q1 && q1 <= n_q_rows && q1 - q0 <= block_rows, FDL_ERR_RANGE,
                "fdl_validate_vblocks: block %lld rows [%d, %d) invalid (n_q_rows %lld, "
                "block_rows %d)",
                (long long)v, q0, q1, (long long)n_q_rows, block_rows);
    if (k1 > k0) FDL_REQUIRE_PTR(key_slots);
    for (int32_t n = k0; n < k1; ++n) {
      FDL_REQUIRE(key_slots[n] >= 0 && key_slots[n] < n_slots, FDL_ERR_RANGE,
                  "fdl_validate_vblocks: key %d has slot %lld outside [0, %lld)", n,
                  (long long)key_slots[n], (long long)n_slots);
    }
  }
  return fdl::ok();
}
