// Block-table attention over the KV cache (gfx950, bf16 MFMA), with the importance side
// output, and the Flash-Verify variant.
//
// Follows _flash_masked_attention_fwd / _flash_tracked_attention_fwd
// (flash_cache_triton.py:103-252): for query row r and head h,
//   O[r, h] = softmax(scale * Q[r, h] . K[n, h]^T over keys n in [k_begin, k_end)) V[n, h]
// with the probabilities cast to bf16 before the PV product (flash_cache_triton.py:168),
// and _flash_verify_attention_fwd (flash_cache_triton.py:341-428): cache keys gathered
// through a slot list followed by the block's own rows as keys under a boolean mask.
//
// One workgroup = one tile (up to 64 query rows of one sequence) x one head; 4
// wavefronts, 16 query rows each. Keys stream through LDS 64 at a time: K row-major with
// XOR-swizzled 16-byte chunks, V transposed (V^T, padded rows). Each wavefront computes
// S^T = K Q^T with 16x16x32 MFMAs, so lane l holds the logits of query row l % 16 for
// keys 4*(l/16) + i of every 16-key block: the online-softmax row max and row sum need
// only two cross-lane steps (xor 16, xor 32), and the bf16 probabilities are already the
// B operand of O^T = V^T P^T. Importance needs column sums over query rows instead, so
// it uses S = Q K^T (the same registers with the operands swapped): the sum over rows is
// then 4 in-lane adds plus the same two cross-lane steps.
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kTileN = 64;     // keys per LDS tile
constexpr int kMaxRows = 64;   // query rows per workgroup (4 wavefronts x 16)
constexpr int kThreads = 256;
constexpr int kVtStride = 68;  // bf16 per V^T row in LDS (136 B: conflict-free column reads)

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* kblk;  // verify: in-block keys, packed by query row
  const uint16_t* vblk;
  uint16_t* out;
  const int32_t* page_table;
  const int32_t* work;
  const int32_t* row_idx;
  const int64_t* key_slots;  // verify
  const int32_t* vblocks;    // verify
  const uint8_t* mask;       // verify
  float* imp_part;
  int64_t n_slots;
  int64_t n_q_rows;
  int64_t n_keys;
  int64_t n_row_idx;
  int n_seq;
  int max_pages;
  int page_log2;
  int d_model;
  int block_rows;
  int imp_mode;
  float scale_log2;  // softmax_scale * log2(e)
};

struct TileState {
  float m;      // running max of this lane's row (log2 domain)
  float l;      // this lane's partial row sum
  f32x4 o[8];   // O^T blocks: lane holds O[row l%16][16*db + 4*(l/16) + i]
};

__device__ __forceinline__ float wave_max16x4(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float wave_sum16x4(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Loads K (and V^T unless kOnlyK) of keys n0 .. n0+63 into LDS. slot_of(n) gives the
// cache row of key n (valid for n < n_end); keys at or past n_end load as zeros.
template <bool kOnlyK, typename SlotOf>
__device__ __forceinline__ void load_kv_tile(u32x4* Ks, uint32_t* Vt, const uint16_t* kbase,
                                             const uint16_t* vbase, int64_t D, int col0, int n0,
                                             int n_end, SlotOf slot_of) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tid + kThreads * i;
    const int kk = id >> 4, c = id & 15;
    const int n = n0 + kk;
    u32x4 val = {0, 0, 0, 0};
    if (n < n_end) val = ld16(kbase + slot_of(n) * D + col0 + 8 * c);
    Ks[kk * 16 + (c ^ (kk & 15))] = val;
  }
  if constexpr (!kOnlyK) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tid + kThreads * i;
      const int pr = id >> 4, c = id & 15;
      const int na = n0 + 2 * pr, nb = na + 1;
      u32x4 va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
      if (na < n_end) va = ld16(vbase + slot_of(na) * D + col0 + 8 * c);
      if (nb < n_end) vb = ld16(vbase + slot_of(nb) * D + col0 + 8 * c);
      // element j of the chunk is dimension 8c + j; V^T[dim][2pr], V^T[dim][2pr+1]
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a2 = va[j], b2 = vb[j];
        Vt[(8 * c + 2 * j) * (kVtStride / 2) + pr] = (a2 & 0xffffu) | (b2 << 16);
        Vt[(8 * c + 2 * j + 1) * (kVtStride / 2) + pr] = (a2 >> 16) | (b2 & 0xffff0000u);
      }
    }
  }
}

// One 64-key tile of the online softmax + PV for this lane's row. valid(i, kb) says whether
// key 16*kb + 4*(l/16) + i of the tile may be attended by this lane's row.
template <typename Valid>
__device__ __forceinline__ void attend_tile(TileState& st, const bf16x8 (&qf)[4],
                                            const u32x4* Ks, const uint32_t* Vt, float scale_log2,
                                            Valid valid) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
  f32x4 s[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = as_bf16x8(Ks[(16 * kb + l16) * 16 + ((4 * sd + g) ^ l16)]);
      acc = mfma16(kf, qf[sd], acc);
    }
    s[kb] = acc;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = valid(i, kb) ? s[kb][i] * scale_log2 : -INFINITY;
      s[kb][i] = v;
      tmax = fmaxf(tmax, v);
    }
  tmax = wave_max16x4(tmax);
  const float m_new = fmaxf(st.m, tmax);
  const float m_use = m_new == -INFINITY ? 0.f : m_new;  // row with nothing to attend yet
  const float alpha = exp2f(st.m - m_use);
  st.m = m_new;
  float psum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = exp2f(s[kb][i] - m_use);
      s[kb][i] = p;
      psum += p;
    }
  st.l = st.l * alpha + psum;
#pragma unroll
  for (int db = 0; db < 8; ++db) st.o[db] *= alpha;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    // k-slot (g, j) of this step is key 32ks + 4g + j (j < 4) or 32ks + 16 + 4g + (j - 4)
    bf16x8 pb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pb[j] = static_cast<__bf16>(s[2 * ks][j]);
      pb[j + 4] = static_cast<__bf16>(s[2 * ks + 1][j]);
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t* vr = Vt + (16 * db + l16) * (kVtStride / 2);
      const u32x2 lo = ld8(vr + 16 * ks + 2 * g);
      const u32x2 hi = ld8(vr + 16 * ks + 8 + 2 * g);
      st.o[db] = mfma16(as_bf16x8(lo, hi), pb, st.o[db]);
    }
  }
}

// Column sums over this wavefront's importance rows of S = Q K^T for the 64 keys in LDS.
// Returns, in every lane, the sum for key 16*kb + (l % 16) of kb = 0..3.
template <typename Term>
__device__ __forceinline__ void column_sums(float (&out)[4], const bf16x8 (&qf)[4],
                                            const u32x4* Ks, Term term) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = as_bf16x8(Ks[(16 * kb + l16) * 16 + ((4 * sd + g) ^ l16)]);
      acc = mfma16(qf[sd], kf, acc);  // S[row 4g+i][key 16kb + l16]
    }
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) cs += term(i, kb, acc[i]);
    out[kb] = wave_sum16x4(cs);
  }
}

template <bool kVerify>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnArgs a) {
  __shared__ u32x4 Ks[kTileN * 16];                  // 16 KB
  __shared__ uint32_t Vt[kHeadDim * kVtStride / 2];  // 17 KB
  __shared__ float imp_buf[4][kTileN];
  __shared__ float lse_buf[kMaxRows];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int64_t D = a.d_model;
  const int col0 = h * kHeadDim;

  int b = 0, k_begin, k_end, n_rows, n_imp = 0, row0 = 0, roff = 0;
  if constexpr (kVerify) {
    const int32_t* vb = a.vblocks + 4 * blockIdx.x;
    k_begin = vb[0];
    k_end = vb[1];
    row0 = vb[2];
    n_rows = vb[3] - vb[2];
    // Out-of-range entries (rejected by the host validator) degrade to an empty range.
    if (k_begin < 0 || k_end > a.n_keys) k_end = k_begin;
    if (row0 < 0 || int64_t(row0) + n_rows > a.n_q_rows) n_rows = 0;
    if (n_rows > a.block_rows) n_rows = a.block_rows;  // mask rows hold block_rows columns
  } else {
    const int32_t* it = a.work + 8 * blockIdx.x;
    b = it[0];
    k_begin = it[1];
    k_end = it[2];
    roff = it[3];
    n_rows = it[4];
    n_imp = a.imp_mode ? it[5] : 0;
    if (b < 0 || b >= a.n_seq || k_begin < 0 ||
        int64_t(k_end) > (int64_t(a.max_pages) << a.page_log2)) {
      b = 0;
      k_end = k_begin;
    }
    if (roff < 0 || int64_t(roff) + (n_rows > 0 ? n_rows : 0) > a.n_row_idx) n_rows = 0;
  }
  n_rows = n_rows < kMaxRows ? n_rows : kMaxRows;
  if (n_rows < 0) n_rows = 0;
  if (n_imp > n_rows) n_imp = n_rows;

  // This lane's query row (B operand of S^T, A operand of S).
  const int rr = wave * 16 + l16;
  const bool row_ok = rr < n_rows;
  int64_t qrow = 0;
  if (row_ok) {
    qrow = kVerify ? int64_t(row0) + rr : int64_t(a.row_idx[roff + rr]);
    if (qrow < 0 || qrow >= a.n_q_rows) qrow = -1;
  }
  bf16x8 qf[4];
#pragma unroll
  for (int sd = 0; sd < 4; ++sd) {
    u32x4 v = {0, 0, 0, 0};
    if (row_ok && qrow >= 0) v = ld16(a.q + qrow * D + col0 + 32 * sd + 8 * g);
    qf[sd] = as_bf16x8(v);
  }

  const int pl = a.page_log2;
  const int pmask = (1 << pl) - 1;
  const int32_t* ptab = a.page_table + int64_t(b) * a.max_pages;
  const int64_t n_slots = a.n_slots;
  auto slot_of = [&](int n) -> int64_t {
    int64_t s;
    if constexpr (kVerify) {
      s = a.key_slots[n];
    } else {
      s = (int64_t(ptab[n >> pl]) << pl) | (n & pmask);
    }
    return (s >= 0 && s < n_slots) ? s : 0;  // the host validators reject such tables
  };

  TileState st;
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int db = 0; db < 8; ++db) st.o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool imp_raw = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_RAW_LOGIT;
  const bool imp_soft = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_SOFTMAX_COLSUM;
  const int imp_waves = (n_imp + 15) >> 4;
  float* imp_out = a.imp_part ? a.imp_part + int64_t(h) * n_slots : nullptr;

  // Writes the importance sums of the previous tile (imp_buf) to imp_part. Call between a
  // barrier that follows the imp_buf writes and the next imp_buf write.
  auto flush_imp = [&](int n0) {
    if (tid < kTileN) {
      const int n = n0 + tid;
      if (n < k_end) {
        float sum = 0.f;
        for (int w = 0; w < imp_waves; ++w) sum += imp_buf[w][tid];
        imp_out[slot_of(n)] = sum;
      }
    }
  };

  int prev_n0 = -1;
  for (int n0 = k_begin; n0 < k_end; n0 += kTileN) {
    __syncthreads();  // LDS tile (and imp_buf) of the previous iteration is consumed
    if (imp_raw && prev_n0 >= 0) flush_imp(prev_n0);
    load_kv_tile<false>(Ks, Vt, a.k, a.v, D, col0, n0, k_end, slot_of);
    __syncthreads();
    const int n_left = k_end - n0;
    attend_tile(st, qf, Ks, Vt, a.scale_log2, [&](int i, int kb) {
      return 16 * kb + 4 * g + i < n_left;
    });
    if (imp_raw && wave < imp_waves) {
      float cs[4];
      column_sums(cs, qf, Ks, [&](int i, int kb, float s) {
        return (wave * 16 + 4 * g + i) < n_imp ? s : 0.f;
      });
      if (g == 0) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) imp_buf[wave][16 * kb + l16] = cs[kb];
      }
    }
    prev_n0 = n0;
  }
  if (imp_raw && prev_n0 >= 0) {
    __syncthreads();
    flush_imp(prev_n0);
  }

  if constexpr (kVerify) {
    // In-block keys: the block's own rows, K/V from the packed verify projections.
    const int br = a.block_rows;
    const uint8_t* mrow = a.mask + (int64_t(blockIdx.x) * br + (rr < br ? rr : 0)) * br;
    __syncthreads();
    load_kv_tile<false>(Ks, Vt, a.kblk, a.vblk, D, col0, 0, n_rows,
                        [&](int n) -> int64_t { return int64_t(row0) + n; });  // rows checked above
    __syncthreads();
    attend_tile(st, qf, Ks, Vt, a.scale_log2, [&](int i, int kb) {
      const int j = 16 * kb + 4 * g + i;
      return j < n_rows && rr < br && mrow[j] != 0;
    });
  }

  const float l_tot = wave_sum16x4(st.l);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok && qrow >= 0) {
    uint16_t* orow = a.out + qrow * D + col0;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const f32x4 o = st.o[db];
      u32x2 pk = {pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
      st8(orow + 16 * db + 4 * g, pk);
    }
  }

  if (imp_soft) {
    // Second pass over K for the importance rows: sum_r exp2(scale_log2 * s - lse2_r).
    if (g == 0) lse_buf[rr] = (l_tot > 0.f) ? st.m + log2f(l_tot) : INFINITY;
    __syncthreads();
    float lse_r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lse_r[i] = lse_buf[wave * 16 + 4 * g + i];
    prev_n0 = -1;
    for (int n0 = k_begin; n0 < k_end; n0 += kTileN) {
      __syncthreads();
      if (prev_n0 >= 0) flush_imp(prev_n0);
      load_kv_tile<true>(Ks, Vt, a.k, a.v, D, col0, n0, k_end, slot_of);
      __syncthreads();
      if (wave < imp_waves) {
        float cs[4];
        column_sums(cs, qf, Ks, [&](int i, int kb, float s) {
          return (wave * 16 + 4 * g + i) < n_imp ? exp2f(s * a.scale_log2 - lse_r[i]) : 0.f;
        });
        if (g == 0) {
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) imp_buf[wave][16 * kb + l16] = cs[kb];
        }
      }
      prev_n0 = n0;
    }
    if (prev_n0 >= 0) {
      __syncthreads();
      flush_imp(prev_n0);
    }
  }
}

// scores[slot] += scale * sum_h imp_part[h][slot] over the keys of each importance tile.
__global__ __launch_bounds__(256) void imp_accumulate_kernel(
    const float* __restrict__ part, int n_heads, int64_t n_slots,
    const int32_t* __restrict__ page_table, int n_seq, int max_pages, int page_log2,
    const int32_t* __restrict__ work, float scale, float* __restrict__ scores) {
  const int32_t* it = work + 8 * blockIdx.x;
  if (it[5] <= 0) return;
  const int b = it[0], k_begin = it[1], k_end = it[2];
  if (b < 0 || b >= n_seq || k_begin < 0 || int64_t(k_end) > (int64_t(max_pages) << page_log2))
    return;  // rejected by the host validator
  const int32_t* ptab = page_table + int64_t(b) * max_pages;
  const int pmask = (1 << page_log2) - 1;
  for (int n = k_begin + threadIdx.x; n < k_end; n += blockDim.x) {
    const int64_t s = (int64_t(ptab[n >> page_log2]) << page_log2) | (n & pmask);
    if (s < 0 || s >= n_slots) continue;
    float sum = 0.f;
    for (int hh = 0; hh < n_heads; ++hh) sum += part[int64_t(hh) * n_slots + s];
    scores[s] += scale * sum;
  }
}

int check_common(const char* fn, const void* q, const void* k_cache, const void* v_cache,
                 const void* out, int64_t d_model, int64_t n_heads, int64_t head_dim) {
  FDL_REQUIRE(head_dim == kHeadDim, FDL_ERR_UNSUPPORTED,
              "%s: head_dim = %lld (only 128 is implemented)", fn, (long long)head_dim);
  FDL_REQUIRE(n_heads >= 1 && n_heads <= 65535 && d_model == n_heads * head_dim, FDL_ERR_SHAPE,
              "%s: d_model (%lld) != n_heads (%lld) * head_dim", fn, (long long)d_model,
              (long long)n_heads);
  FDL_REQUIRE(q && k_cache && v_cache && out, FDL_ERR_NULL, "%s: q/k_cache/v_cache/out is NULL",
              fn);
  FDL_REQUIRE((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
               reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out)) %
                      16 ==
                  0,
              FDL_ERR_SHAPE, "%s: q/k_cache/v_cache/out must be 16-byte aligned", fn);
  return FDL_OK;
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_block_attention(const void* q, const void* k_cache, const void* v_cache,
                                   int64_t n_q_rows, int64_t n_slots, int64_t d_model,
                                   int64_t n_heads, int64_t head_dim,
                                   const int32_t* page_table, int64_t n_seq, int64_t max_pages,
                                   int32_t page_log2, const int32_t* work, int64_t n_work,
                                   const int32_t* row_idx, int64_t n_row_idx,
                                   float softmax_scale, void* out, int32_t imp_mode,
                                   float* imp_part, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_block_attention: n_work = %lld out of range", (long long)n_work);
  if (n_work == 0) return ok();
  int rc = check_common("fdl_block_attention", q, k_cache, v_cache, out, d_model, n_heads,
                        head_dim);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE_PTR(page_table);
  FDL_REQUIRE_PTR(work);
  FDL_REQUIRE_PTR(row_idx);
  FDL_REQUIRE(n_seq >= 1 && max_pages >= 1 && n_slots >= 1 && n_q_rows >= 1 && n_row_idx >= 1,
              FDL_ERR_SHAPE, "fdl_block_attention: empty table or cache");
  FDL_REQUIRE(page_log2 >= 4 && page_log2 <= 12, FDL_ERR_SHAPE,
              "fdl_block_attention: page_log2 = %d outside [4, 12]", page_log2);
  FDL_REQUIRE(max_pages << page_log2 < (int64_t(1) << 31) && n_seq < (int64_t(1) << 31),
              FDL_ERR_SHAPE, "fdl_block_attention: max_pages or n_seq too large");
  FDL_REQUIRE(imp_mode >= FDL_IMP_NONE && imp_mode <= FDL_IMP_SOFTMAX_COLSUM, FDL_ERR_SHAPE,
              "fdl_block_attention: imp_mode = %d unknown", imp_mode);
  FDL_REQUIRE(imp_mode == FDL_IMP_NONE || imp_part != nullptr, FDL_ERR_NULL,
              "fdl_block_attention: imp_part is NULL with imp_mode = %d", imp_mode);
  AttnArgs args = {};
  args.q = static_cast<const uint16_t*>(q);
  args.k = static_cast<const uint16_t*>(k_cache);
  args.v = static_cast<const uint16_t*>(v_cache);
  args.out = static_cast<uint16_t*>(out);
  args.page_table = page_table;
  args.work = work;
  args.row_idx = row_idx;
  args.n_row_idx = n_row_idx;
  args.n_seq = static_cast<int>(n_seq);
  args.imp_part = imp_part;
  args.n_slots = n_slots;
  args.n_q_rows = n_q_rows;
  args.max_pages = static_cast<int>(max_pages);
  args.page_log2 = page_log2;
  args.d_model = static_cast<int>(d_model);
  args.imp_mode = imp_mode;
  args.scale_log2 = softmax_scale * kLog2e;
  hipLaunchKernelGGL(attn_kernel<false>, dim3(static_cast<unsigned>(n_work),
                                              static_cast<unsigned>(n_heads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), args);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_importance_accumulate(const float* imp_part, int64_t n_heads, int64_t n_slots,
                                         const int32_t* page_table, int64_t n_seq,
                                         int64_t max_pages, int32_t page_log2,
                                         const int32_t* work, int64_t n_work, float scale,
                                         float* scores, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_importance_accumulate: n_work = %lld out of range", (long long)n_work);
  if (n_work == 0) return ok();
  FDL_REQUIRE_PTR(imp_part);
  FDL_REQUIRE_PTR(page_table);
  FDL_REQUIRE_PTR(work);
  FDL_REQUIRE_PTR(scores);
  FDL_REQUIRE(n_heads >= 1 && n_slots >= 1 && n_seq >= 1 && max_pages >= 1, FDL_ERR_SHAPE,
              "fdl_importance_accumulate: empty dimension");
  FDL_REQUIRE(page_log2 >= 4 && page_log2 <= 12, FDL_ERR_SHAPE,
              "fdl_importance_accumulate: page_log2 = %d outside [4, 12]", page_log2);
  hipLaunchKernelGGL(imp_accumulate_kernel, dim3(static_cast<unsigned>(n_work)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), imp_part, static_cast<int>(n_heads),
                     n_slots, page_table, static_cast<int>(n_seq), static_cast<int>(max_pages),
                     page_log2, work, scale, scores);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}

extern "C" int fdl_verify_attention(const void* q, const void* k_blk, const void* v_blk,
                                    const void* k_cache, const void* v_cache, int64_t n_q_rows,
                                    int64_t n_slots, int64_t d_model, int64_t n_heads,
                                    int64_t head_dim, const int64_t* key_slots, int64_t n_keys,
                                    const int32_t* vblocks, int64_t n_vblocks,
                                    const uint8_t* mask, int32_t block_rows,
                                    float softmax_scale, void* out, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_vblocks >= 0 && n_vblocks < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_verify_attention: n_vblocks = %lld out of range", (long long)n_vblocks);
  if (n_vblocks == 0) return ok();
  int rc = check_common("fdl_verify_attention", q, k_cache, v_cache, out, d_model, n_heads,
                        head_dim);
  if (rc != FDL_OK) return rc;
  FDL_REQUIRE_PTR(k_blk);
  FDL_REQUIRE_PTR(v_blk);
  FDL_REQUIRE_PTR(vblocks);
  FDL_REQUIRE_PTR(mask);
  FDL_REQUIRE((reinterpret_cast<uintptr_t>(k_blk) | reinterpret_cast<uintptr_t>(v_blk)) % 16 == 0,
              FDL_ERR_SHAPE, "fdl_verify_attention: k_blk/v_blk must be 16-byte aligned");
  FDL_REQUIRE(block_rows >= 1 && block_rows <= kMaxRows, FDL_ERR_UNSUPPORTED,
              "fdl_verify_attention: block_rows = %d outside [1, 64]", block_rows);
  FDL_REQUIRE(n_keys >= 0 && n_keys < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_verify_attention: n_keys out of range");
  FDL_REQUIRE(n_keys == 0 || key_slots != nullptr, FDL_ERR_NULL,
              "fdl_verify_attention: key_slots is NULL");
  FDL_REQUIRE(n_slots >= 1 && n_q_rows >= 1, FDL_ERR_SHAPE, "fdl_verify_attention: empty cache");
  AttnArgs args = {};
  args.q = static_cast<const uint16_t*>(q);
  args.k = static_cast<const uint16_t*>(k_cache);
  args.v = static_cast<const uint16_t*>(v_cache);
  args.kblk = static_cast<const uint16_t*>(k_blk);
  args.vblk = static_cast<const uint16_t*>(v_blk);
  args.out = static_cast<uint16_t*>(out);
  args.key_slots = key_slots;
  args.vblocks = vblocks;
  args.mask = mask;
  args.block_rows = block_rows;
  args.n_slots = n_slots;
  args.n_q_rows = n_q_rows;
  args.n_keys = n_keys;
  args.d_model = static_cast<int>(d_model);
  args.scale_log2 = softmax_scale * kLog2e;
  hipLaunchKernelGGL(attn_kernel<true>, dim3(static_cast<unsigned>(n_vblocks),
                                             static_cast<unsigned>(n_heads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), args);
  FDL_HIP_CHECK(hipGetLastError());
  return ok();
}
