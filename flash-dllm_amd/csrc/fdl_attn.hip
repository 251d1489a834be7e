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
// Workgroup = one tile (up to 64*RB query rows of one sequence) x one head, split into NG
// key groups of 4 wavefronts. Group g streams its share of the tile's 64-key blocks
// through its own LDS buffers (K row-major with XOR-swizzled 16-byte chunks, V transposed
// with padded rows); the next block's global loads are issued into registers before the
// current block is computed, so HBM latency overlaps the MFMA work. With NG = 2 a tile
// has two key streams in flight; the groups' partial (max, sum, O) are merged through
// LDS at the end (exact: rescaled by exp of the max difference).
//
// Each wavefront owns RB blocks of 16 query rows and computes S^T = K Q^T with 16x16x32
// MFMAs, so lane l holds the logits of row l % 16 for keys 4*(l/16) + i of each 16-key
// block: the online-softmax max and sum need two cross-lane steps (xor 16, xor 32), and
// the bf16 probabilities are already the B operand of O^T = V^T P^T. The K and V^T
// fragments read from LDS are shared by the RB row blocks. Importance needs column sums
// over rows instead, so it uses S = Q K^T (the same registers, operands swapped): 4
// in-lane adds plus the same two cross-lane steps.
#include "fdl_device.h"
#include "fdl_host.h"

namespace fdl {
namespace {

constexpr int kHeadDim = 128;
constexpr int kTileN = 64;        // keys per LDS block
constexpr int kGroupThreads = 256;
constexpr int kVtStride = 68;     // bf16 per V^T row in LDS (136 B: conflict-free column reads)
constexpr int kSlotCache = 2048;  // keys per workgroup whose cache slots are staged in LDS

// 2^x on the hardware exponential (v_exp_f32). The softmax arguments are <= 0, so results
// that would be denormal flush to zero, which is harmless here.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
  int tile_rows;
  int imp_mode;
  float scale_log2;  // softmax_scale * log2(e)
};

struct GroupLds {
  u32x4 K[kTileN * 16];                   // 16 KB
  uint32_t Vt[kHeadDim * kVtStride / 2];  // 17 KB
};

struct TileRegs {
  u32x4 k[4];
  u32x4 v[2][2];
};

template <int RB>
struct RowState {
  float m[RB];      // running max of the lane's rows (log2 domain)
  float l[RB];      // partial row sums
  f32x4 o[RB][8];   // O^T blocks: lane holds O[row][16*db + 4*(l/16) + i]
};

__device__ __forceinline__ float xmax(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float xsum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// Per-thread sources of a 64-key block: K chunk (id & 15) of keys n0 + (id >> 4) for
// id = tg + 256 i, and V chunk c of the key pair n0 + 2p, n0 + 2p + 1.
struct TileSrc {
  const uint16_t* kcol;  // kbase + col0 + 8 * (chunk of this thread's K loads)
  const uint16_t* vcol;  // vbase + col0 + 8 * (chunk of this thread's V loads)
  int kkey;              // key offset (within the block) of the first K chunk
  int vkey;              // key offset of the first V pair
};

__device__ __forceinline__ TileSrc tile_src(int tg, const uint16_t* kbase, const uint16_t* vbase,
                                            int col0) {
  TileSrc t;
  t.kcol = kbase + col0 + 8 * (tg & 15);
  t.vcol = vbase + col0 + 8 * (tg & 15);
  t.kkey = tg >> 4;
  t.vkey = 2 * (tg >> 4);
  return t;
}

// Global loads of keys n0 .. n0+63 (K, and V unless kOnlyK) into registers. Keys at or
// past n_end re-read key n_end - 1 (they are masked out of the softmax and their V is
// multiplied by 0), so every load is unconditional: no branches in the loop and exact
// memory wait counts. n_end > n0 is required.
template <bool kOnlyK, typename SlotOf>
__device__ __forceinline__ void tile_issue(TileRegs& r, const TileSrc& src, int64_t D, int n0,
                                           int n_end, SlotOf slot_of) {
  const int last = n_end - 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = min(n0 + src.kkey + 16 * i, last);
    r.k[i] = ld16(src.kcol + slot_of(n) * D);
  }
  if constexpr (!kOnlyK) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int na = min(n0 + src.vkey + 32 * i, last);
      const int nb = min(n0 + src.vkey + 32 * i + 1, last);
      r.v[i][0] = ld16(src.vcol + slot_of(na) * D);
      r.v[i][1] = ld16(src.vcol + slot_of(nb) * D);
    }
  }
}

// Registers -> LDS: K chunk c of key kk at chunk c ^ (kk & 15); V transposed, two keys per
// 32-bit word (V^T[dim][2p], V^T[dim][2p+1]).
template <bool kOnlyK>
__device__ __forceinline__ void tile_commit(const TileRegs& r, GroupLds& s, int tg) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tg + kGroupThreads * i;
    const int kk = id >> 4, c = id & 15;
    s.K[kk * 16 + (c ^ (kk & 15))] = r.k[i];
  }
  if constexpr (!kOnlyK) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int id = tg + kGroupThreads * i;
      const int pr = id >> 4, c = id & 15;
      uint32_t* dst = s.Vt + (8 * c) * (kVtStride / 2) + pr;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t a2 = r.v[i][0][j], b2 = r.v[i][1][j];
        // low halves (dimension 8c + 2j) and high halves (8c + 2j + 1) of the two keys
        dst[(2 * j) * (kVtStride / 2)] = __builtin_amdgcn_perm(b2, a2, 0x05040100u);
        dst[(2 * j + 1) * (kVtStride / 2)] = __builtin_amdgcn_perm(b2, a2, 0x07060302u);
      }
    }
  }
}

// One 64-key block of online softmax + PV for the wave's RB row blocks. valid(rb, i, kb):
// may row block rb's lane row attend key 16*kb + 4*(l/16) + i of the block?
template <int RB, bool kMasked, typename Valid>
__device__ __forceinline__ void attend_block(RowState<RB>& st, const bf16x8 (&qf)[RB][4],
                                             const GroupLds& s, float scale_log2, Valid valid) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
  f32x4 sc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = as_bf16x8(s.K[(16 * kb + l16) * 16 + ((4 * sd + g) ^ l16)]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) sc[rb][kb] = mfma16(kf, qf[rb][sd], sc[rb][kb]);
    }
  bf16x8 pb[RB][2];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = sc[rb][kb][i] * scale_log2;
        if constexpr (kMasked) v = valid(rb, i, kb) ? v : -INFINITY;
        sc[rb][kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = xmax(tmax);
    const float m_new = fmaxf(st.m[rb], tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // nothing attended yet
    const float alpha = fast_exp2(st.m[rb] - m_use);
    st.m[rb] = m_new;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(sc[rb][kb][i] - m_use);
        sc[rb][kb][i] = p;
        psum += p;
      }
    st.l[rb] = st.l[rb] * alpha + psum;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[rb][db] *= alpha;
    // k-slot (g, j) of PV step ks is key 32ks + 4g + j (j < 4) or 32ks + 16 + 4g + (j - 4)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[rb][ks][j] = static_cast<__bf16>(sc[rb][2 * ks][j]);
        pb[rb][ks][j + 4] = static_cast<__bf16>(sc[rb][2 * ks + 1][j]);
      }
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t* vr = s.Vt + (16 * db + l16) * (kVtStride / 2);
      const bf16x8 vf = as_bf16x8(ld8(vr + 16 * ks + 2 * g), ld8(vr + 16 * ks + 8 + 2 * g));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) st.o[rb][db] = mfma16(vf, pb[rb][ks], st.o[rb][db]);
    }
}

// Column sums over the wave's importance rows of S = Q K^T for the 64 keys in LDS:
// out[kb] (in every lane) = sum over rows of term(rb, i, kb, s) for key 16*kb + (l % 16).
template <int RB, typename Term>
__device__ __forceinline__ void column_sums(float (&out)[4], const bf16x8 (&qf)[RB][4],
                                            const GroupLds& s, Term term) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      const bf16x8 kf = as_bf16x8(s.K[(16 * kb + l16) * 16 + ((4 * sd + g) ^ l16)]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma16(qf[rb][sd], kf, acc[rb]);  // S[4g+i][key]
    }
    float cs = 0.f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) cs += term(rb, i, kb, acc[rb][i]);
    out[kb] = xsum(cs);
  }
}

// One key group of short-row tiles runs two workgroups per CU (registers capped at 256).
template <int RB, int NG, bool kVerify>
__global__ __launch_bounds__(kGroupThreads * NG, (RB == 1 && NG == 1) ? 2 : 1) void attn_kernel(
    AttnArgs a) {
  constexpr int kRows = 64 * RB;
  __shared__ __align__(16) uint8_t smem[NG * sizeof(GroupLds)];
  __shared__ float imp_buf[NG][4][kTileN];
  __shared__ float lse_buf[kRows];
  __shared__ int32_t slot_buf[kSlotCache];  // cache slot of key k_begin + i
  static_assert(sizeof(float) * kRows * (kHeadDim + 2) <= NG * sizeof(GroupLds) || NG == 1,
                "combine area must fit in the key-group buffers");

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int grp = wave >> 2, wr = wave & 3, tg = tid & (kGroupThreads - 1);
  const int l16 = lane & 15, g = lane >> 4;
  GroupLds& lds = reinterpret_cast<GroupLds*>(smem)[grp];
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
    // out-of-range entries (rejected by the host validator) degrade to an empty range
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
  if (n_rows > kRows) n_rows = kRows;
  if (n_rows < 0) n_rows = 0;
  if (n_imp > n_rows) n_imp = n_rows;
  if (k_end < k_begin) k_end = k_begin;

  // The lane's query rows: row block id = wr * RB + rb covers rows 16 * id .. 16 * id + 15.
  int64_t qrow[RB];
  bf16x8 qf[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = 16 * (wr * RB + rb) + l16;
    qrow[rb] = -1;
    if (r < n_rows) {
      const int64_t q = kVerify ? int64_t(row0) + r : int64_t(a.row_idx[roff + r]);
      if (q >= 0 && q < a.n_q_rows) qrow[rb] = q;
    }
#pragma unroll
    for (int sd = 0; sd < 4; ++sd) {
      u32x4 v = {0, 0, 0, 0};
      if (qrow[rb] >= 0) v = ld16(a.q + qrow[rb] * D + col0 + 32 * sd + 8 * g);
      qf[rb][sd] = as_bf16x8(v);
    }
  }

  const int pl = a.page_log2;
  const int pmask = (1 << pl) - 1;
  const int32_t* ptab = a.page_table + int64_t(b) * a.max_pages;
  const int64_t n_slots = a.n_slots;
  auto lookup = [&](int n) -> int64_t {
    int64_t s;
    if constexpr (kVerify) {
      s = a.key_slots[n];
    } else {
      s = (int64_t(ptab[n >> pl]) << pl) | (n & pmask);
    }
    return (s >= 0 && s < n_slots) ? s : 0;  // the host validators reject such tables
  };
  // The key -> slot map of the tile's key range is staged in LDS once, so the K/V loads
  // of a block do not wait on a page-table (or key-list) load first.
  const bool slots_staged = k_end - k_begin <= kSlotCache && n_slots < (int64_t(1) << 31);
  if (slots_staged) {
    for (int i = tid; i < k_end - k_begin; i += kGroupThreads * NG)
      slot_buf[i] = static_cast<int32_t>(lookup(k_begin + i));
  }
  __syncthreads();
  auto slot_of = [&](int n) -> int64_t {
    return slots_staged ? int64_t(slot_buf[n - k_begin]) : lookup(n);
  };

  RowState<RB> st;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    st.m[rb] = -INFINITY;
    st.l[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) st.o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const bool imp_raw = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_RAW_LOGIT;
  const bool imp_soft = !kVerify && n_imp > 0 && a.imp_mode == FDL_IMP_SOFTMAX_COLSUM;
  const bool wave_imp = 16 * RB * wr < n_imp;
  const int imp_waves = (n_imp + 16 * RB - 1) / (16 * RB);
  float* imp_out = a.imp_part ? a.imp_part + int64_t(h) * n_slots : nullptr;

  // Block scheduling: the tile's 64-key blocks are split into NG contiguous runs of
  // per_grp blocks; every group makes per_grp passes so barriers stay uniform.
  const int n_blk = (k_end - k_begin + kTileN - 1) / kTileN;
  const int per_grp = (n_blk + NG - 1) / NG;
  const int blk0 = grp * per_grp;
  const int blk_end = min(n_blk, blk0 + per_grp);

  // Writes one group's importance sums of a finished block to imp_part. Called between a
  // barrier that follows the imp_buf writes and the group's next imp_buf write.
  auto flush_imp = [&](int n0) {
    if (tg < kTileN) {
      const int n = n0 + tg;
      if (n < k_end) {
        float sum = 0.f;
        for (int w = 0; w < imp_waves; ++w) sum += imp_buf[grp][w][tg];
        imp_out[slot_of(n)] = sum;
      }
    }
  };

  // Two blocks per key group are in flight in a two-slot register ring: block blk is
  // loaded into regs[blk & 1], two blocks ahead of its use. The prefetch index is clamped
  // to the tile's last block so every load is unconditional (exact wait counts); the
  // clamped extra loads are never committed.
  TileRegs regs[2];
  const TileSrc csrc = tile_src(tg, a.k, a.v, col0);
  const int last_blk = n_blk - 1;
  auto blk_n0 = [&](int blk) { return k_begin + kTileN * min(blk, last_blk); };
  if (n_blk > 0) {
    tile_issue<false>(regs[0], csrc, D, blk_n0(blk0), k_end, slot_of);
    tile_issue<false>(regs[1], csrc, D, blk_n0(blk0 + 1), k_end, slot_of);
    for (int i = 0; i < per_grp; i += 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int blk = blk0 + i + j;
        const bool have = i + j < per_grp && blk < blk_end;
        const int n0 = k_begin + kTileN * blk;
        __syncthreads();  // the group's LDS block and imp_buf have been consumed
        if (imp_raw && have && i + j > 0) flush_imp(n0 - kTileN);
        if (have) tile_commit<false>(regs[j], lds, tg);
        tile_issue<false>(regs[j], csrc, D, blk_n0(blk + 2), k_end, slot_of);
        __syncthreads();
        if (have) {
          const int n_left = k_end - n0;
          if (n_left >= kTileN)
            attend_block<RB, false>(st, qf, lds, a.scale_log2, [](int, int, int) { return true; });
          else
            attend_block<RB, true>(st, qf, lds, a.scale_log2, [&](int, int ii, int kb) {
              return 16 * kb + 4 * g + ii < n_left;
            });
          if (imp_raw && wave_imp) {
            float cs[4];
            column_sums<RB>(cs, qf, lds, [&](int rb, int ii, int, float sv) {
              return 16 * (wr * RB + rb) + 4 * g + ii < n_imp ? sv : 0.f;
            });
            if (g == 0) {
#pragma unroll
              for (int kb = 0; kb < 4; ++kb) imp_buf[grp][wr][16 * kb + l16] = cs[kb];
            }
          }
        }
      }
    }
  }
  if (imp_raw) {
    __syncthreads();
    if (blk_end > blk0) flush_imp(k_begin + kTileN * (blk_end - 1));
  }

  if constexpr (kVerify) {
    // In-block keys (the block's own rows from the packed verify projections) under the
    // block's mask; they belong to the last key group.
    const int br = a.block_rows;
    __syncthreads();
    if (grp == NG - 1 && n_rows > 0) {
      tile_issue<false>(regs[0], tile_src(tg, a.kblk, a.vblk, col0), D, 0, n_rows,
                        [&](int n) -> int64_t { return int64_t(row0) + n; });  // rows checked above
      tile_commit<false>(regs[0], lds, tg);
    }
    __syncthreads();
    if (grp == NG - 1 && n_rows > 0) {
      attend_block<RB, true>(st, qf, lds, a.scale_log2, [&](int rb, int ii, int kb) {
        const int r = 16 * (wr * RB + rb) + l16;
        const int j = 16 * kb + 4 * g + ii;
        return j < n_rows && r < br &&
               a.mask[(int64_t(blockIdx.x) * br + r) * br + j] != 0;
      });
    }
  }

  // Full row sums in every lane of the row.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) st.l[rb] = xsum(st.l[rb]);

  if constexpr (NG > 1) {
    // Merge the key groups: group 1 publishes (m, l, O), group 0 rescales and adds.
    float* comb = reinterpret_cast<float*>(smem);  // [kRows][kHeadDim] then m, l
    float* comb_m = comb + kRows * kHeadDim;
    float* comb_l = comb_m + kRows;
    __syncthreads();
    if (grp == 1) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * (wr * RB + rb) + l16;
        if (g == 0) {
          comb_m[r] = st.m[rb];
          comb_l[r] = st.l[rb];
        }
#pragma unroll
        for (int db = 0; db < 8; ++db)
          *reinterpret_cast<f32x4*>(comb + r * kHeadDim + 16 * db + 4 * g) = st.o[rb][db];
      }
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * (wr * RB + rb) + l16;
        const float m1 = comb_m[r], l1 = comb_l[r];
        const float m = fmaxf(st.m[rb], m1);
        const float mu = m == -INFINITY ? 0.f : m;
        const float a0 = fast_exp2(st.m[rb] - mu), a1 = fast_exp2(m1 - mu);
        st.m[rb] = m;
        st.l[rb] = st.l[rb] * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          const f32x4 o1 = *reinterpret_cast<const f32x4*>(comb + r * kHeadDim + 16 * db + 4 * g);
          st.o[rb][db] = st.o[rb][db] * a0 + o1 * a1;
        }
      }
    }
  }

  if (grp == 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (qrow[rb] < 0) continue;
      const float inv = st.l[rb] > 0.f ? 1.f / st.l[rb] : 0.f;
      uint16_t* orow = a.out + qrow[rb] * D + col0;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const f32x4 o = st.o[rb][db];
        const u32x2 pk = {pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
        st8(orow + 16 * db + 4 * g, pk);
      }
    }
  }

  if (imp_soft) {
    // Second pass over K for the importance rows: sum_r exp2(scale_log2 * s - lse2_r).
    if (grp == 0 && g == 0) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        lse_buf[16 * (wr * RB + rb) + l16] =
            st.l[rb] > 0.f ? st.m[rb] + log2f(st.l[rb]) : INFINITY;
    }
    __syncthreads();
    float lse_r[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) lse_r[rb][ii] = lse_buf[16 * (wr * RB + rb) + 4 * g + ii];
    if (n_blk > 0) {
      tile_issue<true>(regs[0], csrc, D, blk_n0(blk0), k_end, slot_of);
      tile_issue<true>(regs[1], csrc, D, blk_n0(blk0 + 1), k_end, slot_of);
      for (int i = 0; i < per_grp; i += 2) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int blk = blk0 + i + j;
          const bool have = i + j < per_grp && blk < blk_end;
          const int n0 = k_begin + kTileN * blk;
          __syncthreads();
          if (have && i + j > 0) flush_imp(n0 - kTileN);
          if (have) tile_commit<true>(regs[j], lds, tg);
          tile_issue<true>(regs[j], csrc, D, blk_n0(blk + 2), k_end, slot_of);
          __syncthreads();
          if (have && wave_imp) {
            float cs[4];
            column_sums<RB>(cs, qf, lds, [&](int rb, int ii, int, float sv) {
              return 16 * (wr * RB + rb) + 4 * g + ii < n_imp
                         ? fast_exp2(sv * a.scale_log2 - lse_r[rb][ii])
                         : 0.f;
            });
            if (g == 0) {
#pragma unroll
              for (int kb = 0; kb < 4; ++kb) imp_buf[grp][wr][16 * kb + l16] = cs[kb];
            }
          }
        }
      }
    }
    __syncthreads();
    if (blk_end > blk0) flush_imp(k_begin + kTileN * (blk_end - 1));
  }
}

// scores[slot] += scale * sum_h imp_part[h][slot] over the keys of each importance tile;
// blockIdx.y = work item, blockIdx.x strides over its keys.
__global__ __launch_bounds__(256) void imp_accumulate_kernel(
    const float* __restrict__ part, int n_heads, int64_t n_slots,
    const int32_t* __restrict__ page_table, int n_seq, int max_pages, int page_log2,
    const int32_t* __restrict__ work, float scale, float* __restrict__ scores) {
  const int32_t* it = work + 8 * blockIdx.y;
  if (it[5] <= 0) return;
  const int b = it[0], k_begin = it[1], k_end = it[2];
  if (b < 0 || b >= n_seq || k_begin < 0 || int64_t(k_end) > (int64_t(max_pages) << page_log2))
    return;  // rejected by the host validator
  const int32_t* ptab = page_table + int64_t(b) * max_pages;
  const int pmask = (1 << page_log2) - 1;
  for (int n = k_begin + blockIdx.x * blockDim.x + threadIdx.x; n < k_end;
       n += gridDim.x * blockDim.x) {
    const int64_t s = (int64_t(ptab[n >> page_log2]) << page_log2) | (n & pmask);
    if (s < 0 || s >= n_slots) continue;
    // independent loads, summed in ascending head order
    float v[8];
    float sum = 0.f;
    int hh = 0;
    for (; hh + 8 <= n_heads; hh += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[int64_t(hh + u) * n_slots + s];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += v[u];
    }
    for (; hh < n_heads; ++hh) sum += part[int64_t(hh) * n_slots + s];
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

// Two key groups per workgroup while the grid alone would leave CUs idle.
constexpr int64_t kSplitBelow = 768;

template <int RB, int NG, bool kVerify>
hipError_t launch_attn(const AttnArgs& args, int64_t n_tiles, int64_t n_heads, hipStream_t s) {
  hipLaunchKernelGGL((attn_kernel<RB, NG, kVerify>),
                     dim3(static_cast<unsigned>(n_tiles), static_cast<unsigned>(n_heads)),
                     dim3(kGroupThreads * NG), 0, s, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace fdl

extern "C" int fdl_block_attention(const void* q, const void* k_cache, const void* v_cache,
                                   int64_t n_q_rows, int64_t n_slots, int64_t d_model,
                                   int64_t n_heads, int64_t head_dim,
                                   const int32_t* page_table, int64_t n_seq, int64_t max_pages,
                                   int32_t page_log2, const int32_t* work, int64_t n_work,
                                   const int32_t* row_idx, int64_t n_row_idx, int32_t tile_rows,
                                   float softmax_scale, void* out, int32_t imp_mode,
                                   float* imp_part, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < (int64_t(1) << 31), FDL_ERR_SHAPE,
              "fdl_block_attention: n_work = %lld out of range", (long long)n_work);
  FDL_REQUIRE(tile_rows == 64 || tile_rows == 128, FDL_ERR_UNSUPPORTED,
              "fdl_block_attention: tile_rows = %d (64 or 128)", tile_rows);
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
  args.tile_rows = tile_rows;
  args.imp_mode = imp_mode;
  args.scale_log2 = softmax_scale * kLog2e;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool split = n_work * n_heads < kSplitBelow;
  hipError_t e;
  // long-row tiles hold two row blocks per wavefront and run one key group (a second group
  // would not fit the register file)
  if (tile_rows == 64)
    e = split ? launch_attn<1, 2, false>(args, n_work, n_heads, s)
              : launch_attn<1, 1, false>(args, n_work, n_heads, s);
  else
    e = launch_attn<2, 1, false>(args, n_work, n_heads, s);
  FDL_HIP_CHECK(e);
  return ok();
}

extern "C" int fdl_importance_accumulate(const float* imp_part, int64_t n_heads, int64_t n_slots,
                                         const int32_t* page_table, int64_t n_seq,
                                         int64_t max_pages, int32_t page_log2,
                                         const int32_t* work, int64_t n_work, float scale,
                                         float* scores, void* stream) {
  using namespace fdl;
  FDL_REQUIRE(n_work >= 0 && n_work < 65536, FDL_ERR_SHAPE,
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
  hipLaunchKernelGGL(imp_accumulate_kernel, dim3(4, static_cast<unsigned>(n_work)), dim3(256), 0,
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
  FDL_REQUIRE(block_rows >= 1 && block_rows <= 64, FDL_ERR_UNSUPPORTED,
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
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = n_vblocks * n_heads < kSplitBelow
                           ? launch_attn<1, 2, true>(args, n_vblocks, n_heads, s)
                           : launch_attn<1, 1, true>(args, n_vblocks, n_heads, s);
  FDL_HIP_CHECK(e);
  return ok();
}
